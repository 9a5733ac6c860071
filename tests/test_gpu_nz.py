"""The NZ KV layout of the reference's graph mode on the GPU.

npu_scatter_pa_kv_cache and FIA-v2 view each (NB, bs, Hkv, D) cache as
(NB, Hkv*D/16, bs, 16) (auto_infer/layers/attention/gqa.py:202-226).  The
slot write into that view is checked bit for bit against the oracle's
kv_write_nz; attention over NZ caches must give the bits the standard-layout
path gives over the same values (the kernels differ only in where they load
a 16-byte piece from), and that path is itself checked against the oracle.
"""
import pytest
import torch

from auto_infer_amd import ops, workloads
from auto_infer_amd.attention.gqa import GqaHipBackend
from oracle.paged_attn import kv_write, kv_write_nz, nz_from_nd, paged_attention

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
TOL = 2e-2


@pytest.mark.parametrize("T,hkv,d,nb,bs", [(16, 8, 128, 512, 128), (37, 4, 128, 40, 16),
                                           (9, 2, 64, 30, 16), (5, 1, 64, 8, 1),
                                           (0, 8, 128, 8, 4)])
def test_write_kv_nz_bit_exact(T, hkv, d, nb, bs):
    g = torch.Generator().manual_seed(T * 7 + d + bs)
    kc = torch.randn(nb, bs, hkv, d, generator=g).bfloat16()
    vc = torch.randn(nb, bs, hkv, d, generator=g).bfloat16()
    k = torch.randn(T, hkv, d, generator=g).bfloat16()
    v = torch.randn(T, hkv, d, generator=g).bfloat16()
    slots = torch.randperm(nb * bs, generator=g)[:T].to(torch.int32)
    if T > 2:
        slots[1] = -1                 # padding rows are skipped
        slots[2] = nb * bs            # as are slots past the cache
    ek, ev = kc.clone(), vc.clone()
    kv_write_nz(k, v, ek, ev, slots)
    gk, gv = kc.to(DEV), vc.to(DEV)
    print(f"write_kv_nz T={T} hkv={hkv} d={d} nb={nb} bs={bs}", flush=True)
    ops.write_kv_nz(k.to(DEV), v.to(DEV), gk, gv, slots.to(DEV))
    torch.cuda.synchronize()
    assert torch.equal(gk.cpu().view(torch.int16), ek.view(torch.int16))
    assert torch.equal(gv.cpu().view(torch.int16), ev.view(torch.int16))


def test_write_kv_nz_strided_key_only():
    """k as a column slice of a packed projection; no value cache."""
    T, hq, hkv, d, nb, bs = 7, 8, 2, 128, 6, 16
    g = torch.Generator().manual_seed(11)
    qkv = torch.randn(T, (hq + 2 * hkv) * d, generator=g).bfloat16()
    k = qkv[:, hq * d:(hq + hkv) * d].reshape(T, hkv, d)
    kc = torch.zeros(nb, bs, hkv, d).bfloat16()
    slots = torch.tensor([0, 15, 16, 50, 95, 33, 34], dtype=torch.int32)
    exp = kc.clone()
    kv_write_nz(k, None, exp, None, slots)
    gqkv = qkv.to(DEV)
    gk = gqkv[:, hq * d:(hq + hkv) * d].view(T, hkv, d)
    gc = kc.to(DEV)
    ops.write_kv_nz(gk, None, gc, None, slots.to(DEV))
    torch.cuda.synchronize()
    assert torch.equal(gc.cpu(), exp)


# decode (config-1 heads), MTP verify, chunked prefill with many q blocks,
# head blocks (group 32), group past 16, prefill units with/without prefix,
# items cut into key chunks, a mixed launch (4 kv heads), head_dim 64.
CASES = [
    ([1] * 16, [300, 129, 2048, 17, 1, 700, 901, 64, 65, 128, 1000, 5, 6, 1500, 333, 2],
     16, 8, 128, 128, 0),
    ([2] * 4, [1024, 1500, 2, 4096], 32, 8, 128, 128, 3),
    ([37, 1, 5, 1, 64], [137, 300, 5, 77, 64], 28, 4, 128, 16, 0),
    ([2, 2, 1], [513, 40, 999], 64, 2, 128, 128, 7),
    ([1, 3], [700, 90], 40, 2, 128, 16, 0),
    ([200, 1, 130, 19], [300, 77, 130, 40], 28, 4, 128, 16, 0),
    ([256, 3], [256 + 1000, 900], 16, 8, 128, 128, 0),
    ([300], [6000], 16, 8, 128, 128, 0),
    ([300, 1, 1, 3, 200, 1], [1300, 900, 50, 400, 200, 3000], 28, 4, 128, 16, 0),
    ([150, 1, 2], [400, 333, 70], 14, 2, 64, 16, 0),
    ([1] * 5, [100, 37, 513, 1, 64], 16, 8, 64, 128, 0),
]


@pytest.mark.parametrize("fused", [False, True])
@pytest.mark.parametrize("lqs,lks,hq,hkv,d,bs,waves", CASES)
def test_attention_nz_equals_nd_bitwise(lqs, lks, hq, hkv, d, bs, waves, fused):
    step = workloads.make_gqa_step(lqs=lqs, lks=lks, num_q_heads=hq, num_kv_heads=hkv,
                                   head_dim=d, block_size=bs, seed=41, extra_blocks=2)
    plan = ops.AttentionPlan.from_lists(step.block_table.to(DEV), step.cu_seqlens_q,
                                        step.seqlens_kv, hq, hkv, d, bs, num_waves=waves)
    kw = {}
    if fused:
        kw = dict(key_new=step.k_new.to(DEV), value_new=step.v_new.to(DEV))
    print(f"nz vs nd lqs={lqs[:4]} lks={lks[:4]} hq={hq} hkv={hkv} d={d} bs={bs} "
          f"waves={waves} fused={fused}", flush=True)
    kc, vc = step.k_cache.to(DEV), step.v_cache.to(DEV)
    nd = ops.paged_attention_gqa(step.q.to(DEV), kc, vc, plan, step.scale, **kw)
    kz, vz = nz_from_nd(step.k_cache).to(DEV), nz_from_nd(step.v_cache).to(DEV)
    nz = ops.paged_attention_gqa(step.q.to(DEV), kz, vz, plan, step.scale, kv_layout="nz", **kw)
    torch.cuda.synchronize()
    assert torch.equal(nz.view(torch.int16), nd.view(torch.int16))
    assert torch.equal(kz.cpu(), nz_from_nd(kc.cpu())) and torch.equal(vz.cpu(), nz_from_nd(vc.cpu()))
    ek, ev = step.k_cache.clone(), step.v_cache.clone()
    if fused:
        kv_write(step.k_new, step.v_new, ek, ev, step.slot_mapping)
    exp = paged_attention(step.q, ek, ev, step.block_table, step.cu_seqlens_q, step.seqlens_kv,
                          step.scale)
    err = (nz.float().cpu() - exp).abs().max().item()
    print(f"max-abs err {err:.3e}", flush=True)
    assert err <= TOL


def test_attention_nz_rejects_unknown_layout():
    step = workloads.make_gqa_step(lqs=[1], lks=[5], num_q_heads=2, num_kv_heads=1,
                                   block_size=16, seed=1)
    plan = ops.AttentionPlan.from_lists(step.block_table.to(DEV), step.cu_seqlens_q,
                                        step.seqlens_kv, 2, 1, 128, 16)
    with pytest.raises(ValueError, match="kv_layout"):
        ops.paged_attention_gqa(step.q.to(DEV), step.k_cache.to(DEV), step.v_cache.to(DEV),
                                plan, step.scale, kv_layout="nhd")


def test_backend_nz_matches_nd_over_prefill_decode_and_a_foreign_slot_step():
    """Two GqaHipBackends, one per layout, same weights and steps: identical
    outputs, and the NZ caches are the NZ image of the standard ones."""
    from tests.test_gpu_backends import _gqa_weights, make_ctx, rope_tables
    hq, hkv, d, hidden, bs = 8, 2, 128, 256, 16
    w, g = _gqa_weights(5, hq, hkv, d, hidden)
    kw = dict(n_q_heads=hq, n_kv_heads=hkv, head_dim=d, scale=d ** -0.5, num_layers=1,
              device=DEV, dtype=torch.bfloat16, w=w, rms_eps=1e-6)
    nd, nz = GqaHipBackend(**kw), GqaHipBackend(kv_layout="nz", **kw)
    cd, cz = nd.alloc_kv_caches(16, bs), nz.alloc_kv_caches(16, bs)
    assert isinstance(cz[0], tuple) and cz[0][0].shape == (16, bs, hkv, d)
    steps = [([(0, 5, [3]), (0, 20, [7, 1])], True),
             ([(5, 1, [3]), (20, 1, [7, 1])], True),
             ([(6, 11, [3, 9]), (21, 1, [7, 1])], True),
             ([(17, 2, [3, 9]), (22, 1, [7, 1])], False)]     # the write is not fused
    for rows, derived in steps:
        T = sum(n for _, n, _ in rows)
        x = (torch.randn(T, hidden, generator=g) * 0.5).bfloat16().to(DEV)
        ctx_d, positions = make_ctx(nd, cd, rows, bs, derived=derived)
        ctx_z, _ = make_ctx(nz, cz, rows, bs, derived=derived)
        cos, sin = rope_tables(positions, d)
        ctx_d.cos = ctx_z.cos = cos.to(DEV)
        ctx_d.sin = ctx_z.sin = sin.to(DEV)
        out_d = nd.attention(0, x, ctx_d)
        out_z = nz.attention(0, x, ctx_z)
        torch.cuda.synchronize()
        assert torch.equal(out_z.view(torch.int16), out_d.view(torch.int16))
        assert torch.equal(cz[0][0].cpu(), nz_from_nd(cd[0][0].cpu()))
        assert torch.equal(cz[0][1].cpu(), nz_from_nd(cd[0][1].cpu()))


@pytest.mark.parametrize("name", ["configs[1]", "configs[3]"])
def test_full_size_configs_nz_equal_nd(name):
    """BASELINE configs[1] (mixed prefill chunks + 512 decode rows, one mixed
    launch) and configs[3] (MTP verify with the fused write of both tokens)
    at full size over NZ caches: outputs and written caches bit-identical to
    the standard layout (which the config tests check against the oracle)."""
    dev = torch.device(DEV)
    if name == "configs[1]":
        step, fused = workloads.config2_mixed(seed=0, device=dev), False
    else:
        step, fused = workloads.config4_mtp(seed=0, device=dev), True
    print(f"{name}: NZ against ND at full size, fused={fused}", flush=True)
    hq, hkv, d, bs = step.q.shape[1], step.k_cache.shape[2], step.q.shape[2], step.k_cache.shape[1]
    plan = ops.AttentionPlan.from_lists(step.block_table, step.cu_seqlens_q, step.seqlens_kv,
                                        hq, hkv, d, bs)
    kw = dict(key_new=step.k_new, value_new=step.v_new) if fused else {}
    kz, vz = nz_from_nd(step.k_cache), nz_from_nd(step.v_cache)
    nz = ops.paged_attention_gqa(step.q, kz, vz, plan, step.scale, kv_layout="nz", **kw)
    nd = ops.paged_attention_gqa(step.q, step.k_cache, step.v_cache, plan, step.scale, **kw)
    torch.cuda.synchronize()
    assert torch.equal(nz.view(torch.int16), nd.view(torch.int16))
    if fused:
        assert torch.equal(kz, nz_from_nd(step.k_cache)) and torch.equal(vz, nz_from_nd(step.v_cache))
    del step, kz, vz
    torch.cuda.empty_cache()
