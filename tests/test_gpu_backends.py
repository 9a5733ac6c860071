"""Backends through the reference's seam on the GPU.

Each backend runs ``attention(layer_idx, x, ctx)`` end to end; a twin
backend whose op pair (``_write_kv`` / ``_attn``) is the CPU oracle runs the
identical torch code around it.  KV caches must match bit for bit and the
attention op outputs within 2e-2 max-abs.
"""
import pytest
import torch

from auto_infer_amd.attention.base import ForwardContext
from auto_infer_amd.attention.gqa import GqaHipBackend
from auto_infer_amd.attention.mla import MlaHipBackend
from oracle.paged_attn import kv_write, mla_absorbed_attention, paged_attention

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
TOL = 2e-2


def rope_tables(positions, dim, base=10000.0):
    inv = 1.0 / (base ** (torch.arange(0, dim, 2, dtype=torch.float32) / dim))
    f = positions.float()[:, None] * inv[None]
    emb = torch.cat([f, f], dim=-1)
    return emb.cos()[:, None].bfloat16(), emb.sin()[:, None].bfloat16()


def make_ctx(backend, caches, plan_rows, block_size, derived=True):
    """plan_rows: list of (start, n, block_ids) per request.  ``derived``:
    declare the slot mapping block-table derived (as this package's packers
    do), which lets the GQA backend fuse the KV write into attention."""
    slots, pos, cu, kv, acc = [], [], [], [], 0
    width = max(len(r[2]) for r in plan_rows)
    bt = torch.zeros(len(plan_rows), width, dtype=torch.int32)
    for i, (start, n, blocks) in enumerate(plan_rows):
        bt[i, :len(blocks)] = torch.tensor(blocks)
        for p in range(start, start + n):
            slots.append(blocks[p // block_size] * block_size + p % block_size)
            pos.append(p)
        acc += n
        cu.append(acc)
        kv.append(start + n)
    positions = torch.tensor(pos)
    ctx = ForwardContext(
        token_ids=torch.zeros(acc, dtype=torch.long, device=DEV), positions=positions.to(DEV),
        slot_mapping=torch.tensor(slots, dtype=torch.int32, device=DEV), block_table=bt.to(DEV),
        cu_seqlens_q=cu, seqlens_kv=kv, attn_mask=None, attn_backend=backend,
        kv_caches=caches, is_decode=all(n == 1 for _, n, _ in plan_rows))
    if derived:
        ctx.aia_slots_from_block_table = True
    return ctx, positions


class _Capture:
    def __init__(self):
        self.outs = []


def oracle_twin(cls):
    class Twin(cls):
        captured = None

        def _write_kv(self, layer_idx, k, v, ctx):
            cache = ctx.kv_caches[layer_idx]
            if isinstance(cache, tuple):
                c = cache[0].cpu()
                kv_write(k.cpu(), None, c, None, ctx.slot_mapping.cpu())
                cache[0].copy_(c)
            else:
                kc, vc = cache[0].cpu(), cache[1].cpu()
                kv_write(k.cpu(), v.cpu(), kc, vc, ctx.slot_mapping.cpu())
                cache[0].copy_(kc)
                cache[1].copy_(vc)

        def _attn(self, layer_idx, q, k, v, ctx):
            cache = ctx.kv_caches[layer_idx]
            bt = ctx.block_table.cpu()
            if isinstance(cache, tuple):
                o = mla_absorbed_attention(q.cpu(), cache[0].cpu(), bt, ctx.cu_seqlens_q,
                                           ctx.seqlens_kv, self.softmax_scale, 512)
            else:
                o = paged_attention(q.cpu(), cache[0].cpu(), cache[1].cpu(), bt,
                                    ctx.cu_seqlens_q, ctx.seqlens_kv, self.scale)
            o = o.to(q.dtype).to(q.device)
            self.captured.append(o)
            return o
    return Twin


def run_pair(hip, twin, steps, caches_hip, caches_ref, block_size, hidden, seed):
    g = torch.Generator().manual_seed(seed)
    for rows in steps:
        T = sum(n for _, n, _ in rows)
        x = (torch.randn(T, hidden, generator=g) * 0.5).bfloat16().to(DEV)
        ctx_h, positions = make_ctx(hip, caches_hip, rows, block_size)
        ctx_r, _ = make_ctx(twin, caches_ref, rows, block_size)
        rope_dim = getattr(hip, "qk_rope", None) or hip.head_dim
        cos, sin = rope_tables(positions, rope_dim)
        ctx_h.cos = ctx_r.cos = cos.to(DEV)
        ctx_h.sin = ctx_r.sin = sin.to(DEV)
        got_attn = []
        orig = hip._attn

        def spy(*a, **k):
            o = orig(*a, **k)
            got_attn.append(o)
            return o
        hip._attn = spy
        twin.captured = []
        out_h = hip.attention(0, x, ctx_h)
        out_r = twin.attention(0, x, ctx_r)
        hip._attn = orig
        torch.cuda.synchronize()
        for a, b in zip(caches_hip[0] if not isinstance(caches_hip[0], tuple) else caches_hip[0][:1],
                        caches_ref[0] if not isinstance(caches_ref[0], tuple) else caches_ref[0][:1]):
            assert torch.equal(a.cpu(), b.cpu()), "KV cache differs from the oracle's"
        err = (got_attn[0].float() - twin.captured[0].float()).abs().max().item()
        print(f"attention op max-abs err {err:.3e}", flush=True)
        assert err <= TOL
        scale = out_r.float().abs().max().item()
        assert (out_h.float() - out_r.float()).abs().max().item() <= TOL * max(1.0, scale)


def test_gqa_backend_prefill_then_decode_qwen3_style():
    g = torch.Generator().manual_seed(0)
    hq, hkv, d, hidden, bs = 4, 2, 128, 256, 16
    p = "model.layers.0.self_attn."
    w = {
        p + "qkv_proj.weight": (torch.randn((hq + 2 * hkv) * d, hidden, generator=g) / 16).bfloat16(),
        p + "q_norm.weight": (1 + 0.1 * torch.randn(d, generator=g)).bfloat16(),
        p + "k_norm.weight": (1 + 0.1 * torch.randn(d, generator=g)).bfloat16(),
        p + "o_proj.weight": (torch.randn(hidden, hq * d, generator=g) / 23).bfloat16(),
    }
    w = {k: v.to(DEV) for k, v in w.items()}
    kw = dict(n_q_heads=hq, n_kv_heads=hkv, head_dim=d, scale=d ** -0.5, num_layers=1,
              device=DEV, dtype=torch.bfloat16, w=w, rms_eps=1e-6)
    hip = GqaHipBackend(**kw)
    twin = oracle_twin(GqaHipBackend)(**kw)
    caches_h = hip.alloc_kv_caches(12, bs)
    caches_r = twin.alloc_kv_caches(12, bs)
    steps = [
        [(0, 5, [3]), (0, 20, [7, 1])],            # prefill two prompts
        [(5, 1, [3]), (20, 1, [7, 1])],            # decode
        [(6, 11, [3, 9]), (21, 1, [7, 1])],        # chunked prefill continuation + decode
    ]
    run_pair(hip, twin, steps, caches_h, caches_r, bs, hidden, seed=1)


def test_mla_backend_absorbed_prefill_then_decode():
    g = torch.Generator().manual_seed(2)
    nh, nope, rope, vd, kvl, hidden, bs = 4, 32, 64, 32, 512, 256, 16
    p = "model.layers.0."
    w = {
        p + "self_attn.q_proj.weight": torch.randn(nh * (nope + rope), hidden, generator=g) / 16,
        p + "self_attn.kv_a_proj_with_mqa.weight": torch.randn(kvl + rope, hidden, generator=g) / 16,
        p + "self_attn.kv_a_layernorm.weight": 1 + 0.1 * torch.randn(kvl, generator=g),
        p + "self_attn.kv_b_proj.weight": torch.randn(nh * (nope + vd), kvl, generator=g) / 22,
        p + "self_attn.o_proj.weight": torch.randn(hidden, nh * vd, generator=g) / 11,
    }
    w = {k: v.bfloat16().to(DEV) for k, v in w.items()}
    kw = dict(num_heads=nh, qk_nope=nope, qk_rope=rope, v_head_dim=vd, kv_lora_rank=kvl,
              q_lora_rank=None, rms_eps=1e-6, softmax_scale=(nope + rope) ** -0.5,
              num_layers=1, device=DEV, dtype=torch.bfloat16)
    hip = MlaHipBackend(w, **kw)
    twin = oracle_twin(MlaHipBackend)(w, **kw)
    caches_h = hip.alloc_kv_caches(8, bs)
    caches_r = twin.alloc_kv_caches(8, bs)
    steps = [[(0, 7, [2]), (0, 18, [5, 0])], [(7, 1, [2]), (18, 1, [5, 0])]]
    run_pair(hip, twin, steps, caches_h, caches_r, bs, hidden, seed=3)


@pytest.mark.parametrize("qwen3", [False, True])
@pytest.mark.parametrize("d", [128, 64])
def test_gqa_fused_pre_attention_matches_torch_path(qwen3, d):
    """The in-place QK-norm + RoPE kernel against the torch ops it replaces
    (split, rms_norm, rotate_half), end to end through attention(): without
    QK-norm the KV caches are bit-exact, with it within one bf16 ulp of each
    row's largest value."""
    g = torch.Generator().manual_seed(7)
    hq, hkv, hidden, bs = 8, 2, 256, 16
    p = "model.layers.0.self_attn."
    w = {p + "qkv_proj.weight": (torch.randn((hq + 2 * hkv) * d, hidden, generator=g) / 16).bfloat16(),
         p + "o_proj.weight": (torch.randn(hidden, hq * d, generator=g) / 32).bfloat16()}
    if qwen3:
        w[p + "q_norm.weight"] = (1 + 0.1 * torch.randn(d, generator=g)).bfloat16()
        w[p + "k_norm.weight"] = (1 + 0.1 * torch.randn(d, generator=g)).bfloat16()
    else:
        w[p + "qkv_proj.bias"] = (0.1 * torch.randn((hq + 2 * hkv) * d, generator=g)).bfloat16()
    w = {k: v.to(DEV) for k, v in w.items()}
    kw = dict(n_q_heads=hq, n_kv_heads=hkv, head_dim=d, scale=d ** -0.5, num_layers=1,
              device=DEV, dtype=torch.bfloat16, w=w, rms_eps=1e-6 if qwen3 else None)
    fused = GqaHipBackend(**kw)
    plain = GqaHipBackend(fuse_pre_attention=False, **kw)
    cf, cp = fused.alloc_kv_caches(10, bs), plain.alloc_kv_caches(10, bs)
    for rows in ([(0, 9, [4]), (0, 30, [1, 6])], [(9, 1, [4]), (30, 1, [1, 6])]):
        T = sum(n for _, n, _ in rows)
        x = (torch.randn(T, hidden, generator=g) * 0.5).bfloat16().to(DEV)
        ctx_f, positions = make_ctx(fused, cf, rows, bs)
        ctx_p, _ = make_ctx(plain, cp, rows, bs)
        cos, sin = rope_tables(positions * 37, d)
        ctx_f.cos = ctx_p.cos = cos.to(DEV)
        ctx_f.sin = ctx_p.sin = sin.to(DEV)
        of = fused.attention(0, x, ctx_f)
        op = plain.attention(0, x, ctx_p)
        torch.cuda.synchronize()
        if qwen3:
            diff = (cf[0].float() - cp[0].float()).abs()
            assert bool((diff <= cp[0].float().abs().amax(-1, keepdim=True) * 2.0 ** -7).all())
        else:
            assert torch.equal(cf[0].cpu(), cp[0].cpu())
        scale = op.float().abs().max().item()
        assert (of.float() - op.float()).abs().max().item() <= TOL * max(1.0, scale)


def test_gqa_backend_long_prefill_on_prefill_kernel():
    """Prompts long enough to fill 128-row items (tokens x group 4) run on the
    prefill kernel, with the new K/V rows written by it: caches bit-exact and
    outputs within tolerance, across a prefill, a chunked continuation beside
    a decode row, and a decode step."""
    g = torch.Generator().manual_seed(5)
    hq, hkv, d, hidden, bs = 8, 2, 128, 256, 16
    p = "model.layers.0.self_attn."
    w = {
        p + "qkv_proj.weight": (torch.randn((hq + 2 * hkv) * d, hidden, generator=g) / 16).bfloat16(),
        p + "o_proj.weight": (torch.randn(hidden, hq * d, generator=g) / 32).bfloat16(),
    }
    w = {k: v.to(DEV) for k, v in w.items()}
    kw = dict(n_q_heads=hq, n_kv_heads=hkv, head_dim=d, scale=d ** -0.5, num_layers=1,
              device=DEV, dtype=torch.bfloat16, w=w, rms_eps=1e-6)
    hip = GqaHipBackend(**kw)
    twin = oracle_twin(GqaHipBackend)(**kw)
    caches_h = hip.alloc_kv_caches(24, bs)
    caches_r = twin.alloc_kv_caches(24, bs)
    a, b = [3, 9, 4], [7, 1, 11, 2, 5, 13, 17, 6, 19, 20]
    steps = [
        [(0, 40, a), (0, 70, b[:5])],              # two prompts: 160 and 280 rows
        [(40, 1, a), (70, 64, b[:9])],             # decode + 64-token continuation (256 rows)
        [(41, 1, a), (134, 1, b[:9])],             # decode
    ]
    run_pair(hip, twin, steps, caches_h, caches_r, bs, hidden, seed=6)


def test_mla_fused_pre_attention_matches_torch_path():
    """The latent-query and latent-KV kernels against the torch ops they
    replace (split, rms_norm, ds_rope_interleave, RoPE, einsum with W_UK,
    cat), and the W_UV kernel against the einsum after attention, end to end
    through attention() with DeepSeek-V2-Lite head shapes
    (nope 128, rope 64, latent 512): the latent caches within one bf16 ulp of
    each row's largest value (the norm's sum order), outputs within 2e-2."""
    g = torch.Generator().manual_seed(9)
    nh, nope, rope, vd, kvl, hidden, bs = 16, 128, 64, 128, 512, 512, 16
    p = "model.layers.0."
    w = {
        p + "self_attn.q_proj.weight": torch.randn(nh * (nope + rope), hidden, generator=g) / 22,
        p + "self_attn.kv_a_proj_with_mqa.weight": torch.randn(kvl + rope, hidden, generator=g) / 22,
        p + "self_attn.kv_a_layernorm.weight": 1 + 0.1 * torch.randn(kvl, generator=g),
        p + "self_attn.kv_b_proj.weight": torch.randn(nh * (nope + vd), kvl, generator=g) / 22,
        p + "self_attn.o_proj.weight": torch.randn(hidden, nh * vd, generator=g) / 45,
    }
    w = {k: v.bfloat16().to(DEV) for k, v in w.items()}
    kw = dict(num_heads=nh, qk_nope=nope, qk_rope=rope, v_head_dim=vd, kv_lora_rank=kvl,
              q_lora_rank=None, rms_eps=1e-6, softmax_scale=(nope + rope) ** -0.5,
              num_layers=1, device=DEV, dtype=torch.bfloat16)
    fused = MlaHipBackend(w, **kw)
    plain = MlaHipBackend(w, fuse_pre_attention=False, **kw)
    cf, cp = fused.alloc_kv_caches(12, bs), plain.alloc_kv_caches(12, bs)
    for rows in ([(0, 11, [4]), (0, 40, [1, 6, 7])], [(11, 1, [4]), (40, 1, [1, 6, 7])]):
        T = sum(n for _, n, _ in rows)
        x = (torch.randn(T, hidden, generator=g) * 0.5).bfloat16().to(DEV)
        ctx_f, positions = make_ctx(fused, cf, rows, bs)
        ctx_p, _ = make_ctx(plain, cp, rows, bs)
        cos, sin = rope_tables(positions * 53, rope)
        ctx_f.cos = ctx_p.cos = cos.to(DEV)
        ctx_f.sin = ctx_p.sin = sin.to(DEV)
        assert fused._fusable(torch.zeros(T, nh, 192, dtype=torch.bfloat16, device=DEV),
                              torch.zeros(T, 576, dtype=torch.bfloat16, device=DEV), ctx_f)
        of = fused.attention(0, x, ctx_f)
        op = plain.attention(0, x, ctx_p)
        torch.cuda.synchronize()
        a, b = cf[0][0].float(), cp[0][0].float()
        assert bool(((a - b).abs() <= b.abs().amax(-1, keepdim=True) * 2.0 ** -7).all())
        scale = op.float().abs().max().item()
        err = (of.float() - op.float()).abs().max().item()
        print(f"output max-abs diff {err:.3e} (scale {scale:.2f})", flush=True)
        assert err <= TOL * max(1.0, scale)


def test_gqa_backend_head_dim_64_qwen25_05b_shape():
    """Qwen2.5-0.5B attention shape (14 query heads, 2 KV heads, head_dim 64
    = 896 / 14, qkv bias; the reference's own smoke-test model): prefill,
    decode, and a chunked continuation beside a decode row on the split-K
    path, caches bit-exact and outputs within tolerance."""
    g = torch.Generator().manual_seed(11)
    hq, hkv, d, hidden, bs = 14, 2, 64, 896, 16
    p = "model.layers.0.self_attn."
    w = {
        p + "qkv_proj.weight": (torch.randn((hq + 2 * hkv) * d, hidden, generator=g) / 30).bfloat16(),
        p + "qkv_proj.bias": (torch.randn((hq + 2 * hkv) * d, generator=g) / 4).bfloat16(),
        p + "o_proj.weight": (torch.randn(hidden, hq * d, generator=g) / 30).bfloat16(),
    }
    w = {k: v.to(DEV) for k, v in w.items()}
    kw = dict(n_q_heads=hq, n_kv_heads=hkv, head_dim=d, scale=d ** -0.5, num_layers=1,
              device=DEV, dtype=torch.bfloat16, w=w, rms_eps=1e-6)
    hip = GqaHipBackend(**kw)
    twin = oracle_twin(GqaHipBackend)(**kw)
    caches_h = hip.alloc_kv_caches(20, bs)
    caches_r = twin.alloc_kv_caches(20, bs)
    a, b = [3, 9, 4], [7, 1, 11, 2, 5, 13, 17, 6]
    steps = [
        [(0, 37, a), (0, 70, b[:5])],              # two prompts
        [(37, 1, a), (70, 1, b[:5])],              # decode
        [(38, 1, a), (71, 50, b)],                 # decode + chunked continuation
    ]
    run_pair(hip, twin, steps, caches_h, caches_r, bs, hidden, seed=12)


def _gqa_weights(seed, hq, hkv, d, hidden):
    g = torch.Generator().manual_seed(seed)
    p = "model.layers.0.self_attn."
    w = {p + "qkv_proj.weight": (torch.randn((hq + 2 * hkv) * d, hidden, generator=g) / 16).bfloat16(),
         p + "o_proj.weight": (torch.randn(hidden, hq * d, generator=g) / 32).bfloat16()}
    return {k: v.to(DEV) for k, v in w.items()}, g


def test_gqa_backend_writes_a_foreign_slot_mapping_as_given():
    """A context whose slot_mapping is not the block-table slot of each
    position (a caller's own padding or scratch slots) and that does not
    declare it derived: the backend writes K/V where slot_mapping says (the
    reference's write_kv semantics, base.py:41-45) instead of fusing the
    write, so the caches match the oracle bit for bit and attention reads
    what the block table points at."""
    hq, hkv, d, hidden, bs = 8, 2, 128, 256, 16
    w, g = _gqa_weights(21, hq, hkv, d, hidden)
    kw = dict(n_q_heads=hq, n_kv_heads=hkv, head_dim=d, scale=d ** -0.5, num_layers=1,
              device=DEV, dtype=torch.bfloat16, w=w, rms_eps=1e-6)
    hip = GqaHipBackend(**kw)
    twin = oracle_twin(GqaHipBackend)(**kw)
    ch, cr = hip.alloc_kv_caches(16, bs), twin.alloc_kv_caches(16, bs)
    rows = [(20, 3, [2, 5]), (7, 1, [9])]
    T = 4
    x = (torch.randn(T, hidden, generator=g) * 0.5).bfloat16().to(DEV)
    ctx_h, positions = make_ctx(hip, ch, rows, bs, derived=False)
    ctx_r, _ = make_ctx(twin, cr, rows, bs, derived=False)
    # the first request's rows go to scratch block 14, the decode row to 15
    foreign = torch.tensor([14 * bs, 14 * bs + 1, 14 * bs + 2, 15 * bs + 3], dtype=torch.int32,
                           device=DEV)
    ctx_h.slot_mapping = ctx_r.slot_mapping = foreign
    cos, sin = rope_tables(positions, d)
    ctx_h.cos = ctx_r.cos = cos.to(DEV)
    ctx_h.sin = ctx_r.sin = sin.to(DEV)
    twin.captured = []
    out_h = hip.attention(0, x, ctx_h)
    out_r = twin.attention(0, x, ctx_r)
    torch.cuda.synchronize()
    assert torch.equal(ch[0].cpu(), cr[0].cpu()), "KV cache differs from the oracle's"
    assert ch[0][:, 14].abs().sum().item() > 0 and ch[0][:, 2].abs().sum().item() == 0
    scale = out_r.float().abs().max().item()
    assert (out_h.float() - out_r.float()).abs().max().item() <= TOL * max(1.0, scale)


def test_two_contexts_in_flight_on_two_streams_through_the_backends():
    """Two steps of different shapes through GqaHipBackend.attention and
    MlaHipBackend.attention, launched back to back on two streams with no
    synchronisation between them (the reference runs per-slot steps on
    their own streams, graph_decode_runner.py:202-207, 475-481): each
    context plans into its own workspace, and both results match the
    oracle."""
    from oracle.paged_attn import mla_absorbed_attention as mla_ref
    hq, hkv, d, hidden, bs = 8, 2, 128, 256, 16
    w, g = _gqa_weights(31, hq, hkv, d, hidden)
    kw = dict(n_q_heads=hq, n_kv_heads=hkv, head_dim=d, scale=d ** -0.5, num_layers=1,
              device=DEV, dtype=torch.bfloat16, w=w, rms_eps=1e-6)
    gqa = GqaHipBackend(**kw)
    nh = 16
    mla = MlaHipBackend({}, num_heads=nh, qk_nope=128, qk_rope=64, v_head_dim=128,
                        kv_lora_rank=512, q_lora_rank=None, rms_eps=1e-6,
                        softmax_scale=192 ** -0.5, num_layers=1, device=DEV,
                        dtype=torch.bfloat16)
    gc = gqa.alloc_kv_caches(64, bs)
    mc = mla.alloc_kv_caches(64, bs)
    gc[0].normal_(generator=None)
    mc[0][0].normal_()
    perm = torch.randperm(64, generator=g).tolist()
    rows_a = [(300, 1, perm[:19]), (40, 90, perm[19:28]), (5, 1, perm[28:29])]
    rows_b = [(600, 1, perm[:38]), (100, 2, perm[38:45]), (33, 1, perm[45:48])]
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    ctx_a, _ = make_ctx(gqa, gc, rows_a, bs)
    ctx_b, _ = make_ctx(mla, mc, rows_b, bs)
    Ta, Tb = sum(r[1] for r in rows_a), sum(r[1] for r in rows_b)
    qa = (torch.randn(Ta, hq, d, generator=g) / 4).bfloat16().to(DEV)
    qb = torch.randn(Tb, nh, 576, generator=g).bfloat16().to(DEV)
    torch.cuda.synchronize()
    outs = {}
    for rep in range(3):
        with torch.cuda.stream(s1):
            oa = gqa._attn(0, qa, None, None, ctx_a)
        with torch.cuda.stream(s2):
            ob = mla._attn(0, qb, None, None, ctx_b)
        outs.setdefault("a", []).append(oa)
        outs.setdefault("b", []).append(ob)
        if rep == 0:      # new contexts for the later rounds: fresh plans and workspaces
            ctx_a, _ = make_ctx(gqa, gc, rows_a, bs)
            ctx_b, _ = make_ctx(mla, mc, rows_b, bs)
    torch.cuda.synchronize()
    assert ctx_a._aia_plans and ctx_b._aia_plans
    pa = next(iter(ctx_a._aia_plans.values()))
    pb = next(iter(ctx_b._aia_plans.values()))
    assert pa.workspace.data_ptr() != pb.workspace.data_ptr()
    ref_a = paged_attention(qa.cpu(), gc[0][0].cpu(), gc[0][1].cpu(), ctx_a.block_table.cpu(),
                            ctx_a.cu_seqlens_q, ctx_a.seqlens_kv, d ** -0.5)
    ref_b = mla_ref(qb.cpu(), mc[0][0].cpu(), ctx_b.block_table.cpu(), ctx_b.cu_seqlens_q,
                    ctx_b.seqlens_kv, 192 ** -0.5, 512)
    for o in outs["a"]:
        assert (o.float().cpu() - ref_a).abs().max().item() <= TOL
    for o in outs["b"]:
        assert (o.float().cpu() - ref_b).abs().max().item() <= TOL


def test_two_host_threads_gqa_and_mla_planning_every_step():
    """Two host threads, each with its own stream, plan and run attention
    steps at the same time (GQA in one, absorbed MLA in the other, a new
    plan every step): the C-ABI holds no shared mutable state beyond its
    thread-local error text, so every step of both matches the oracle."""
    import threading
    from auto_infer_amd import ops, workloads
    from oracle.paged_attn import mla_absorbed_attention as mla_ref
    ga = workloads.make_gqa_step(lqs=[1, 3, 1, 40], lks=[500, 90, 1200, 300], num_q_heads=16,
                                 num_kv_heads=4, block_size=16, seed=71)
    mb = workloads.make_mla_step(lqs=[1, 1, 2], lks=[2000, 300, 700], num_heads=16,
                                 block_size=64, seed=72)
    exp_a = paged_attention(ga.q, ga.k_cache, ga.v_cache, ga.block_table, ga.cu_seqlens_q,
                            ga.seqlens_kv, ga.scale)
    exp_b = mla_ref(mb.q_latent, mb.cache, mb.block_table, mb.cu_seqlens_q, mb.seqlens_kv,
                    mb.scale, 512)
    dev_a = {n: getattr(ga, n).to(DEV) for n in ("q", "k_cache", "v_cache", "block_table")}
    dev_b = {n: getattr(mb, n).to(DEV) for n in ("q_latent", "cache", "block_table")}
    torch.cuda.synchronize()
    outs, errs = {"a": [], "b": []}, []

    def run_a():
        try:
            s = torch.cuda.Stream()
            with torch.cuda.stream(s):
                for _ in range(20):
                    plan = ops.AttentionPlan.from_lists(dev_a["block_table"], ga.cu_seqlens_q,
                                                        ga.seqlens_kv, 16, 4, 128, 16)
                    outs["a"].append(ops.paged_attention_gqa(dev_a["q"], dev_a["k_cache"],
                                                             dev_a["v_cache"], plan, ga.scale))
            s.synchronize()
        except Exception as e:      # surfaced by the main thread
            errs.append(e)

    def run_b():
        try:
            s = torch.cuda.Stream()
            with torch.cuda.stream(s):
                for _ in range(20):
                    plan = ops.AttentionPlan.from_lists(dev_b["block_table"], mb.cu_seqlens_q,
                                                        mb.seqlens_kv, 16, 1, 512, 64)
                    outs["b"].append(ops.paged_attention_mla(dev_b["q_latent"], dev_b["cache"],
                                                             plan, mb.scale))
            s.synchronize()
        except Exception as e:
            errs.append(e)

    ts = [threading.Thread(target=run_a), threading.Thread(target=run_b)]
    for t in ts:
        t.start()
    for t in ts:
        t.join(timeout=120)
    assert not errs, errs
    torch.cuda.synchronize()
    assert len(outs["a"]) == 20 and len(outs["b"]) == 20
    for o in outs["a"]:
        assert (o.float().cpu() - exp_a).abs().max().item() <= 2e-2
    for o in outs["b"]:
        assert (o.float().cpu() - exp_b).abs().max().item() <= 2e-2


def _overflow_ctx(backend, caches, bs):
    """A context whose device metadata (as a packer attaches it) does not add
    up: cu_seqlens_q describes 100 query tokens in a 10-token step."""
    rows = [(0, 5, [3]), (0, 5, [7, 1])]
    ctx, positions = make_ctx(backend, caches, rows, bs, derived=False)
    ctx.aia_cu_seqlens_q = torch.tensor([0, 5, 100], dtype=torch.int32, device=DEV)
    ctx.aia_seqlens_kv = torch.tensor([5, 100], dtype=torch.int32, device=DEV)
    cos, sin = rope_tables(positions, 128)
    ctx.cos, ctx.sin = cos.to(DEV), sin.to(DEV)
    return ctx


def _small_gqa(seed):
    g = torch.Generator().manual_seed(seed)
    hq, hkv, d, hidden = 4, 2, 128, 256
    p = "model.layers.0.self_attn."
    w = {p + "qkv_proj.weight": (torch.randn((hq + 2 * hkv) * d, hidden, generator=g) / 16).bfloat16(),
         p + "o_proj.weight": (torch.randn(hidden, hq * d, generator=g) / 23).bfloat16()}
    w = {k: v.to(DEV) for k, v in w.items()}
    return GqaHipBackend(n_q_heads=hq, n_kv_heads=hkv, head_dim=d, scale=d ** -0.5,
                         num_layers=1, device=DEV, dtype=torch.bfloat16, w=w), hidden


def test_gqa_backend_planner_overflow_is_visible(monkeypatch):
    """Device metadata that overflows the planner: the attention op's output
    is all NaN (not uninitialised memory), and with AIA_CHECK_PLAN=1 the
    step's planning raises the stager contract's ValueError
    (prefill_input_stager.py:77-81)."""
    bs = 16
    hip, hidden = _small_gqa(3)
    caches = hip.alloc_kv_caches(12, bs)
    x = (torch.randn(10, hidden) * 0.5).bfloat16().to(DEV)
    ctx = _overflow_ctx(hip, caches, bs)
    got = []
    orig = hip._attn

    def spy(*a, **k):
        o = orig(*a, **k)
        got.append(o)
        return o
    hip._attn = spy
    monkeypatch.delenv("AIA_CHECK_PLAN", raising=False)
    hip.attention(0, x, ctx)
    torch.cuda.synchronize()
    assert got[0].shape == (10, 4, 128)
    assert torch.isnan(got[0].float()).all(), "overflowed plan left output values"
    hip._attn = orig
    monkeypatch.setenv("AIA_CHECK_PLAN", "1")
    ctx2 = _overflow_ctx(hip, caches, bs)
    with pytest.raises(ValueError, match="overflow"):
        hip.attention(0, x, ctx2)


def test_mla_planner_overflow_fills_nan():
    """The same for the absorbed-MLA call: its merge pass fills the latent
    output with NaN when the plan overflowed."""
    from auto_infer_amd import ops
    bt = torch.arange(8, dtype=torch.int32, device=DEV).view(2, 4)
    cu = torch.tensor([0, 5, 100], dtype=torch.int32, device=DEV)
    kv = torch.tensor([5, 100], dtype=torch.int32, device=DEV)
    plan = ops.AttentionPlan(bt, cu, kv, 10, 16, 1, 512, 64)
    q = torch.randn(10, 16, 576, device=DEV).bfloat16()
    cache = torch.randn(8, 64, 1, 576, device=DEV).bfloat16()
    out = ops.paged_attention_mla(q, cache, plan, 0.1)
    torch.cuda.synchronize()
    assert torch.isnan(out.float()).all()
