"""The allocation-free GQA entry point (aia_paged_attention_gqa_noalloc,
plan and partials in the library's static device scratch) through the
C-ABI, against the workspace entry point aia_paged_attention_gqa: outputs
and KV caches bit-identical, on two calls in a row, the second with a
smaller step, and within 2e-2 of the oracle."""
import pytest
import torch

from auto_infer_amd import _native, ops, workloads
from oracle.paged_attn import paged_attention

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _noalloc(q, kc, vc, bt, cu, kv, batch, T, hq, hkv, d, bs, nb, scale, out, kn, vn,
             num_waves=0):
    _native.call("aia_paged_attention_gqa_noalloc", q.data_ptr(), q.stride(0), q.stride(1),
                 kc.data_ptr(), vc.data_ptr(), bt.data_ptr(), bt.stride(0), cu.data_ptr(),
                 kv.data_ptr(), batch, T, hq, hkv, d, bs, nb, float(scale), out.data_ptr(),
                 out.stride(0), out.stride(1), kn.data_ptr() if kn is not None else None,
                 vn.data_ptr() if vn is not None else None,
                 kn.stride(0) if kn is not None else 0, vn.stride(0) if vn is not None else 0,
                 num_waves, 0, torch.cuda.current_stream(DEV).cuda_stream)


def _run_both(step, fused):
    hq, hkv, d = step.q.shape[1], step.k_cache.shape[2], step.q.shape[2]
    bs, nb = step.k_cache.shape[1], step.k_cache.shape[0]
    T, B = step.num_tokens, len(step.seqlens_kv)
    q = step.q.to(DEV)
    bt = step.block_table.to(DEV)
    kn = step.k_new.to(DEV) if fused else None
    vn = step.v_new.to(DEV) if fused else None
    k1, v1 = step.k_cache.to(DEV), step.v_cache.to(DEV)
    k2, v2 = k1.clone(), v1.clone()
    plan = ops.AttentionPlan.from_lists(bt, step.cu_seqlens_q, step.seqlens_kv, hq, hkv, d, bs)
    want = ops.paged_attention_gqa(q, k1, v1, plan, step.scale, key_new=kn, value_new=vn)
    got = torch.empty_like(want)
    _noalloc(q, k2, v2, bt, plan.cu_seqlens_q, plan.seqlens_kv, B, T, hq, hkv, d, bs, nb,
             step.scale, got, kn, vn)
    torch.cuda.synchronize()
    assert torch.equal(got, want), "no-alloc output differs from the workspace entry point"
    assert torch.equal(k1, k2) and torch.equal(v1, v2)
    ref = paged_attention(step.q, k1.cpu(), v1.cpu(), step.block_table, step.cu_seqlens_q,
                          step.seqlens_kv, step.scale)
    assert (got.float().cpu() - ref).abs().max().item() <= 2e-2


def test_noalloc_matches_workspace_entry_on_two_calls():
    big = workloads.config1_decode(seed=3)
    small = workloads.make_gqa_step(lqs=[1, 2, 1], lks=[300, 33, 5], num_q_heads=16,
                                    num_kv_heads=8, block_size=128, seed=4, extra_blocks=2)
    print("no-alloc: config-1 step, then a 3-request step", flush=True)
    _run_both(big, fused=True)
    _run_both(small, fused=True)
    print("no-alloc: mixed prefill + decode, then config-1 step without the fused write",
          flush=True)
    mixed = workloads.make_gqa_step(lqs=[200, 1, 1], lks=[900, 77, 4000], num_q_heads=28,
                                    num_kv_heads=4, block_size=128, seed=5)
    _run_both(mixed, fused=False)
    _run_both(big, fused=False)


def test_noalloc_rejects_steps_past_its_scratch():
    step = workloads.config1_decode(seed=3)
    q = step.q.to(DEV)
    out = torch.empty_like(q)
    bt = step.block_table.to(DEV)
    cu = torch.tensor([0, *step.cu_seqlens_q], dtype=torch.int32, device=DEV)
    kv = torch.tensor(step.seqlens_kv, dtype=torch.int32, device=DEV)
    k, v = step.k_cache.to(DEV), step.v_cache.to(DEV)
    with pytest.raises(ValueError, match="static scratch"):
        _noalloc(q, k, v, bt, cu, kv, 16, 16, 16, 8, 128, 128, k.shape[0], step.scale, out,
                 None, None, num_waves=16384)
