"""The allocation-free GQA entry point (aia_paged_attention_gqa_noalloc,
plan and partials in the library's static device scratch) through the
C-ABI, against the workspace entry point aia_paged_attention_gqa: outputs
and KV caches bit-identical, on two calls in a row, the second with a
smaller step, and within 2e-2 of the oracle."""
import os
import subprocess
import sys
import textwrap

import pytest
import torch

from auto_infer_amd import _native, ops, workloads
from oracle.paged_attn import paged_attention

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _noalloc(q, kc, vc, bt, cu, kv, batch, T, hq, hkv, d, bs, nb, scale, out, kn, vn,
             num_waves=0, flags=0):
    _native.call("aia_paged_attention_gqa_noalloc", q.data_ptr(), q.stride(0), q.stride(1),
                 kc.data_ptr(), vc.data_ptr(), bt.data_ptr(), bt.stride(0), cu.data_ptr(),
                 kv.data_ptr(), batch, T, hq, hkv, d, bs, nb, float(scale), out.data_ptr(),
                 out.stride(0), out.stride(1), kn.data_ptr() if kn is not None else None,
                 vn.data_ptr() if vn is not None else None,
                 kn.stride(0) if kn is not None else 0, vn.stride(0) if vn is not None else 0,
                 num_waves, flags, torch.cuda.current_stream(DEV).cuda_stream)


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


def test_noalloc_nz_layout_matches_workspace_entry():
    """AIA_ATTN_KV_NZ through the allocation-free entry point: caches in the
    reference's graph-mode NZ layout, fused write included, bit-identical to
    the workspace entry point over the same caches."""
    from oracle.paged_attn import nz_from_nd
    step = workloads.make_gqa_step(lqs=[1, 2, 150, 1], lks=[700, 33, 400, 2000], num_q_heads=28,
                                   num_kv_heads=4, block_size=16, seed=6, extra_blocks=2)
    hq, hkv, d, bs, nb = 28, 4, 128, 16, step.k_cache.shape[0]
    T, B = step.num_tokens, len(step.seqlens_kv)
    q, bt = step.q.to(DEV), step.block_table.to(DEV)
    kn, vn = step.k_new.to(DEV), step.v_new.to(DEV)
    k1, v1 = nz_from_nd(step.k_cache).to(DEV), nz_from_nd(step.v_cache).to(DEV)
    k2, v2 = k1.clone(), v1.clone()
    plan = ops.AttentionPlan.from_lists(bt, step.cu_seqlens_q, step.seqlens_kv, hq, hkv, d, bs)
    want = ops.paged_attention_gqa(q, k1, v1, plan, step.scale, key_new=kn, value_new=vn,
                                   kv_layout="nz")
    got = torch.empty_like(want)
    print("no-alloc: NZ caches, mixed step with the fused write", flush=True)
    _noalloc(q, k2, v2, bt, plan.cu_seqlens_q, plan.seqlens_kv, B, T, hq, hkv, d, bs, nb,
             step.scale, got, kn, vn, flags=ops.KV_LAYOUTS["nz"])
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    assert torch.equal(k1, k2) and torch.equal(v1, v2)


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


def test_noalloc_allocates_nothing_and_replays_in_a_graph():
    """A warm call changes neither torch's allocated nor reserved device
    memory; one call captured in a HIP graph and replayed (with eager work
    and synchronisations between replays) matches the workspace entry point
    on every replay."""
    step = workloads.config1_decode(seed=7)
    hq, hkv, d = 16, 8, 128
    bs, nb = step.k_cache.shape[1], step.k_cache.shape[0]
    q, bt = step.q.to(DEV), step.block_table.to(DEV)
    kc, vc = step.k_cache.to(DEV), step.v_cache.to(DEV)
    plan = ops.AttentionPlan.from_lists(bt, step.cu_seqlens_q, step.seqlens_kv, hq, hkv, d, bs)
    want = ops.paged_attention_gqa(q, kc, vc, plan, step.scale)
    got = torch.empty_like(want)
    args = (q, kc, vc, bt, plan.cu_seqlens_q, plan.seqlens_kv, 16, 16, hq, hkv, d, bs, nb,
            step.scale, got, None, None)
    _noalloc(*args)                      # warm: the scratch address is resolved
    torch.cuda.synchronize()
    alloc0, res0 = torch.cuda.memory_allocated(DEV), torch.cuda.memory_reserved(DEV)
    free0 = torch.cuda.mem_get_info(DEV)[0]
    _noalloc(*args)
    torch.cuda.synchronize()
    assert torch.cuda.memory_allocated(DEV) == alloc0
    assert torch.cuda.memory_reserved(DEV) == res0
    assert torch.cuda.mem_get_info(DEV)[0] == free0
    assert torch.equal(got, want)

    side = torch.cuda.Stream(DEV)
    side.wait_stream(torch.cuda.current_stream(DEV))
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        got.zero_()
        with torch.cuda.graph(graph, stream=side):
            _noalloc(*args)               # on the capturing stream (current)
    torch.cuda.current_stream(DEV).wait_stream(side)
    for i in range(3):
        got.fill_(7.0)
        junk = torch.randn(1 << 20, device=DEV).sum()        # eager work between replays
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"replay {i} differs from the workspace entry point"
        del junk


def test_scratch_is_reserved_only_by_the_noalloc_entry():
    """In a fresh process, launching the workspace entry points leaves the
    static scratch unreserved (device free memory drops by far less than its
    size); the first allocation-free call then reserves it."""
    code = textwrap.dedent("""
        import torch, ctypes
        from auto_infer_amd import _native, ops, workloads
        dev = torch.device("cuda:0")
        n = ctypes.c_int64(0)
        _native.call("aia_noalloc_scratch_bytes", ctypes.byref(n))
        step = workloads.config1_decode(seed=1)
        q, bt = step.q.to(dev), step.block_table.to(dev)
        kc, vc = step.k_cache.to(dev), step.v_cache.to(dev)
        torch.cuda.synchronize()
        free0 = torch.cuda.mem_get_info(dev)[0]
        plan = ops.AttentionPlan.from_lists(bt, step.cu_seqlens_q, step.seqlens_kv, 16, 8, 128, 128)
        out = ops.paged_attention_gqa(q, kc, vc, plan, step.scale)
        got = torch.empty_like(out)
        torch.cuda.synchronize()
        free1 = torch.cuda.mem_get_info(dev)[0]
        _native.call("aia_paged_attention_gqa_noalloc", q.data_ptr(), q.stride(0), q.stride(1),
                     kc.data_ptr(), vc.data_ptr(), bt.data_ptr(), bt.stride(0),
                     plan.cu_seqlens_q.data_ptr(), plan.seqlens_kv.data_ptr(), 16, 16, 16, 8,
                     128, 128, kc.shape[0], float(step.scale), got.data_ptr(), got.stride(0),
                     got.stride(1), None, None, 0, 0, 0, 0,
                     torch.cuda.current_stream(dev).cuda_stream)
        torch.cuda.synchronize()
        free2 = torch.cuda.mem_get_info(dev)[0]
        assert torch.equal(got, out)
        print(n.value, free0 - free1, free1 - free2)
    """)
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=240,
                       cwd=root)
    assert r.returncode == 0, r.stderr[-2000:]
    scratch, first, second = map(int, r.stdout.split()[-3:])
    print(f"scratch {scratch >> 20} MiB; workspace launches took {first >> 20} MiB of device "
          f"memory, the first no-alloc call {second >> 20} MiB", flush=True)
    assert first < scratch // 2, "the workspace entry points reserved the static scratch"
    assert second >= scratch, "the first no-alloc call did not reserve its scratch"
