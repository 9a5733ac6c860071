"""Paged GQA attention on the GPU vs the float32 gather-softmax oracle.

Tolerance (north star): 2e-2 max-abs, bf16 in/out, fp32 accumulation.
"""
import numpy as np
import pytest
import torch

from auto_infer_amd import ops, workloads
from oracle.paged_attn import kv_write, paged_attention

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
TOL = 2e-2


def run_gpu(step, num_waves=0):
    s = step
    plan = ops.AttentionPlan.from_lists(s.block_table.to(DEV), s.cu_seqlens_q, s.seqlens_kv,
                                        s.q.shape[1], s.k_cache.shape[2], s.q.shape[2],
                                        s.k_cache.shape[1], num_waves=num_waves)
    out = ops.paged_attention_gqa(s.q.to(DEV), s.k_cache.to(DEV), s.v_cache.to(DEV), plan,
                                  s.scale)
    torch.cuda.synchronize()
    return out.float().cpu()


def oracle(step):
    return paged_attention(step.q, step.k_cache, step.v_cache, step.block_table,
                           step.cu_seqlens_q, step.seqlens_kv, step.scale)


def check(step, num_waves=0):
    got = run_gpu(step, num_waves)
    exp = oracle(step)
    err = (got - exp).abs().max().item()
    print(f"max-abs err {err:.3e}", flush=True)
    assert err <= TOL, err
    return got


def test_config1_decode_shape():
    check(workloads.config1_decode(seed=3))


@pytest.mark.parametrize("waves", [1, 7, 64, 0])
def test_split_count_invariance(waves):
    """The result does not depend on how the key range is split."""
    step = workloads.make_gqa_step(lqs=[1, 1, 1], lks=[300, 17, 1000], num_q_heads=8,
                                   num_kv_heads=2, block_size=16, seed=11)
    check(step, waves)


def test_repeated_calls_on_one_plan():
    """Many layers on one plan give the same result (the plan is read-only)."""
    step = workloads.make_gqa_step(lqs=[1, 2, 1], lks=[900, 40, 2000], num_q_heads=16,
                                   num_kv_heads=8, block_size=128, seed=13)
    plan = ops.AttentionPlan.from_lists(step.block_table.to(DEV), step.cu_seqlens_q,
                                        step.seqlens_kv, 16, 8, 128, 128, num_waves=37)
    q, kc, vc = step.q.to(DEV), step.k_cache.to(DEV), step.v_cache.to(DEV)
    first = ops.paged_attention_gqa(q, kc, vc, plan, step.scale).clone()
    for _ in range(5):
        again = ops.paged_attention_gqa(q, kc, vc, plan, step.scale)
    torch.cuda.synchronize()
    assert torch.equal(first.cpu(), again.cpu())
    exp = oracle(step)
    assert (first.float().cpu() - exp).abs().max().item() <= TOL


@pytest.mark.parametrize("group", [1, 2, 4, 7, 8, 16])
def test_gqa_groups_decode(group):
    hkv = 2
    step = workloads.make_gqa_step(lqs=[1] * 5, lks=[1, 15, 16, 129, 700],
                                   num_q_heads=hkv * group, num_kv_heads=hkv,
                                   block_size=16, seed=group)
    check(step)


def test_mtp_verify_two_token_causal():
    """Lq = 2 per request, causal inside the pair (config 4 shape, small)."""
    step = workloads.make_gqa_step(lqs=[2] * 4, lks=[1024, 1500, 2, 4096], num_q_heads=32,
                                   num_kv_heads=8, block_size=128, seed=4)
    check(step)


def test_chunked_prefill_and_decode_mixed():
    """Ragged batch: prefill chunks continuing a prefix plus decode rows."""
    step = workloads.make_gqa_step(lqs=[37, 1, 5, 1, 64], lks=[37 + 100, 300, 5, 77, 64],
                                   num_q_heads=28, num_kv_heads=4, block_size=16, seed=9)
    check(step)


@pytest.mark.parametrize("lqs,lks,hq,hkv,bs", [
    ([37, 1, 5, 1, 64], [137, 300, 5, 77, 64], 28, 4, 16),   # group 7: 2 tokens per block
    ([3], [50], 7, 1, 16),                                  # second block holds one token
    ([100, 1], [130, 40], 4, 4, 16),                        # group 1: 16 tokens per block
    ([40, 3], [400, 3], 64, 2, 128),                        # group 32: head blocks
])
@pytest.mark.parametrize("waves", [1, 7, 64, 0])
def test_two_row_blocks(lqs, lks, hq, hkv, bs, waves):
    """Launches whose requests average more query tokens than a 16-row block
    holds run segments of two row blocks (every K/V tile feeds both); the
    result does not depend on it, nor on the split count."""
    step = workloads.make_gqa_step(lqs=lqs, lks=lks, num_q_heads=hq, num_kv_heads=hkv,
                                   block_size=bs, seed=41)
    check(step, waves)


def test_block_size_not_multiple_of_tile():
    step = workloads.make_gqa_step(lqs=[1, 3], lks=[45, 90], num_q_heads=4,
                                   num_kv_heads=2, block_size=4, seed=2)
    check(step)


def test_large_group_split_heads():
    """Hq/Hkv = 32 > 16 query rows per tile: heads are split over segments."""
    step = workloads.make_gqa_step(lqs=[1, 2], lks=[200, 513], num_q_heads=64,
                                   num_kv_heads=2, block_size=128, seed=5)
    check(step)


def test_block_permutation_invariance():
    """Moving KV blocks in the pool (and the table with them) changes nothing."""
    step = workloads.make_gqa_step(lqs=[1, 4], lks=[333, 260], num_q_heads=8,
                                   num_kv_heads=4, block_size=16, seed=21, extra_blocks=13)
    a = run_gpu(step)
    nb = step.k_cache.shape[0]
    perm = torch.randperm(nb, generator=torch.Generator().manual_seed(1))
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(nb)
    step.k_cache = step.k_cache[perm]
    step.v_cache = step.v_cache[perm]
    step.block_table = inv[step.block_table.long()].to(torch.int32)
    b = run_gpu(step)
    assert torch.equal(a, b)


def test_empty_context_rows_are_zero():
    step = workloads.make_gqa_step(lqs=[1, 1], lks=[1, 40], num_q_heads=4, num_kv_heads=2,
                                   block_size=16, seed=3)
    step.seqlens_kv = [0, 40]        # request 0 sees nothing
    got = run_gpu(step)
    assert torch.count_nonzero(got[0]) == 0


def test_plan_from_another_stream_is_waited_for():
    """A plan made on one stream is used on another: the attention waits."""
    step = workloads.make_gqa_step(lqs=[1, 3], lks=[700, 90], num_q_heads=8, num_kv_heads=2,
                                   block_size=16, seed=17)
    q, kc, vc = step.q.to(DEV), step.k_cache.to(DEV), step.v_cache.to(DEV)
    plan = ops.AttentionPlan.from_lists(step.block_table.to(DEV), step.cu_seqlens_q,
                                        step.seqlens_kv, 8, 2, 128, 16)
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        out = ops.paged_attention_gqa(q, kc, vc, plan, step.scale)
    torch.cuda.synchronize()
    assert (out.float().cpu() - oracle(step)).abs().max().item() <= TOL
    g = torch.cuda.CUDAGraph()
    with pytest.raises(ValueError, match="another stream"):
        with torch.cuda.graph(g, stream=side):
            ops.paged_attention_gqa(q, kc, vc, plan, step.scale)


@pytest.mark.parametrize("lqs,lks,hq,hkv,bs,waves", [
    ([1] * 16, [300, 129, 2048, 17, 1, 700, 901, 64, 65, 128, 1000, 5, 6, 1500, 333, 2],
     16, 8, 128, 0),                                    # decode, config-1 heads
    ([37, 1, 5, 1, 64], [137, 300, 5, 77, 64], 28, 4, 16, 0),   # chunked prefill, many q-blocks
    ([2, 2, 1], [513, 40, 999], 64, 2, 128, 7),        # head blocks (group 32), splits
    ([2] * 4, [1024, 1500, 2, 4096], 32, 8, 128, 3),   # MTP verify shape
    ([200, 1, 130, 19], [300, 77, 130, 40], 28, 4, 16, 0),   # prefill route, with/without prefix
    ([256, 3], [256 + 1000, 900], 16, 8, 128, 0),      # prefill route, group 2
    ([300], [6000], 16, 8, 128, 0),                    # prefill items cut into key chunks
])
def test_fused_kv_write(lqs, lks, hq, hkv, bs, waves):
    """The attention kernel performs the KV slot write of the step's new rows:
    caches bit-exact with the oracle write, output within tolerance."""
    step = workloads.make_gqa_step(lqs=lqs, lks=lks, num_q_heads=hq, num_kv_heads=hkv,
                                   block_size=bs, seed=31, extra_blocks=2)
    ek, ev = step.k_cache.clone(), step.v_cache.clone()
    kv_write(step.k_new, step.v_new, ek, ev, step.slot_mapping)
    exp = paged_attention(step.q, ek, ev, step.block_table, step.cu_seqlens_q, step.seqlens_kv,
                          step.scale)
    kc, vc = step.k_cache.to(DEV), step.v_cache.to(DEV)
    plan = ops.AttentionPlan.from_lists(step.block_table.to(DEV), step.cu_seqlens_q,
                                        step.seqlens_kv, hq, hkv, 128, bs, num_waves=waves)
    out = ops.paged_attention_gqa(step.q.to(DEV), kc, vc, plan, step.scale,
                                  key_new=step.k_new.to(DEV), value_new=step.v_new.to(DEV))
    torch.cuda.synchronize()
    assert torch.equal(kc.cpu(), ek) and torch.equal(vc.cpu(), ev)
    err = (out.float().cpu() - exp).abs().max().item()
    print(f"max-abs err {err:.3e}", flush=True)
    assert err <= TOL


def test_two_host_threads_on_two_streams():
    """The boundary is reentrant (no mutable global state; errors are
    thread-local): two host threads, each with its own stream and plan,
    call the attention concurrently and both match the oracle."""
    import threading
    steps = [workloads.make_gqa_step(lqs=[1, 3, 1], lks=[500, 90, 1500], num_q_heads=16,
                                     num_kv_heads=8, block_size=128, seed=s) for s in (51, 52)]
    exp = [oracle(st) for st in steps]
    got, errors = [None, None], []

    def worker(i):
        try:
            st = steps[i]
            stream = torch.cuda.Stream()
            with torch.cuda.stream(stream):
                q, kc, vc = st.q.to(DEV), st.k_cache.to(DEV), st.v_cache.to(DEV)
                plan = ops.AttentionPlan.from_lists(st.block_table.to(DEV), st.cu_seqlens_q,
                                                    st.seqlens_kv, 16, 8, 128, 128)
                for _ in range(20):
                    out = ops.paged_attention_gqa(q, kc, vc, plan, st.scale)
                stream.synchronize()
                got[i] = out.float().cpu()
        except Exception as e:          # reported by the main thread
            errors.append(e)

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors
    for g, e in zip(got, exp):
        assert (g - e).abs().max().item() <= TOL


def _fast_decode_step(B, hq, hkv, bs, lks, seed):
    """A decode step built without per-request Python loops (large batches):
    consecutive blocks per request, random bf16 Q and caches."""
    g = torch.Generator().manual_seed(seed)
    lks = np.asarray(lks)
    nblk = (lks + bs - 1) // bs
    first = np.concatenate([[0], np.cumsum(nblk)[:-1]])
    width = int(nblk.max())
    cols = np.arange(width)[None, :]
    bt = np.where(cols < nblk[:, None], first[:, None] + cols, 0).astype(np.int32)
    NB = int(nblk.sum())
    s = workloads.GqaStep(
        q=(torch.randn(B, hq, 128, generator=g) * 0.5).bfloat16(),
        k_new=None, v_new=None,
        k_cache=torch.randn(NB, bs, hkv, 128, generator=g).bfloat16(),
        v_cache=torch.randn(NB, bs, hkv, 128, generator=g).bfloat16(),
        block_table=torch.from_numpy(bt), cu_seqlens_q=list(range(1, B + 1)),
        seqlens_kv=lks.tolist(), slot_mapping=None, scale=128 ** -0.5)
    return s


@pytest.mark.parametrize("B,hq,hkv", [(5000, 8, 8), (8192, 16, 16)])
def test_planner_large_batch_paths(B, hq, hkv):
    """Batches past the planner's LDS copy of the request metadata (> 4095
    requests) and past its register copy of the segment tile counts (> 8192
    segments: 8192 requests x 2 kv-head groups)."""
    lks = [1 + (i * 7) % 40 for i in range(B)]
    check(_fast_decode_step(B, hq, hkv, 16, lks, seed=B))


def test_planner_rejects_batches_past_its_limit():
    st = _fast_decode_step(8193, 8, 8, 16, [1] * 8193, seed=1)
    with pytest.raises(ValueError, match="exceeds planner limit"):
        ops.AttentionPlan.from_lists(st.block_table.to(DEV), st.cu_seqlens_q, st.seqlens_kv,
                                     8, 8, 128, 16)


@pytest.mark.parametrize("lq", [1, 3])
def test_very_long_context(lq):
    """131072 keys: many 64-block windows of block ids per range."""
    check(workloads.make_gqa_step(lqs=[lq], lks=[131072], num_q_heads=4, num_kv_heads=1,
                                  block_size=128, seed=4), 0)


def test_empty_step():
    """No query tokens: nothing is launched and the output is empty."""
    plan = ops.AttentionPlan.from_lists(torch.zeros(0, 1, dtype=torch.int32, device=DEV), [],
                                        [], 16, 8, 128, 16)
    q = torch.zeros(0, 16, 128, dtype=torch.bfloat16, device=DEV)
    kc = torch.zeros(4, 16, 8, 128, dtype=torch.bfloat16, device=DEV)
    out = ops.paged_attention_gqa(q, kc, kc, plan, 128 ** -0.5)
    assert out.shape == (0, 16, 128)


@pytest.mark.parametrize("lqs,lks,hq,hkv,bs", [
    ([512, 512, 512], [1383, 1164, 1035], 28, 4, 128),    # configs[1] prefill chunks
    ([19, 18, 1], [19, 50, 300], 28, 4, 16),              # 133 rows routed, 126 stay split-K
    ([200], [200], 16, 8, 16),                            # group 2, no prefix
    ([130, 7], [1000, 7], 8, 8, 128),                     # group 1
    ([64, 9], [100, 700], 64, 4, 16),                     # group 16
    ([8, 2], [8, 600], 64, 2, 128),                       # group 32: 256 rows from 8 tokens
    ([300], [300 + 4000], 32, 8, 128),                    # long prefix
    ([129, 1], [129, 5], 4, 1, 4),                        # block size 4: blocks inside a tile
    ([100, 70], [700, 70], 28, 4, 64),                    # block size = tile
    ([300], [1300], 16, 8, 256),                          # tiles inside a block
])
@pytest.mark.parametrize("d", [128, 64])
def test_prefill_route(lqs, lks, hq, hkv, bs, d):
    """Requests whose query rows (tokens x group) fill a 128-row item run on
    the prefill kernel (K/V tiles staged in LDS once per 128 rows); the rest
    of the batch stays on split-K.  Both against the oracle, at head_dim 128
    and 64; the plan's header shows the prefill units."""
    step = workloads.make_gqa_step(lqs=lqs, lks=lks, num_q_heads=hq, num_kv_heads=hkv,
                                   head_dim=d, block_size=bs, seed=57)
    plan = ops.AttentionPlan.from_lists(step.block_table.to(DEV), step.cu_seqlens_q,
                                        step.seqlens_kv, hq, hkv, d, bs)
    torch.cuda.synchronize()
    assert plan.workspace[:64].cpu().view(torch.int32)[6].item() > 0     # prefill units
    check(step)


def test_prefill_whole_items_past_64_tiles():
    """63 items of 128 rows x 8 kv heads = 504 work-groups fit one round, so
    no item is cut and each unit walks all of its 65-72 key tiles: the block
    ids (one per 64-key tile, fetched 64 tiles at a time) are fetched again
    past tile 64.  Against the oracle."""
    step = workloads.make_gqa_step(lqs=[504], lks=[4600], num_q_heads=128, num_kv_heads=8,
                                   block_size=128, seed=59)
    plan = ops.AttentionPlan.from_lists(step.block_table.to(DEV), step.cu_seqlens_q,
                                        step.seqlens_kv, 128, 8, 128, 128)
    torch.cuda.synchronize()
    assert plan.workspace[:64].cpu().view(torch.int32)[6].item() == 63   # units: whole items
    check(step)


def test_prefill_route_repeated_and_deterministic():
    """The prefill kernel has no split: repeated calls on one plan are
    bit-identical, with a decode batch beside it on split-K."""
    step = workloads.make_gqa_step(lqs=[300, 1, 1, 2], lks=[700, 2000, 30, 90], num_q_heads=28,
                                   num_kv_heads=4, block_size=16, seed=8)
    plan = ops.AttentionPlan.from_lists(step.block_table.to(DEV), step.cu_seqlens_q,
                                        step.seqlens_kv, 28, 4, 128, 16)
    q, kc, vc = step.q.to(DEV), step.k_cache.to(DEV), step.v_cache.to(DEV)
    first = ops.paged_attention_gqa(q, kc, vc, plan, step.scale).clone()
    for _ in range(3):
        again = ops.paged_attention_gqa(q, kc, vc, plan, step.scale)
    torch.cuda.synchronize()
    assert torch.equal(first, again)
    assert (first.float().cpu() - oracle(step)).abs().max().item() <= TOL


@pytest.mark.parametrize("lqs,lks,hq,hkv,bs", [
    ([128], [16384], 16, 8, 128),                         # 16 items: 32 chunks each
    ([512], [8192], 28, 4, 128),                          # 112 items: a few chunks each
    ([200, 1, 3], [5000, 300, 40], 32, 8, 16),            # chunks + split-K rows, block 16
    ([64, 64], [64, 3000], 16, 8, 64),                    # one item short, one chunked
])
@pytest.mark.parametrize("d", [128, 64])
def test_prefill_chunked_items(lqs, lks, hq, hkv, bs, d):
    """Too few prefill items to fill the chip: each item's keys are cut into
    balanced chunks whose partials are merged (log-sum-exp) in the merge
    pass; the result matches the oracle and does not depend on the cut
    (head_dim 128 and 64)."""
    step = workloads.make_gqa_step(lqs=lqs, lks=lks, num_q_heads=hq, num_kv_heads=hkv,
                                   head_dim=d, block_size=bs, seed=61)
    check(step)


@pytest.mark.parametrize("hq,hkv", [(16, 8), (28, 4)])
def test_prefill_route_in_a_hip_graph(hq, hkv):
    """The planner, the split-K kernel, the prefill kernel (with chunked
    items) and the merge captured in one HIP graph -- with 4 kv heads the
    prefill units and split-K ranges are one mixed launch: every replay, with
    eager work and synchronisation between replays, equals the eager result,
    and the metadata updated in place between replays is picked up."""
    step = workloads.make_gqa_step(lqs=[128, 1, 2], lks=[6000, 700, 90], num_q_heads=hq,
                                   num_kv_heads=hkv, block_size=64, seed=71)
    q, kc, vc = step.q.to(DEV), step.k_cache.to(DEV), step.v_cache.to(DEV)
    bt = step.block_table.to(DEV)
    cu = torch.tensor([0, *step.cu_seqlens_q], dtype=torch.int32, device=DEV)
    kv = torch.tensor(step.seqlens_kv, dtype=torch.int32, device=DEV)
    T = step.cu_seqlens_q[-1]
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        plan = ops.AttentionPlan(bt, cu, kv, T, hq, hkv, 128, 64)
        eager = ops.paged_attention_gqa(q, kc, vc, plan, step.scale).clone()
        out = torch.empty_like(eager)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            plan.replan()
            ops.paged_attention_gqa(q, kc, vc, plan, step.scale, out=out)
    torch.cuda.synchronize()
    assert (eager.float().cpu() - oracle(step)).abs().max().item() <= TOL
    for _ in range(3):
        out.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
        _ = (q.float() * 2).sum()            # unrelated eager work between replays
    # shorter contexts written into the same metadata tensors: the replayed
    # plan follows them
    kv.copy_(torch.tensor([5000, 600, 80], dtype=torch.int32))
    step.seqlens_kv = [5000, 600, 80]
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    assert (out.float().cpu() - oracle(step)).abs().max().item() <= TOL


def test_prefill_chunk_at_32k_keys():
    """One 512-token chunk behind a 32K-key context (group 7): chunked items,
    many 64-block windows, against the oracle."""
    check(workloads.make_gqa_step(lqs=[512], lks=[32768], num_q_heads=28, num_kv_heads=4,
                                  block_size=128, seed=73))


def test_mixed_launch_with_fused_kv_write():
    """4 kv heads: prefill chunks (routed to prefill units) beside decode and
    verify rows (split-K ranges) in one mixed launch, with this step's new
    K/V rows written by the kernel: caches bit-exact, outputs within TOL."""
    from oracle.paged_attn import kv_write
    step = workloads.make_gqa_step(lqs=[300, 1, 1, 3, 200, 1], lks=[1300, 900, 50, 400, 200, 3000],
                                   num_q_heads=28, num_kv_heads=4, block_size=16, seed=33,
                                   extra_blocks=5)
    kc, vc = step.k_cache.to(DEV), step.v_cache.to(DEV)
    plan = ops.AttentionPlan.from_lists(step.block_table.to(DEV), step.cu_seqlens_q,
                                        step.seqlens_kv, 28, 4, 128, 16)
    out = ops.paged_attention_gqa(step.q.to(DEV), kc, vc, plan, step.scale,
                                  key_new=step.k_new.to(DEV), value_new=step.v_new.to(DEV))
    torch.cuda.synchronize()
    ek, ev = step.k_cache.clone(), step.v_cache.clone()
    kv_write(step.k_new, step.v_new, ek, ev, step.slot_mapping)
    assert torch.equal(kc.cpu(), ek) and torch.equal(vc.cpu(), ev)
    step.k_cache, step.v_cache = ek, ev
    err = (out.float().cpu() - oracle(step)).abs().max().item()
    print(f"max-abs err {err:.3e}", flush=True)
    assert err <= TOL



@pytest.mark.parametrize("hq,hkv", [(40, 2), (24, 1), (52, 2)])
@pytest.mark.parametrize("waves", [7, 64, 0])
def test_group_above_16_not_a_multiple(hq, hkv, waves):
    """Groups of 20, 24 and 26 query heads: the second 16-head block of a kv
    head is part-filled, and split rows past the group must not be merged
    into the next kv head's outputs (the output is pre-filled with a
    sentinel, so a stray write shows).  Decode, verify and a prefill-routed
    request in one step."""
    step = workloads.make_gqa_step(lqs=[1, 3, 1, 2, 40], lks=[700, 90, 1500, 33, 300],
                                   num_q_heads=hq, num_kv_heads=hkv, block_size=16,
                                   seed=hq + waves)
    s = step
    plan = ops.AttentionPlan.from_lists(s.block_table.to(DEV), s.cu_seqlens_q, s.seqlens_kv,
                                        hq, hkv, 128, 16, num_waves=waves)
    out = torch.full(s.q.shape, 7.0, dtype=torch.bfloat16, device=DEV)
    ops.paged_attention_gqa(s.q.to(DEV), s.k_cache.to(DEV), s.v_cache.to(DEV), plan, s.scale,
                            out=out)
    torch.cuda.synchronize()
    err = (out.float().cpu() - oracle(step)).abs().max().item()
    print(f"max-abs err {err:.3e}", flush=True)
    assert err <= TOL, err


@pytest.mark.parametrize("waves", [0, 300])
def test_more_segments_than_the_planner_keeps_in_registers(waves):
    """1100 decode requests of one segment each: past the 1024 segments the
    planner keeps in registers, it reads its segment records back from the
    workspace instead."""
    r = np.random.default_rng(5)
    lks = r.integers(1, 200, size=1100).tolist()
    step = workloads.make_gqa_step(lqs=[1] * 1100, lks=lks, num_q_heads=8, num_kv_heads=1,
                                   block_size=16, seed=5)
    check(step, waves)


@pytest.mark.parametrize("seed", [0, 1])
def test_gqa_plan_ranges_spread_over_the_xcds(seed):
    """Read a config-1 plan back.  The planner writes every range it uses
    into a record slot so that slot b (run by work-group b, dealt to XCD
    b % 8) holds XCD b % 8's next range: every range start appears exactly
    once, each XCD's ranges are consecutive, and the XCDs' counts differ by
    at most one; unused slots hold empty records."""
    step = workloads.config1_decode(seed=seed)
    plan = ops.AttentionPlan.from_lists(step.block_table.to(DEV), step.cu_seqlens_q,
                                        step.seqlens_kv, 16, 8, 128, 128)
    torch.cuda.synchronize()
    ws = plan.workspace.cpu().view(torch.int32)
    hdr = ws[:64].tolist()
    total, tpw, waves = hdr[1], hdr[2], hdr[4]
    rec_off = ops.workspace_layout(16, 16, 16, 8, 128)["wave"]
    recs = ws[rec_off // 4: rec_off // 4 + waves * 32].view(waves, 32)
    nr = -(-total // tpw)
    assert tpw >= 1 and nr <= waves
    starts = {}
    for b in range(waves):
        r = recs[b].tolist()
        if r[0] < 0:
            continue
        assert r[1] % tpw == 0 and r[2] == min(total, r[1] + tpw)
        starts.setdefault(b % 8, []).append(r[1] // tpw)
    got = sorted(i for v in starts.values() for i in v)
    assert got == list(range(nr))
    counts = [len(starts.get(x, [])) for x in range(8)]
    assert max(counts) - min(counts) <= 1
    for x, v in starts.items():
        assert v == list(range(v[0], v[0] + len(v)))


@pytest.mark.parametrize("hq,hkv", [(24, 12), (9, 3), (40, 2), (64, 8)])
@pytest.mark.parametrize("waves", [0, 64, 7])
def test_fixed_slot_merge_decode_steps(hq, hkv, waves):
    """Decode steps small enough for fixed partial slots (header word 10):
    a last kv-head group with fewer waves than the first (12 = 8 + 4 kv
    heads), groups of 3, 20 and 8 query heads, and range counts from 7 to
    the default.  The output is pre-filled with a sentinel, so a row the
    merge misses or a stray write shows."""
    lks = [700, 90, 1500, 33, 1, 2048, 17]
    step = workloads.make_gqa_step(lqs=[1] * len(lks), lks=lks, num_q_heads=hq,
                                   num_kv_heads=hkv, block_size=16, seed=hq + hkv + waves)
    s = step
    plan = ops.AttentionPlan.from_lists(s.block_table.to(DEV), s.cu_seqlens_q, s.seqlens_kv,
                                        hq, hkv, 128, 16, num_waves=waves)
    out = torch.full(s.q.shape, 7.0, dtype=torch.bfloat16, device=DEV)
    ops.paged_attention_gqa(s.q.to(DEV), s.k_cache.to(DEV), s.v_cache.to(DEV), plan, s.scale,
                            out=out)
    torch.cuda.synchronize()
    hdr = plan.workspace[:64].cpu().view(torch.int32)
    err = (out.float().cpu() - oracle(step)).abs().max().item()
    print(f"hq {hq} hkv {hkv} waves {waves}: header {hdr[:11].tolist()}, max-abs err {err:.3e}",
          flush=True)
    assert err <= TOL, err
