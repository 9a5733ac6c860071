"""Absorbed-MLA paged attention on the GPU vs the float32 oracle (2e-2)."""
import pytest
import torch

from auto_infer_amd import ops, workloads
from oracle.paged_attn import kv_write, mla_absorbed_attention

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
TOL = 2e-2


def run(step, num_waves=0):
    plan = ops.AttentionPlan.from_lists(step.block_table.to(DEV), step.cu_seqlens_q,
                                        step.seqlens_kv, step.q_latent.shape[1], 1, 512,
                                        step.cache.shape[1],
                                        num_waves=num_waves)
    out = ops.paged_attention_mla(step.q_latent.to(DEV), step.cache.to(DEV), plan, step.scale)
    torch.cuda.synchronize()
    return out.float().cpu()


def check(step, num_waves=0):
    got = run(step, num_waves)
    exp = mla_absorbed_attention(step.q_latent, step.cache, step.block_table,
                                 step.cu_seqlens_q, step.seqlens_kv, step.scale, 512)
    err = (got - exp).abs().max().item()
    print(f"max-abs err {err:.3e}", flush=True)
    assert err <= TOL, err


def test_mla_config3_shape_small():
    step = workloads.make_mla_step(lqs=[1] * 8, lks=[512, 700, 1, 129, 2000, 33, 8192, 3000],
                                   seed=3)
    check(step)


@pytest.mark.parametrize("waves", [1, 5, 0])
def test_mla_split_invariance(waves):
    step = workloads.make_mla_step(lqs=[1, 1], lks=[900, 77], block_size=16, seed=8)
    check(step, waves)


def test_mla_multi_token_query_causal():
    step = workloads.make_mla_step(lqs=[2, 3, 1], lks=[300, 40, 5], block_size=64, seed=6)
    check(step)


def test_mla_write_then_attend_single_cache():
    """The absorbed path writes one latent row per token into the one cache
    that serves as both K and V (mla.py:111-113), then attends."""
    step = workloads.make_mla_step(lqs=[1] * 4, lks=[10, 200, 130, 1], block_size=128, seed=12)
    cache = step.cache.to(DEV)
    ops.write_kv(step.latent_new.to(DEV), None, cache, None, step.slot_mapping.to(DEV))
    exp_cache = step.cache.clone()
    kv_write(step.latent_new, None, exp_cache, None, step.slot_mapping)
    torch.cuda.synchronize()
    assert torch.equal(cache.cpu(), exp_cache)
    step.cache = exp_cache
    check(step)


@pytest.mark.parametrize("seed", [0, 1])
def test_mla_config2_full_workload(seed):
    """BASELINE configs[2] at full size: 64 requests, query length 1,
    contexts log-uniform in [512, 8192], 16 heads, latent 512 + rope 64,
    block 128, scale 1/sqrt(192) -- the size-dealt balanced plan of the
    default 768 ranges, against the oracle."""
    step = workloads.config3_mla(seed=seed)
    assert len(step.seqlens_kv) == 64 and max(step.seqlens_kv) > 4000
    check(step)


@pytest.mark.parametrize("waves", [256, 512, 1024])
def test_mla_balanced_plan_other_range_counts(waves):
    """Balanced plans at other multiples of the CU count, with context
    lengths whose tile counts do not divide evenly over their ranges."""
    lks = [16 * 37 + 5, 16 * 101 + 1, 16 * 13, 7, 16 * 250 + 9, 16 * 64 - 1] * 6
    step = workloads.make_mla_step(lqs=[1] * len(lks), lks=lks, num_heads=16, block_size=128,
                                   seed=waves)
    check(step, waves)


def _read_plan(plan):
    """(header, segment records, range records) of an MLA decode plan read
    back from its workspace, at the offsets aia_attn_workspace_layout
    gives (header at 0, 8-int segment records, 32-int range records)."""
    ws = plan.workspace.cpu().view(torch.int32)
    hdr = ws[:64].tolist()
    L = ops.workspace_layout(plan.batch, plan.num_tokens, plan.num_q_heads, plan.num_kv_heads,
                             plan.head_dim_v, plan.num_waves)
    seg_off, rec_off = L["seg"], L["wave"]
    nseg = hdr[0]
    seg = ws[seg_off // 4: seg_off // 4 + nseg * 8].view(nseg, 8)
    recs = ws[rec_off // 4: rec_off // 4 + hdr[4] * 32].view(hdr[4], 32)
    return hdr, seg, recs


@pytest.mark.parametrize("seed,waves,balanced", [(0, 0, True), (1, 0, False), (2, 256, True),
                                                  (3, 1024, True)])
def test_mla_plan_covers_every_tile_once(seed, waves, balanced):
    """Read the plan back.  Short ranges (< 16 tiles) give a padded plan
    whose ranges are size-dealt: every key tile of every request is covered
    by exactly one range, a request's k ranges are numbered 0..k-1 and
    differ in size by at most one tile, and the number of ranges used
    matches the header.  Longer ranges (configs[2] seed 1) keep the even
    split of the concatenated tiles: range w covers tiles [w tpw, (w + 1)
    tpw) and together they cover every segment's tiles."""
    if seed < 2:
        step = workloads.config3_mla(seed=seed)
    else:     # short enough ranges (< 16 tiles) for a padded, hence balanced, plan
        top = 1800 if waves == 256 else 9000
        lks = torch.randint(1, top, (48,), generator=torch.Generator().manual_seed(seed)).tolist()
        step = workloads.make_mla_step(lqs=[1] * 48, lks=lks, num_heads=16, block_size=128,
                                       seed=seed)
    plan = ops.AttentionPlan.from_lists(step.block_table.to(DEV), step.cu_seqlens_q,
                                        step.seqlens_kv, 16, 1, 512, 128, num_waves=waves)
    torch.cuda.synchronize()
    hdr, seg, recs = _read_plan(plan)
    assert hdr[8] == 0
    nseg, total, tpw, nwaves = hdr[0], hdr[1], hdr[2], hdr[4]
    assert nseg == len(step.seqlens_kv)
    for s in range(nseg):
        assert int(seg[s, 6] - seg[s, 5]) == max(1, -(-step.seqlens_kv[s] // 16))
    used = recs[recs[:, 0] >= 0]
    assert bool((used[:, 15] >= 1).all()) == balanced
    if not balanced:
        assert used.shape[0] == -(-total // tpw) <= nwaves
        assert used[:, 1].tolist() == list(range(0, total, tpw))
        assert used[:, 2].tolist() == [min(total, t + tpw) for t in range(0, total, tpw)]
        assert int(seg[0, 5]) == 0 and int(seg[nseg - 1, 6]) == total
        assert all(int(seg[s, 6]) == int(seg[s + 1, 5]) for s in range(nseg - 1))
        return
    assert used.shape[0] == hdr[3] <= nwaves
    per_seg = {}
    for r in used.tolist():
        per_seg.setdefault(r[0], []).append((r[1], r[2], r[14], r[15]))
    assert sorted(per_seg) == list(range(nseg))
    for s, rs in per_seg.items():
        tb, te = int(seg[s, 5]), int(seg[s, 6])
        rs.sort()
        k = len(rs)
        assert [r[2] for r in rs] == list(range(k)) and all(r[3] == k for r in rs)
        assert rs[0][0] == tb and rs[-1][1] == te
        assert all(rs[i][1] == rs[i + 1][0] for i in range(k - 1))
        sizes = [r[1] - r[0] for r in rs]
        assert max(sizes) - min(sizes) <= 1 and min(sizes) >= 1


def test_planner_status_reports_overflow():
    """Query lengths that do not add up to the step's token count: the
    planner plans nothing and says so in its status word."""
    bt = torch.arange(8, dtype=torch.int32, device=DEV).view(2, 4)
    cu = torch.tensor([0, 5, 100], dtype=torch.int32, device=DEV)
    kv = torch.tensor([5, 100], dtype=torch.int32, device=DEV)
    plan = ops.AttentionPlan(bt, cu, kv, 10, 8, 2, 128, 64)
    with pytest.raises(ValueError, match="overflow"):
        plan.status()
    ok = ops.AttentionPlan(bt, cu, kv, 100, 8, 2, 128, 64)
    ok.status()


def test_caller_outputs_are_checked():
    """A caller-supplied ``out`` of the wrong dtype, shape or device raises
    ValueError before any launch."""
    step = workloads.make_mla_step(lqs=[1, 1], lks=[40, 9], block_size=16, seed=4)
    plan = ops.AttentionPlan.from_lists(step.block_table.to(DEV), step.cu_seqlens_q,
                                        step.seqlens_kv, 16, 1, 512, 16)
    q, cache = step.q_latent.to(DEV), step.cache.to(DEV)
    for bad in (torch.empty(2, 16, 512, dtype=torch.float32, device=DEV),
                torch.empty(2, 16, 256, dtype=torch.bfloat16, device=DEV),
                torch.empty(2, 16, 512, dtype=torch.bfloat16)):
        with pytest.raises(ValueError):
            ops.paged_attention_mla(q, cache, plan, step.scale, out=bad)
    g = workloads.make_gqa_step(lqs=[1], lks=[30], num_q_heads=8, num_kv_heads=2, block_size=16,
                                seed=2)
    gp = ops.AttentionPlan.from_lists(g.block_table.to(DEV), g.cu_seqlens_q, g.seqlens_kv, 8, 2,
                                      128, 16)
    with pytest.raises(ValueError):
        ops.paged_attention_gqa(g.q.to(DEV), g.k_cache.to(DEV), g.v_cache.to(DEV), gp, g.scale,
                                out=torch.empty(1, 8, 64, dtype=torch.bfloat16, device=DEV))


def test_mla_more_segments_than_the_planner_keeps_in_registers():
    """1100 requests of one segment each (past the planner's 1024 in
    registers) through the size-dealt MLA plan."""
    lks = torch.randint(1, 300, (1100,), generator=torch.Generator().manual_seed(9)).tolist()
    step = workloads.make_mla_step(lqs=[1] * 1100, lks=lks, num_heads=16, block_size=64, seed=9)
    check(step)


@pytest.mark.parametrize("waves", [5, 0])
def test_mla_twenty_heads(waves):
    """20 heads: the second 16-head block is part-filled; split rows past
    the head count are neither merged nor written."""
    step = workloads.make_mla_step(lqs=[1, 1, 2], lks=[3000, 200, 900], num_heads=20,
                                   block_size=64, seed=20 + waves)
    check(step, waves)


# MLA prefill-sized steps (two row blocks per segment from 2048 query rows,
# tokens x heads, with more tokens than requests): long chunks, forced
# splits, ragged batches with a decode row, 20 heads.
@pytest.mark.parametrize("lqs,lks,heads,bs,waves", [
    ([100, 60], [100 + 700, 60 + 33], 16, 64, 0),
    ([512], [1536], 16, 128, 0),
    ([512], [1536], 16, 128, 37),
    ([300, 1, 200, 37], [800, 900, 200, 1037], 16, 64, 0),
    ([420], [420 + 77], 20, 16, 0),
])
def test_mla_prefill_row_blocks(lqs, lks, heads, bs, waves):
    print(f"mla prefill lqs={lqs} lks={lks} heads={heads} bs={bs} waves={waves}", flush=True)
    step = workloads.make_mla_step(lqs=lqs, lks=lks, num_heads=heads, block_size=bs, seed=31)
    check(step, waves)


# MLA prefill units (requests of 8+ tokens, 4+ tokens per request on
# average): 128-row items in two 64-row passes, 32-key sub-tiles in a ring
# of four LDS buffers.  Cases: units cut into key chunks (partials and the
# chunk merge), one request against 16K keys, a block size of 4 with more
# than 2048 blocks under one unit (the staged block ids are replaced
# mid-unit), units beside split-K rows, and scores spread so wide that a
# row exceeds its reference max by 2^64 (the unit runs its tiles again).
@pytest.mark.parametrize("lqs,lks,bs,heads", [
    ([64] * 8, [4096] * 8, 128, 16),
    ([512], [16384], 128, 16),
    ([64], [12000], 4, 16),
    ([40, 1, 1, 9, 24], [2000, 300, 5000, 9, 24 + 700], 16, 16),
    ([16] * 6, [((i * 777) % 3000) + 16 for i in range(6)], 64, 32),
])
def test_mla_prefill_units(lqs, lks, bs, heads):
    print(f"mla prefill units lqs={lqs[:5]} lks={lks[:5]} bs={bs} heads={heads}", flush=True)
    step = workloads.make_mla_step(lqs=lqs, lks=lks, num_heads=heads, block_size=bs, seed=41)
    check(step)


def test_mla_prefill_unit_reruns_with_exact_row_maxima():
    step = workloads.make_mla_step(lqs=[96, 40], lks=[1500, 40 + 900], block_size=64, seed=43)
    step.q_latent = (step.q_latent.float() * 40).to(torch.bfloat16)
    print("mla prefill units with scores spread past 2^64", flush=True)
    check(step)
