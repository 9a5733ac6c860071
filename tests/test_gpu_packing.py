"""GPU packing kernel vs the numpy packing oracle: bit-exact metadata."""
import numpy as np
import pytest
import torch

from auto_infer_amd import packing
from oracle import pack
from tests.plans import load, make_plan
from tests.sim import simulate

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _eq(t, ref, name):
    got = t.cpu().numpy() if isinstance(t, torch.Tensor) else np.asarray(t)
    assert got.dtype == np.asarray(ref).dtype or name in ("cu", "kv"), (name, got.dtype)
    assert np.array_equal(got, np.asarray(ref)), f"{name}: {got} != {ref}"


def check_build(packer, plan, bs):
    ctx, sample_idx, splice = packer.build(plan)
    exp = pack.build(plan, bs)
    torch.cuda.synchronize()
    _eq(ctx.token_ids, exp["token_ids"], "token_ids")
    _eq(ctx.positions, exp["positions"], "positions")
    _eq(ctx.slot_mapping, exp["slot_mapping"], "slot_mapping")
    _eq(ctx.block_table, exp["block_table"], "block_table")
    assert ctx.cu_seqlens_q == exp["cu_seqlens_q"]
    assert ctx.seqlens_kv == exp["seqlens_kv"]
    assert ctx.is_decode == exp["is_decode"]
    assert sample_idx == exp["sample_idx"]
    assert splice == exp["decode_splice"]
    assert ctx.aia_cu_seqlens_q.cpu().tolist() == [0] + exp["cu_seqlens_q"]
    assert ctx.aia_seqlens_kv.cpu().tolist() == exp["seqlens_kv"]


@pytest.mark.parametrize("case", load("build")["cases"], ids=lambda c: c["name"])
def test_build_golden(case):
    bs = load("build")["block_size"]
    packer = packing.DeviceBatchPacker(bs, DEV, max_num_batched_tokens=4, max_num_seqs=1,
                                       max_blocks=1)      # tiny caps: exercise growth
    check_build(packer, make_plan(case["requests"], case["scheduled"]), bs)


@pytest.mark.parametrize("seed,depth", [(0, 0), (1, 0), (2, 1), (3, 3)])
def test_build_over_a_simulated_run(seed, depth):
    """Many steps through one packer: incremental device state stays exact
    (new blocks, new tokens, drafts, finished requests, slot reuse)."""
    table = packing.DeviceRequestTable(DEV, max_slots=4, max_blocks=2, max_len=8)
    packer = packing.DeviceBatchPacker(16, DEV, table=table)
    n = 0
    for plan in simulate(60, seed=seed, block_size=16, draft_depth=depth):
        check_build(packer, plan, 16)
        n += 1
    assert n > 30


def _decode_stager(gear=4, max_blocks=4, bs=4, scratch0=100, mask=False):
    return packing.DecodeInputStager(
        tid=torch.zeros(gear, dtype=torch.long, device=DEV),
        positions=torch.zeros(gear, dtype=torch.long, device=DEV),
        slots=torch.zeros(gear, dtype=torch.int32, device=DEV),
        block_table=torch.zeros(gear, max_blocks, dtype=torch.int32, device=DEV),
        active_token_mask=torch.zeros(gear, dtype=torch.bool, device=DEV) if mask else None,
        block_size=bs, scratch0=scratch0)


def test_decode_stager_golden_and_fixed_addresses():
    fx = load("decode_stager")
    st = fx["stager"]
    stager = _decode_stager(st["gear"], st["max_blocks"], st["block_size"], st["scratch0"],
                            mask=True)
    ptrs = None
    for step in fx["dirty_sequence"]:
        plan = make_plan(step["requests"], step["scheduled"])
        staged = stager.stage(plan)
        exp = pack.decode_stage(plan, **st)
        torch.cuda.synchronize()
        _eq(staged.token_ids, exp["token_ids"], "tid")
        _eq(staged.positions, exp["positions"], "pos")
        _eq(staged.slots, exp["slots"], "slots")
        _eq(staged.block_table, exp["block_table"], "bt")
        _eq(stager.active_token_mask, exp["active_token_mask"], "mask")
        assert staged.kv_lengths == exp["kv_lengths"] and staged.order == exp["order"]
        assert staged.seqlens_kv.cpu().tolist() == exp["kv_lengths"]
        ptrs = ptrs or staged.data_ptrs()
        assert staged.data_ptrs() == ptrs
    exp0 = fx["cases"][0]["expect"]
    plan = make_plan(fx["cases"][0]["requests"], fx["cases"][0]["scheduled"])
    staged = stager.stage(plan)
    torch.cuda.synchronize()
    assert staged.slots.cpu().tolist() == exp0["slots"]
    assert staged.block_table.cpu().tolist() == exp0["block_table"]


def test_decode_stager_rejects_overflow():
    fx = load("decode_stager")
    case = fx["cases"][0]
    stager = _decode_stager(gear=1)
    with pytest.raises(ValueError, match="exceeds gear"):
        stager.stage(make_plan(case["requests"], case["scheduled"]))


@pytest.mark.parametrize("ci", [0, 1])
def test_spec_stager_golden(ci):
    case = load("spec_decode_stager")["cases"][ci]
    st = case["stager"]
    g, w, d = st["gear"], st["draft_depth"] + 1, st["draft_depth"]
    active = torch.zeros(g, dtype=torch.int32, device=DEV)
    stager = packing.SpecDecodeInputStager(
        tid=torch.zeros(g * w, dtype=torch.long, device=DEV),
        positions=torch.zeros(g * w, dtype=torch.long, device=DEV),
        slots=torch.zeros(g * w, dtype=torch.int32, device=DEV),
        block_table=torch.zeros(g, st["max_blocks"], dtype=torch.int32, device=DEV),
        drafts=torch.zeros(g, d, dtype=torch.long, device=DEV), active_mask=active,
        block_size=st["block_size"], scratch0=st["scratch0"], draft_depth=d)
    plans = [make_plan(case["requests"], case["scheduled"])]
    if "second" in case:
        plans.append(make_plan(case["second"]["requests"], case["scheduled"]))
    for plan in plans:
        staged = stager.stage(plan)
        exp = pack.spec_decode_stage(plan, **st)
        torch.cuda.synchronize()
        _eq(staged.token_ids, exp["token_ids"], "tid")
        _eq(staged.positions, exp["positions"], "pos")
        _eq(staged.slots, exp["slots"], "slots")
        _eq(staged.block_table, exp["block_table"], "bt")
        _eq(stager.drafts, exp["drafts"], "drafts")
        _eq(active, exp["active_mask"], "active")
        assert staged.kv_lengths == exp["kv_lengths"]


def test_spec_stager_over_simulated_run():
    g, d = 12, 2
    w = d + 1
    stager = packing.SpecDecodeInputStager(
        tid=torch.zeros(g * w, dtype=torch.long, device=DEV),
        positions=torch.zeros(g * w, dtype=torch.long, device=DEV),
        slots=torch.zeros(g * w, dtype=torch.int32, device=DEV),
        block_table=torch.zeros(g, 16, dtype=torch.int32, device=DEV),
        drafts=torch.zeros(g, d, dtype=torch.long, device=DEV),
        block_size=16, scratch0=4000, draft_depth=d)
    n = 0
    for plan in simulate(80, seed=5, block_size=16, draft_depth=d, num_blocks=3900):
        decode = [s for s in plan.scheduled if not s.is_prefill]
        if not decode:
            continue
        staged = stager.stage(plan, decode)
        exp = pack.spec_decode_stage(plan, gear=g, max_blocks=16, block_size=16, scratch0=4000,
                                     draft_depth=d, scheduled=decode)
        torch.cuda.synchronize()
        _eq(staged.token_ids, exp["token_ids"], "tid")
        _eq(staged.slots, exp["slots"], "slots")
        _eq(staged.block_table, exp["block_table"], "bt")
        assert staged.kv_lengths == exp["kv_lengths"]
        n += 1
    assert n > 20


def _prefill_stager(st, mask=False):
    qg, sg, mb = st["query_gear"], st["sequence_gear"], st["max_blocks"]
    return packing.PrefillInputStager(
        token_ids=torch.zeros(qg, dtype=torch.long, device=DEV),
        positions=torch.zeros(qg, dtype=torch.long, device=DEV),
        slots=torch.zeros(qg, dtype=torch.int32, device=DEV),
        block_table=torch.zeros(sg, mb, dtype=torch.int32, device=DEV),
        sample_rows=torch.zeros(sg, dtype=torch.long, device=DEV),
        active_token_mask=torch.zeros(qg, dtype=torch.bool, device=DEV) if mask else None,
        block_size=st["block_size"], scratch0=st["scratch0"])


@pytest.mark.parametrize("case", load("prefill_stager")["cases"], ids=lambda c: c["name"])
def test_prefill_stager_golden(case):
    stager = _prefill_stager(case["stager"], mask=True)
    plan = make_plan(case["requests"], case["scheduled"])
    staged = stager.stage(plan)
    exp = pack.prefill_stage(plan, **case["stager"])
    torch.cuda.synchronize()
    _eq(staged.token_ids, exp["token_ids"], "tid")
    _eq(staged.positions, exp["positions"], "pos")
    _eq(staged.slots, exp["slots"], "slots")
    _eq(staged.block_table, exp["block_table"], "bt")
    _eq(staged.sample_rows, exp["sample_rows"], "sample_rows")
    _eq(stager.active_token_mask, exp["active_token_mask"], "mask")
    for key in ("cumulative_query_lengths", "kv_lengths", "sample_order", "splice_order",
                "splice_rows", "query_tokens", "real_query_tokens", "sequence_count"):
        assert getattr(staged, key) == exp[key], key


def test_prefill_stager_rejects_overflow():
    fx = load("prefill_stager")["overflow"]
    stager = _prefill_stager(fx["stager"])
    for p in fx["plans"]:
        with pytest.raises(ValueError, match=fx["message"]):
            stager.stage(make_plan(p["requests"], p["scheduled"]))


def test_prefill_stager_over_simulated_run():
    st = dict(query_gear=128, sequence_gear=16, max_blocks=16, block_size=16, scratch0=4000)
    stager = _prefill_stager(st)
    n = 0
    for plan in simulate(60, seed=9, block_size=16, budget=96, num_blocks=3900):
        staged = stager.stage(plan)
        exp = pack.prefill_stage(plan, **st)
        torch.cuda.synchronize()
        _eq(staged.token_ids, exp["token_ids"], "tid")
        _eq(staged.slots, exp["slots"], "slots")
        _eq(staged.block_table, exp["block_table"], "bt")
        _eq(staged.sample_rows, exp["sample_rows"], "sample_rows")
        assert staged.cumulative_query_lengths == exp["cumulative_query_lengths"]
        assert staged.kv_lengths == exp["kv_lengths"]
        n += 1
    assert n > 30


@pytest.mark.parametrize("inline", [True, False])
def test_build_inline_and_staged_uploads_agree(inline, monkeypatch):
    """Small steps go out inline (aia_pack_rows_inline: updates and rows in
    the launch's arguments), larger ones through the staging copy
    (aia_pack_rows); a simulated run through either path matches the
    oracle step by step."""
    if not inline:
        monkeypatch.setattr(packing, "_USE_INLINE", False)
    table = packing.DeviceRequestTable(DEV, max_slots=4, max_blocks=2, max_len=8)
    packer = packing.DeviceBatchPacker(16, DEV, table=table)
    n = 0
    for plan in simulate(40, seed=7, block_size=16, draft_depth=1):
        check_build(packer, plan, 16)
        n += 1
    assert n > 20


@pytest.mark.parametrize("batch", [16, 44, 90])
def test_build_of_each_inline_argument_size(batch):
    """Decode steps of 16, 44 and 90 requests growing one token a step: in
    steady state their rows (32 B each) and new token ids (16 B each) take
    the 1 KB inline argument block, the 3 KB one, and (90 requests) the
    staging copy.  Every step matches the oracle."""
    from auto_infer_amd.execution import BatchPlan, RequestView, ScheduledRequest
    rng = np.random.default_rng(batch)
    bs = 16
    lens = rng.integers(5, 40, size=batch).tolist()
    perm = rng.permutation(4 * batch).tolist()
    packer = packing.DeviceBatchPacker(bs, DEV)
    for k in range(4):
        views, tables, sched = {}, {}, []
        for i, lk in enumerate(lens):
            lk += k
            rid = f"q{i}"
            tables[rid] = tuple(perm[4 * i: 4 * i + (lk + bs - 1) // bs])
            views[rid] = RequestView(rid, tuple(range(100 + i, 100 + i + lk)), lk - 1, 1, 1, ())
            sched.append(ScheduledRequest(rid, 1, False, tables[rid]))
        check_build(packer, BatchPlan.make(sched, views, tables), bs)
