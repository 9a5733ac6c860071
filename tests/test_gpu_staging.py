"""GPU stagers against the reference's staging goldens and the numpy
oracle: the reference's dirty-row counts (worker/staging.py:30-48), the
MTP continuation gear (decode_input_stager.py:178-251) and the device
token splice (staging.py:51-70, decode_input_stager.py:125-170)."""
import random

import pytest
import torch

from auto_infer_amd import packing
from auto_infer_amd.execution import DeviceTokenBatch
from oracle import pack
from tests.plans import load, make_plan
from tests.sim import simulate

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _decode_stager(gear, max_blocks, block_size, scratch0):
    return packing.DecodeInputStager(
        tid=torch.zeros(gear, dtype=torch.long, device=DEV),
        positions=torch.zeros(gear, dtype=torch.long, device=DEV),
        slots=torch.zeros(gear, dtype=torch.int32, device=DEV),
        block_table=torch.zeros(gear, max_blocks, dtype=torch.int32, device=DEV),
        block_size=block_size, scratch0=scratch0)


def test_decode_stager_dirty_rows_golden():
    """Unchanged rows are not counted again; a row that turns into padding
    is counted exactly once more (reference test_decode_input_stager.py:
    62-69, 101-110)."""
    fx = load("decode_stager")
    st = fx["stager"]
    stager = _decode_stager(st["gear"], st["max_blocks"], st["block_size"], st["scratch0"])
    for step in fx["dirty_sequence"]:
        before = stager.copied_block_rows
        staged = stager.stage(make_plan(step["requests"], step["scheduled"]))
        torch.cuda.synchronize()
        assert stager.copied_block_rows - before == step["copied_rows"]
        assert stager.copied_block_elements == stager.copied_block_rows * st["max_blocks"]
        if "row1" in step:
            assert staged.block_table[1].cpu().tolist() == step["row1"]


def test_spec_stager_dirty_rows_golden():
    for case in load("spec_decode_stager")["cases"]:
        if "second" not in case:
            continue
        st = case["stager"]
        g, d = st["gear"], st["draft_depth"]
        w = d + 1
        stager = packing.SpecDecodeInputStager(
            tid=torch.zeros(g * w, dtype=torch.long, device=DEV),
            positions=torch.zeros(g * w, dtype=torch.long, device=DEV),
            slots=torch.zeros(g * w, dtype=torch.int32, device=DEV),
            block_table=torch.zeros(g, st["max_blocks"], dtype=torch.int32, device=DEV),
            drafts=torch.zeros(g, d, dtype=torch.long, device=DEV),
            block_size=st["block_size"], scratch0=st["scratch0"], draft_depth=d)
        stager.stage(make_plan(case["requests"], case["scheduled"]))
        before = stager.copied_block_rows
        stager.stage(make_plan(case["second"]["requests"], case["scheduled"]))
        assert stager.copied_block_rows - before == case["second"]["extra_copied_rows"]


def _continuation(st, steps=None):
    g, mb = st["gear"], st["max_blocks"]
    shape = (g,) if steps is None else (steps, g)
    return packing.ContinuationInputStager(
        positions=torch.zeros(shape, dtype=torch.long, device=DEV),
        slots=torch.zeros(shape, dtype=torch.int32, device=DEV),
        block_table=torch.zeros(g, mb, dtype=torch.int32, device=DEV),
        block_size=st["block_size"], scratch0=st["scratch0"])


def test_continuation_stager_golden():
    """Positions, slots, kv lengths and dirty rows of the reference's
    continuation cases (test_decode_input_stager.py:208-269), each step
    also against the oracle restatement."""
    fx = load("continuation_stager")
    st = fx["stager"]
    reuse = fx["reuse"]
    plan = make_plan(reuse["requests"], [["a", 1, False]])
    stager = _continuation(st)
    for step in reuse["steps"]:
        before = stager.copied_block_rows
        got = stager.stage(plan, plan.scheduled, step["accepted"], step["step"])
        exp = pack.continuation_stage(plan, plan.scheduled, step["accepted"], [step["step"]],
                                      **st)
        torch.cuda.synchronize()
        assert got.kv_lengths == step["kv_lengths"] == exp["kv_by_step"][0]
        assert stager.positions.cpu().tolist() == exp["positions"][0].tolist()
        assert stager.slots.cpu().tolist() == exp["slots"][0].tolist()
        assert stager.block_table.cpu().tolist() == exp["block_table"].tolist()
        if "positions" in step:
            assert stager.positions.cpu().tolist() == step["positions"]
            assert stager.slots.cpu().tolist() == step["slots"]
            assert stager.copied_block_rows - before == step["extra_copied_rows"]

    two = fx["two_dirty"]
    stager = _continuation(st)
    first = make_plan(two["first"], [["a", 1, False], ["b", 1, False]])
    stager.stage(first, first.scheduled, two["accepted"], two["step"])
    rows, elems = stager.copied_block_rows, stager.copied_block_elements
    second_req = {rid: dict(r, blocks=two["second_blocks"][rid]) for rid, r in two["first"].items()}
    second = make_plan(second_req, [["a", 1, False], ["b", 1, False]])
    stager.stage(second, second.scheduled, two["accepted"], two["step"])
    torch.cuda.synchronize()
    assert stager.copied_block_rows - rows == two["extra_copied_rows"]
    assert stager.copied_block_elements - elems == two["extra_copied_elements"]
    assert stager.block_table.cpu()[:2, :3].tolist() == [[7, 8, 10], [4, 0, 0]]

    sa = fx["stage_all"]
    plan = make_plan(sa["requests"], [["a", 1, False]])
    stager = _continuation(st, steps=len(sa["steps"]))
    kv = stager.stage_all(plan, plan.scheduled, sa["accepted"])
    torch.cuda.synchronize()
    assert kv == sa["kv_by_step"]
    assert stager.positions.cpu().tolist() == sa["positions"]
    with pytest.raises(ValueError, match="stage_all"):
        stager.stage(plan, plan.scheduled, sa["accepted"], 1)


def test_continuation_rejects_mismatched_gear():
    st = load("continuation_stager")["stager"]
    stager = _continuation(st)
    plan = make_plan(load("continuation_stager")["reuse"]["requests"], [["a", 1, False]])
    with pytest.raises(ValueError, match="does not match graph gear"):
        stager.stage(plan, plan.scheduled, [1, 2], 1)


@pytest.mark.parametrize("steps", [1, 3])
def test_continuation_over_simulated_run(steps):
    """Continuation gears over a simulated run with random accepted counts:
    positions, slots, block table, kv lengths and dirty counts identical to
    the oracle restatement at every step."""
    g, mb, bs, s0 = 12, 16, 16, 4000
    stager = _continuation(dict(gear=g, max_blocks=mb, block_size=bs, scratch0=s0),
                           steps=None if steps == 1 else steps)
    dirty = pack.DirtyRows((g, mb))
    rng = random.Random(steps)
    n = 0
    for plan in simulate(60, seed=11 + steps, block_size=bs, num_blocks=3900, draft_depth=3):
        dec = [s for s in plan.scheduled if not s.is_prefill][:g]
        ok = []
        for s in dec:       # keep rows whose blocks hold every drafted position
            req = plan.get_request(s.request_id)
            if len(plan.block_tables[s.request_id]) * bs > req.num_computed_tokens + 5:
                ok.append(s)
        if not ok:
            continue
        acc = [rng.randint(0, 2) for _ in ok]
        step_ids = [rng.randint(1, 3)] if steps == 1 else list(range(1, steps + 1))
        if steps == 1:
            kv = [stager.stage(plan, ok, acc, step_ids[0]).kv_lengths]
        else:
            kv = stager.stage_all(plan, ok, acc)
        exp = pack.continuation_stage(plan, ok, acc, step_ids, gear=g, max_blocks=mb,
                                      block_size=bs, scratch0=s0, dirty=dirty)
        torch.cuda.synchronize()
        assert kv == exp["kv_by_step"]
        want_pos = exp["positions"] if steps > 1 else exp["positions"][0]
        want_slots = exp["slots"] if steps > 1 else exp["slots"][0]
        assert stager.positions.cpu().tolist() == want_pos.tolist()
        assert stager.slots.cpu().tolist() == want_slots.tolist()
        assert stager.block_table.cpu().tolist() == exp["block_table"].tolist()
        assert stager.copied_block_rows == dirty.rows
        assert stager.copied_block_elements == dirty.elements
        n += 1
    assert n > 20


def test_dirty_counts_over_simulated_runs_match_the_oracle():
    """Decode and prefill gears over simulated runs: the reference's
    copied-row / copied-element counters, step by step."""
    dec = _decode_stager(12, 16, 16, 4000)
    ddirty = pack.DirtyRows((12, 16))
    pst = dict(query_gear=128, sequence_gear=16, max_blocks=16, block_size=16, scratch0=4000)
    pre = packing.PrefillInputStager(
        token_ids=torch.zeros(128, dtype=torch.long, device=DEV),
        positions=torch.zeros(128, dtype=torch.long, device=DEV),
        slots=torch.zeros(128, dtype=torch.int32, device=DEV),
        block_table=torch.zeros(16, 16, dtype=torch.int32, device=DEV),
        sample_rows=torch.zeros(16, dtype=torch.long, device=DEV),
        block_size=16, scratch0=4000)
    pdirty = pack.DirtyRows((16, 16))
    nd = 0
    for plan in simulate(80, seed=21, block_size=16, budget=96, num_blocks=3900):
        d = [s for s in plan.scheduled if not s.is_prefill][:12]
        if d:
            dec.stage(plan, d)
            pack.decode_stage(plan, gear=12, max_blocks=16, block_size=16, scratch0=4000,
                              dirty=ddirty, scheduled=d)
            assert (dec.copied_block_rows, dec.copied_block_elements) == (ddirty.rows,
                                                                           ddirty.elements)
            nd += 1
        pre.stage(plan)
        pack.prefill_stage(plan, dirty=pdirty, **pst)
        assert (pre.copied_block_rows, pre.copied_block_elements) == (pdirty.rows,
                                                                       pdirty.elements)
    assert nd > 20


def _owners(spec):
    return [DeviceTokenBatch.from_output(torch.tensor(o["tokens"], device=DEV), o["order"])
            for o in spec]


@pytest.mark.parametrize("case", load("splice")["stager_cases"], ids=lambda c: c["name"])
def test_stager_splice_golden(case):
    stager = _decode_stager(case["gear"], 4, 4, 100)
    refs = {}
    for o in _owners(case["owners"]):
        refs.update(o.refs())
    prepared = stager.prepare_splice(refs, case["order"])
    stager.apply_splice(prepared)
    torch.cuda.synchronize()
    assert (prepared.fast_owner is not None) == case["expect_fast"]
    n = len(case["expect_prefix"])
    assert stager.tid[:n].cpu().tolist() == case["expect_prefix"]


@pytest.mark.parametrize("case", load("splice")["function_cases"], ids=lambda c: c["name"])
def test_splice_device_tokens_golden(case):
    refs = {}
    for o in _owners(case["owners"]):
        refs.update(o.refs())
    target = torch.zeros(case["target_len"], dtype=torch.long, device=DEV)
    packing.splice_device_tokens(target, case["target_rows"], case["order"], refs)
    torch.cuda.synchronize()
    assert target.cpu().tolist() == case["expect"]


def test_splice_many_owners_one_launch_matches_index_ops():
    """Rows from 20 owners in random order against the index_select /
    index_copy_ form the reference uses, repeated on a prefill stager's
    token buffer (its splice(refs, order, rows) entry)."""
    g = torch.Generator().manual_seed(3)
    owners, order = [], []
    for k in range(20):
        n = int(torch.randint(1, 9, (1,), generator=g))
        rids = [f"o{k}r{i}" for i in range(n)]
        owners.append(DeviceTokenBatch.from_output(
            torch.randint(0, 1 << 40, (n,), generator=g).to(DEV), rids))
        order += rids
    refs = {}
    for o in owners:
        refs.update(o.refs())
    perm = torch.randperm(len(order), generator=g).tolist()
    order = [order[i] for i in perm][:100] + ["missing"]
    st = dict(query_gear=128, sequence_gear=16, max_blocks=4, block_size=16, scratch0=100)
    pre = packing.PrefillInputStager(
        token_ids=torch.full((128,), -1, dtype=torch.long, device=DEV),
        positions=torch.zeros(128, dtype=torch.long, device=DEV),
        slots=torch.zeros(128, dtype=torch.int32, device=DEV),
        block_table=torch.zeros(16, 4, dtype=torch.int32, device=DEV),
        sample_rows=torch.zeros(16, dtype=torch.long, device=DEV),
        block_size=16, scratch0=100)
    rows = torch.randperm(128, generator=g)[:len(order)].tolist()
    want = pre.token_ids.clone()
    for r, rid in zip(rows, order):
        if rid in refs:
            want[r] = refs[rid].owner.tokens[refs[rid].row]
    for _ in range(3):
        pre.splice(refs, order, rows)
    torch.cuda.synchronize()
    assert torch.equal(pre.token_ids, want)
    del st
