"""The numpy packing oracle against the reference's literal golden vectors."""
import numpy as np
import pytest

from oracle import pack
from tests.plans import load, make_plan


def test_slot_mapping_closed_form():
    bt = np.array([7, 8, 9])
    pos = np.arange(12)
    got = pack.slot_mapping(bt, pos, 4)
    assert got.tolist() == [28, 29, 30, 31, 32, 33, 34, 35, 36, 37, 38, 39]
    assert pack.slot_mapping(bt, 5, 4) == 33


@pytest.mark.parametrize("case", load("build")["cases"], ids=lambda c: c["name"])
def test_build_golden(case):
    bs = load("build")["block_size"]
    plan = make_plan(case["requests"], case["scheduled"])
    got = pack.build(plan, bs)
    exp = case["expect"]
    assert got["token_ids"].dtype == np.int64 and got["positions"].dtype == np.int64
    assert got["slot_mapping"].dtype == np.int32 and got["block_table"].dtype == np.int32
    for key in ("token_ids", "positions", "slot_mapping", "block_table"):
        if key in exp:
            assert got[key].tolist() == exp[key], key
    for key in ("cu_seqlens_q", "seqlens_kv", "is_decode", "sample_idx"):
        if key in exp:
            assert got[key] == exp[key], key
    if "decode_splice" in exp:
        assert [list(x) for x in got["decode_splice"]] == exp["decode_splice"]


def test_decode_stage_golden():
    fx = load("decode_stager")
    case = fx["cases"][0]
    got = pack.decode_stage(make_plan(case["requests"], case["scheduled"]),
                            **fx["stager"])
    exp = case["expect"]
    assert got["order"] == exp["order"]
    assert got["kv_lengths"] == exp["kv_lengths"]
    assert got["token_ids"].tolist() == exp["token_ids"]
    assert got["positions"].tolist() == exp["positions"]
    assert got["slots"].tolist() == exp["slots"]
    assert got["block_table"].tolist() == exp["block_table"]
    assert got["active_token_mask"].tolist() == exp["active_token_mask"]


def test_decode_stage_dirty_rows_golden():
    fx = load("decode_stager")
    st = fx["stager"]
    dirty = pack.DirtyRows((st["gear"], st["max_blocks"]))
    for step in fx["dirty_sequence"]:
        before = dirty.rows
        got = pack.decode_stage(make_plan(step["requests"], step["scheduled"]),
                                dirty=dirty, **st)
        assert dirty.rows - before == step["copied_rows"]
        if "row1" in step:
            assert got["block_table"][1].tolist() == step["row1"]
            assert got["active_token_mask"].tolist() == step["active_token_mask"]


def test_decode_stage_rejects_overflow():
    fx = load("decode_stager")
    case = fx["cases"][0]
    st = dict(fx["stager"], gear=1)
    with pytest.raises(ValueError, match="exceeds gear"):
        pack.decode_stage(make_plan(case["requests"], case["scheduled"]), **st)


def test_spec_decode_stage_golden():
    fx = load("spec_decode_stager")
    for case in fx["cases"]:
        st = case["stager"]
        dirty = pack.DirtyRows((st["gear"], st["max_blocks"]))
        got = pack.spec_decode_stage(make_plan(case["requests"], case["scheduled"]),
                                     dirty=dirty, **st)
        exp = case["expect"]
        for key in ("token_ids", "positions", "slots", "drafts", "active_mask"):
            if key in exp:
                assert got[key].tolist() == exp[key], key
        for key in ("order", "kv_lengths"):
            if key in exp:
                assert got[key] == exp[key], key
        if "second" in case:
            before = dirty.rows
            pack.spec_decode_stage(make_plan(case["second"]["requests"], case["scheduled"]),
                                   dirty=dirty, **st)
            assert dirty.rows - before == case["second"]["extra_copied_rows"]


def test_spec_decode_stage_rejects_wrong_depth():
    fx = load("spec_decode_stager")
    case = fx["cases"][0]
    st = dict(case["stager"], draft_depth=2)
    with pytest.raises(ValueError, match="expected 2"):
        pack.spec_decode_stage(make_plan(case["requests"], case["scheduled"]), **st)


def test_continuation_stage_golden():
    fx = load("continuation_stager")
    st = fx["stager"]
    reuse = fx["reuse"]
    plan = make_plan(reuse["requests"], [["a", 1, False]])
    dirty = pack.DirtyRows((st["gear"], st["max_blocks"]))
    for step in reuse["steps"]:
        before = dirty.rows
        got = pack.continuation_stage(plan, plan.scheduled, step["accepted"],
                                      [step["step"]], dirty=dirty, **st)
        assert got["kv_by_step"][0] == step["kv_lengths"]
        if "positions" in step:
            assert got["positions"][0].tolist() == step["positions"]
            assert got["slots"][0].tolist() == step["slots"]
            assert dirty.rows - before == step["extra_copied_rows"]

    two = fx["two_dirty"]
    dirty = pack.DirtyRows((st["gear"], st["max_blocks"]))
    first = make_plan(two["first"], [["a", 1, False], ["b", 1, False]])
    pack.continuation_stage(first, first.scheduled, two["accepted"], [two["step"]],
                            dirty=dirty, **st)
    rows, elems = dirty.rows, dirty.elements
    second_req = {rid: dict(r, blocks=two["second_blocks"][rid])
                  for rid, r in two["first"].items()}
    second = make_plan(second_req, [["a", 1, False], ["b", 1, False]])
    pack.continuation_stage(second, second.scheduled, two["accepted"], [two["step"]],
                            dirty=dirty, **st)
    assert dirty.rows - rows == two["extra_copied_rows"]
    assert dirty.elements - elems == two["extra_copied_elements"]

    sa = fx["stage_all"]
    plan = make_plan(sa["requests"], [["a", 1, False]])
    got = pack.continuation_stage(plan, plan.scheduled, sa["accepted"], sa["steps"], **st)
    assert got["kv_by_step"] == sa["kv_by_step"]
    assert got["positions"].tolist() == sa["positions"]


@pytest.mark.parametrize("case", load("prefill_stager")["cases"], ids=lambda c: c["name"])
def test_prefill_stage_golden(case):
    got = pack.prefill_stage(make_plan(case["requests"], case["scheduled"]),
                             **case["stager"])
    exp = case["expect"]
    for key in ("query_tokens", "real_query_tokens", "sequence_count",
                "cumulative_query_lengths", "kv_lengths", "sample_order",
                "splice_order", "splice_rows"):
        if key in exp:
            assert got[key] == exp[key], key
    for key in ("token_ids", "positions", "slots", "sample_rows", "active_token_mask"):
        if key in exp:
            assert got[key].tolist() == exp[key], key
    if "sample_rows_head" in exp:
        n = len(exp["sample_rows_head"])
        assert got["sample_rows"][:n].tolist() == exp["sample_rows_head"]
    if "block_table_rows" in exp:
        assert got["block_table"].shape[0] == exp["block_table_rows"]
    for key, (r, c) in (("bt00", (0, 0)), ("bt10", (1, 0)), ("bt11", (1, 1))):
        if key in exp:
            assert got["block_table"][r, c] == exp[key]
    real = got["real_query_tokens"]
    bs = case["stager"]["block_size"]
    if "padding_slot_min" in exp:
        assert all(s >= exp["padding_slot_min"] for s in got["slots"][real:].tolist())
    if "padding_block_range" in exp:
        lo, hi = exp["padding_block_range"]
        assert all(lo <= s // bs < hi for s in got["slots"][real:].tolist())


def test_prefill_stage_rejects_overflow():
    fx = load("prefill_stager")["overflow"]
    for p in fx["plans"]:
        with pytest.raises(ValueError, match=fx["message"]):
            pack.prefill_stage(make_plan(p["requests"], p["scheduled"]), **fx["stager"])
