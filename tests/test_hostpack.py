"""The packer's native per-request host loop (``_hostpack.build_rows``,
auto_infer_amd/csrc/hostpack.cpp) against its Python specification
(``packing.build_rows_py``): identical returned lists, upload queues, row
descriptors and request-table state over simulated continuous-batching
runs (prefill chunks, decode, MTP drafts, requests finishing, slot reuse
and pool growth).  CPU only: the table lives on the CPU here."""
import pytest

from auto_infer_amd import packing
from tests.sim import simulate

pytestmark = pytest.mark.skipif(packing._hostpack is None, reason="_hostpack not built")


def table_state(t):
    return (dict(t._slot), dict(t._blocks), dict(t._ntok), dict(t._last_use), list(t._free),
            t._step, t.uploaded_block_rows, t.uploaded_block_elements, t._cap_blocks,
            t._cap_tokens, tuple(t.block_pool.shape), tuple(t.token_pool.shape))


def upd_state(u):
    return (u.rows, u.tok_slot, u.tok_idx, u.tok_val, u.blk_slot, u.blk_idx, u.blk_val)


@pytest.mark.parametrize("depth,seed,slots", [(0, 1, 64), (1, 2, 64), (3, 3, 4), (0, 4, 2)])
def test_native_loop_matches_python(depth, seed, slots):
    # small tables force LRU slot recycling and pool growth
    tn = packing.DeviceRequestTable("cpu", max_slots=slots, max_blocks=2, max_len=8)
    tp = packing.DeviceRequestTable("cpu", max_slots=slots, max_blocks=2, max_len=8)
    steps = 0
    for plan in simulate(50, seed=seed, block_size=16, draft_depth=depth):
        live = {sr.request_id for sr in plan.scheduled}
        un, up = tn.begin_step(), tp.begin_step()
        rn = packing._hostpack.build_rows(tn, plan.scheduled, plan.get_request,
                                          plan.block_tables, 16, un, live)
        rp = packing.build_rows_py(tp, plan.scheduled, plan.get_request, plan.block_tables, 16,
                                   up, live)
        assert rn == rp
        assert upd_state(un) == upd_state(up)
        assert table_state(tn) == table_state(tp)
        steps += 1
    assert steps > 20


def test_native_loop_raises_like_python():
    from auto_infer_amd.execution import BatchPlan, RequestView, ScheduledRequest
    plan = BatchPlan.make([ScheduledRequest("a", 5, True, (0,))],
                          {"a": RequestView("a", tuple(range(20)), 0, 20, 20, ())}, {"a": (7,)})
    t = packing.DeviceRequestTable("cpu")
    with pytest.raises(ValueError, match="request a: 1 blocks cannot hold position 4"):
        packing._hostpack.build_rows(t, plan.scheduled, plan.get_request, plan.block_tables, 4,
                                     t.begin_step(), {"a"})
    with pytest.raises(ValueError, match="request a: 1 blocks cannot hold position 4"):
        packing.build_rows_py(t, plan.scheduled, plan.get_request, plan.block_tables, 4,
                              t.begin_step(), {"a"})
