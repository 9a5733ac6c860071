"""The packer's native per-request host loop (``_hostpack.build_rows``,
auto_infer_amd/csrc/hostpack.cpp) against its Python specification
(``packing.build_rows_py``): identical returned lists, upload queues, row
descriptors and request-table state over simulated continuous-batching
runs (prefill chunks, decode, MTP drafts, requests finishing, slot reuse
and pool growth); and its upload staging (``_hostpack.stage``) against the
numpy specification (``packing._stage_py``).  CPU only: the table lives on
the CPU here."""
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


@pytest.mark.parametrize("by_map", [False, True])
@pytest.mark.parametrize("lazy_live", [False, True])
@pytest.mark.parametrize("depth,seed,slots", [(0, 1, 64), (1, 2, 64), (3, 3, 4), (0, 4, 2)])
def test_native_loop_matches_python(depth, seed, slots, lazy_live, by_map):
    # small tables force LRU slot recycling and pool growth; with lazy_live
    # the native loop builds the step's request-id set itself when a slot
    # is needed; with by_map it reads the plan's request mapping instead of
    # calling get_request (what DeviceBatchPacker.build passes for a BatchPlan)
    tn = packing.DeviceRequestTable("cpu", max_slots=slots, max_blocks=2, max_len=8)
    tp = packing.DeviceRequestTable("cpu", max_slots=slots, max_blocks=2, max_len=8)
    steps = 0
    for plan in simulate(50, seed=seed, block_size=16, draft_depth=depth):
        live = {sr.request_id for sr in plan.scheduled}
        un, up = tn.begin_step(), tp.begin_step()
        lookup = plan.requests if by_map else plan.get_request
        rn = packing._hostpack.build_rows(tn, plan.scheduled, lookup,
                                          plan.block_tables, 16, un, None if lazy_live else live)
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


@pytest.mark.parametrize("seed", range(5))
def test_native_staging_matches_numpy(seed):
    """_hostpack.stage writes the same upload bytes as its numpy
    specification (_stage_py): pool indices slot * width + column, values,
    block ids and the 8-int row descriptors, at the upload layout's offsets."""
    import random

    import numpy as np
    from auto_infer_amd.packing import _ROW_INTS, _stage_py, _Updates
    if packing._hostpack is None:
        pytest.skip("the native extension is not built")
    r = random.Random(seed)
    upd = _Updates()
    for _ in range(r.randint(0, 40)):
        upd.tok_slot.append(r.randint(0, 63))
        upd.tok_idx.append(r.randint(0, 4095))
        upd.tok_val.append(r.randint(0, 2 ** 40))
    for _ in range(r.randint(0, 40)):
        upd.blk_slot.append(r.randint(0, 63))
        upd.blk_idx.append(r.randint(0, 255))
        upd.blk_val.append(r.randint(0, 2 ** 31 - 1))
    for _ in range(r.randint(0, 30)):
        upd.row(*[r.randint(-5, 10 ** 6) for _ in range(_ROW_INTS)])
    nt, nb, nr = len(upd.tok_idx), len(upd.blk_idx), len(upd.rows)
    offs, total = [], 0
    for s in (nt * 8, nt * 8, nb * 8, nb * 4, nr * _ROW_INTS * 4):
        offs.append(total)
        total += (s + 15) & ~15
    a = np.full(total + 16, 0xAB, dtype=np.uint8)
    b = a.copy()
    _stage_py(upd, a, 4096, 256, offs)
    packing._hostpack.stage(upd, b.ctypes.data, 4096, 256, *offs, _ROW_INTS)
    assert np.array_equal(a, b)


def test_native_staging_rejects_bad_input():
    import numpy as np
    from auto_infer_amd.packing import _ROW_INTS, _Updates
    if packing._hostpack is None:
        pytest.skip("the native extension is not built")
    buf = np.zeros(256, dtype=np.uint8)
    upd = _Updates()
    upd.blk_slot.append(0)
    upd.blk_idx.append(0)
    upd.blk_val.append(2 ** 31)
    with pytest.raises(OverflowError):
        packing._hostpack.stage(upd, buf.ctypes.data, 8, 8, 0, 0, 0, 16, 32, _ROW_INTS)
    upd = _Updates()
    upd.rows.append((1, 2, 3))
    with pytest.raises(ValueError, match="row descriptors"):
        packing._hostpack.stage(upd, buf.ctypes.data, 8, 8, 0, 0, 0, 0, 0, _ROW_INTS)
