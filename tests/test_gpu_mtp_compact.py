"""On-device MTP verify compaction vs the oracle restatement of
GraphMtpRunner._target_body (graph_mtp_runner.py:224-248): all outputs
bit-exact (integer and copied bf16 rows)."""
import pytest
import torch

from auto_infer_amd import ops
from oracle.mtp import target_compact
from tests.test_oracle_mtp import random_gear

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


@pytest.mark.parametrize("g,depth,active,hdim", [(4, 1, 4, 24), (16, 1, 11, 4096),
                                                 (5, 3, 5, 1000), (64, 2, 40, 64),
                                                 (3, 1, 0, 16), (64, 1, 64, 7168)])
def test_mtp_compact_vs_oracle(g, depth, active, hdim):
    preds, drafts, mask, hidden, pos, slots, spos, sslot = random_gear(g, depth, active, seed=g + depth)
    hidden = torch.randn(g * (depth + 1), hdim, generator=torch.Generator().manual_seed(1)).bfloat16()
    exp = target_compact(preds, drafts, mask, hidden, pos, slots, spos, sslot)
    got = ops.mtp_compact(preds.to(DEV), drafts.to(DEV), mask.to(DEV), hidden.to(DEV),
                          pos.to(DEV), slots.to(DEV), spos.to(DEV), sslot.to(DEV))
    torch.cuda.synchronize()
    for a, b in zip(got, exp):
        assert torch.equal(a.cpu(), b.to(a.dtype))


def test_mtp_compact_into_fixed_buffers_twice():
    """Fixed output buffers (a graph's) are fully rewritten by each call."""
    g, depth = 8, 1
    bufs = None
    for seed in (3, 4):
        preds, drafts, mask, hidden, pos, slots, spos, sslot = random_gear(g, depth, 6, seed=seed)
        exp = target_compact(preds, drafts, mask, hidden, pos, slots, spos, sslot)
        if bufs is None:
            bufs = dict(accepted=torch.full((g,), -1, dtype=torch.int64, device=DEV),
                        out_hidden=torch.full((g * 2, 24), 9.0, dtype=torch.bfloat16, device=DEV),
                        out_tokens=torch.full((g * 2,), -1, dtype=torch.int64, device=DEV),
                        out_positions=torch.full((g * 2,), -1, dtype=torch.int64, device=DEV),
                        out_slots=torch.full((g * 2,), -1, dtype=torch.int32, device=DEV))
        got = ops.mtp_compact(preds.to(DEV), drafts.to(DEV), mask.to(DEV), hidden.to(DEV),
                              pos.to(DEV), slots.to(DEV), spos.to(DEV), sslot.to(DEV), **bufs)
        torch.cuda.synchronize()
        for a, b in zip(got, exp):
            assert torch.equal(a.cpu(), b.to(a.dtype))
