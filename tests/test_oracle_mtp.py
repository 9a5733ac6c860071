"""MTP compaction oracle pinned by the reference's confirmed_layout goldens
(tests/test_spec_decode.py:254-285) and by the identity that the compacted
rows are exactly confirmed_layout's source rows."""
import pytest
import torch

from oracle.mtp import confirmed_layout, target_compact


def test_confirmed_layout_goldens():
    # tests/test_spec_decode.py:254-261
    assert confirmed_layout([0, 1, 0, 1], 1) == ((0, 2, 3, 4, 6, 7), (1, 2, 1, 2), (1, 3, 4, 6),
                                                 (0, 2, 3, 5), 6)
    # tests/test_spec_decode.py:264-279
    assert confirmed_layout([0, 0, 0], 1) == ((0, 2, 4), (1, 1, 1), (1, 2, 3), (0, 1, 2), 3)
    assert confirmed_layout([1, 1, 1], 1) == ((0, 1, 2, 3, 4, 5), (2, 2, 2), (2, 4, 6),
                                              (1, 3, 5), 6)
    # tests/test_spec_decode.py:281-285
    with pytest.raises(ValueError, match="between 0 and 1"):
        confirmed_layout([0, 2], 1)


def random_gear(g, depth, active, seed):
    gen = torch.Generator().manual_seed(seed)
    w = depth + 1
    preds = torch.randint(0, 5, (g, w), generator=gen)
    drafts = torch.where(torch.rand(g, depth, generator=gen) < 0.7, preds[:, :-1],
                         torch.randint(0, 5, (g, depth), generator=gen))
    mask = torch.zeros(g, dtype=torch.int64)
    mask[:active] = 1
    hidden = torch.randn(g * w, 24, generator=gen).bfloat16()
    pos = torch.randint(0, 9999, (g * w,), generator=gen)
    slots = torch.randint(0, 9999, (g * w,), generator=gen, dtype=torch.int64).to(torch.int32)
    spos = torch.full((g * w,), -7, dtype=torch.int64)
    sslot = torch.full((g * w,), 12345, dtype=torch.int32)
    return preds, drafts, mask, hidden, pos, slots, spos, sslot


@pytest.mark.parametrize("g,depth,active", [(4, 1, 4), (16, 1, 11), (5, 3, 5), (64, 2, 40),
                                            (3, 1, 0)])
def test_compaction_is_confirmed_layout(g, depth, active):
    args = random_gear(g, depth, active, seed=g * 10 + depth)
    preds, drafts, mask, hidden, pos, slots, spos, sslot = args
    acc, hid, tok, p, sl = target_compact(*args)
    # accepted = leading matches (brute force), zero for inactive requests
    for r in range(g):
        n = 0
        while n < depth and drafts[r, n] == preds[r, n]:
            n += 1
        assert acc[r].item() == (n if r < active else 0)
    src, _, _, _, total = confirmed_layout(acc[:active].tolist(), depth)
    src = torch.tensor(src, dtype=torch.long)
    assert torch.equal(hid[:total], hidden[src])
    assert torch.equal(tok[:total], preds.reshape(-1)[src])
    assert torch.equal(p[:total], pos[src]) and torch.equal(sl[:total], slots[src])
    assert bool((hid[total:] == 0).all()) and bool((tok[total:] == 0).all())
    assert bool((p[total:] == -7).all()) and bool((sl[total:] == 12345).all())
