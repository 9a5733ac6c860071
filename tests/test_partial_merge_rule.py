"""The log-sum-exp rule the merge pass and the prefill units fold partials
with, restated on the CPU (float64), including the per-row scaled form the
prefill units store their partials in: y = O / c, (m + log2 c, l / c) with
c = the row's largest |O|.  Folding the scaled partials gives the same rows
as folding (O, m, l), exactly without rounding and within fp16 rounding of
y, and both equal softmax attention over all the keys."""
import numpy as np
import pytest


def _partials(s, v, cuts):
    """(O, m, l) per key chunk in the log2 domain: m the chunk's row max of
    s * log2(e), l = sum exp2(s' - m), O = sum exp2(s' - m) v."""
    out = []
    for a, b in zip(cuts[:-1], cuts[1:]):
        t = s[:, a:b] * np.log2(np.e)
        m = t.max(axis=1)
        p = np.exp2(t - m[:, None])
        out.append((p @ v[a:b], m, p.sum(axis=1)))
    return out


def _fold(parts):
    """The merge's rule: start empty (m = -1e30), fold part by part."""
    rows, d = parts[0][0].shape
    acc, mx, ls = np.zeros((rows, d)), np.full(rows, -1e30), np.zeros(rows)
    for o, m, l in parts:
        mn = np.maximum(mx, m)
        sa, sb = np.exp2(mx - mn), np.exp2(m - mn)
        acc = acc * sa[:, None] + o * sb[:, None]
        ls = ls * sa + l * sb
        mx = mn
    return acc / ls[:, None]


def _scaled(parts, fp16):
    res = []
    for o, m, l in parts:
        c = np.abs(o).max(axis=1)
        c = np.where(c > 0, c, 1.0)
        y = o / c[:, None]
        if fp16:
            y = y.astype(np.float16).astype(np.float64)
        res.append((y, m + np.log2(c), l / c))
    return res


@pytest.mark.parametrize("nchunks", [2, 3, 7])
def test_scaled_partials_fold_like_plain_ones(nchunks):
    rng = np.random.default_rng(nchunks)
    rows, keys, d = 32, 700, 128
    s = rng.normal(size=(rows, keys)) * 3.0          # a wide spread of scores
    v = rng.normal(size=(keys, d)) * 5.0
    cuts = np.linspace(0, keys, nchunks + 1).astype(int)
    parts = _partials(s, v, cuts)
    p = np.exp(s - s.max(axis=1, keepdims=True))
    want = (p / p.sum(axis=1, keepdims=True)) @ v
    plain = _fold(parts)
    assert np.abs(plain - want).max() < 1e-10
    assert np.abs(_fold(_scaled(parts, fp16=False)) - plain).max() < 1e-10
    # fp16 y: an error of at most about 2^-11 of the row's largest |O| / l
    err = np.abs(_fold(_scaled(parts, fp16=True)) - plain).max()
    assert err < 2.0 ** -10 * np.abs(v).max(), err


def test_a_chunk_that_sees_no_key_of_a_row():
    """A row with no visible key in one chunk has (O, m, l) = (0, -inf, 0);
    scaled with c = 1 it folds to nothing."""
    rng = np.random.default_rng(5)
    s = rng.normal(size=(4, 64))
    v = rng.normal(size=(64, 16))
    parts = _partials(s, v, [0, 32, 64])
    o, m, l = parts[1]
    m[0], l[0], o[0] = -np.inf, 0.0, 0.0              # row 0 sees none of chunk 1
    parts[1] = (o, m, l)
    with np.errstate(invalid="ignore"):
        got = _fold(_scaled(parts, fp16=False))
    p = np.exp(s[0, :32] - s[0, :32].max())
    assert np.allclose(got[0], (p / p.sum()) @ v[:32])
