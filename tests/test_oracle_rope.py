"""Pins the pre-attention oracle (oracle/pre_attention.py) by identities of
the mathematics it restates, checked on the float64 form and by agreement of
the bf16 restatement with it.  No reference vectors exist for these steps:
the reference runs them as NPU ops (npu_rms_norm) and plain torch ops."""
import math

import pytest
import torch

from oracle.pre_attention import (qk_norm_rope, qk_norm_rope_f64, rms_norm, rope_tables,
                                  rotate_half)

HQ, HKV, D = 4, 2, 128


def packed(T, seed=0, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(T, (HQ + 2 * HKV) * D, generator=g) * scale).bfloat16()


def test_rotate_half_closed_form():
    x = torch.arange(8.0)
    assert rotate_half(x).tolist() == [-4.0, -5.0, -6.0, -7.0, 0.0, 1.0, 2.0, 3.0]


def test_position_zero_is_identity():
    """cos = 1, sin = 0 at position 0: q, k unchanged (bf16 path exactly)."""
    qkv = packed(3)
    cos, sin = rope_tables([0, 0, 0], D)
    q, k, v = qkv_ = qk_norm_rope(qkv, HQ, HKV, cos, sin)
    assert torch.equal(q, qkv[:, :HQ * D].reshape(3, HQ, D))
    assert torch.equal(k, qkv[:, HQ * D:(HQ + HKV) * D].reshape(3, HKV, D))
    assert torch.equal(v, qkv[:, (HQ + HKV) * D:].reshape(3, HKV, D))


def test_rope_rotates_pairs_norm_preserving():
    """RoPE rotates each (d, d + 64) pair: pair norms are unchanged (f64)."""
    qkv = packed(5, seed=1)
    pos = [0, 3, 17, 1000, 4095]
    q, k, _ = qk_norm_rope_f64(qkv, HQ, HKV, pos)
    x = qkv.double()[:, :HQ * D].reshape(5, HQ, D)
    n_in = x[..., :64] ** 2 + x[..., 64:] ** 2
    n_out = q[..., :64] ** 2 + q[..., 64:] ** 2
    assert torch.allclose(n_in, n_out, atol=1e-9)


def test_rope_scores_depend_on_relative_position_only():
    """<rope(q, m), rope(k, n)> is a function of m - n (f64)."""
    g = torch.Generator().manual_seed(2)
    qv = torch.randn(1, D, generator=g, dtype=torch.float64)
    kv = torch.randn(1, D, generator=g, dtype=torch.float64)

    def score(m, n):
        row_q = torch.cat([qv, torch.zeros(1, (HQ - 1) * D + 2 * HKV * D, dtype=torch.float64)], 1)
        row_k = torch.cat([torch.zeros(1, HQ * D, dtype=torch.float64), kv,
                           torch.zeros(1, (2 * HKV - 1) * D, dtype=torch.float64)], 1)
        q, _, _ = qk_norm_rope_f64(row_q, HQ, HKV, [m])
        _, k, _ = qk_norm_rope_f64(row_k, HQ, HKV, [n])
        return float((q[0, 0] * k[0, 0]).sum())
    assert math.isclose(score(10, 3), score(107, 100), rel_tol=1e-9)
    assert math.isclose(score(5, 5), score(0, 0), rel_tol=1e-9)
    assert not math.isclose(score(10, 3), score(3, 10), rel_tol=1e-3)


def test_rms_norm_unit_rms_and_scale_invariance():
    g = torch.Generator().manual_seed(3)
    x = torch.randn(6, D, generator=g)
    y = rms_norm(x, torch.ones(D), 0.0)
    assert torch.allclose(y.pow(2).mean(-1), torch.ones(6), atol=1e-5)
    assert torch.allclose(rms_norm(7.5 * x, torch.ones(D), 0.0), y, atol=1e-5)
    w = torch.randn(D, generator=g)
    assert torch.allclose(rms_norm(x, w, 0.0), y * w, atol=1e-5)


@pytest.mark.parametrize("norm", [False, True])
def test_bf16_restatement_tracks_float64(norm):
    """The bf16 op sequence stays within a few bf16 ulps of exact math."""
    T = 7
    qkv = packed(T, seed=4)
    pos = list(range(0, 7 * 300, 300))
    g = torch.Generator().manual_seed(5)
    wq = (1 + 0.1 * torch.randn(D, generator=g)).bfloat16() if norm else None
    wk = (1 + 0.1 * torch.randn(D, generator=g)).bfloat16() if norm else None
    cos, sin = rope_tables(pos, D)
    q, k, v = qk_norm_rope(qkv, HQ, HKV, cos, sin, wq, wk)
    q64, k64, v64 = qk_norm_rope_f64(qkv, HQ, HKV, pos, wq, wk)
    # bf16 tables and results: a few 2^-8 relative steps of values ~N(0, 1)
    for a, b in ((q, q64), (k, k64)):
        err = (a.double() - b).abs().max().item()
        assert err < 0.05, err
        assert (a.double() - b).abs().mean().item() < 0.01
    assert torch.equal(v.double(), v64)
