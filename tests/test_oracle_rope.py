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


# ------------------------------------------------------------- absorbed MLA

from oracle.pre_attention import ds_rope_interleave, mla_kv_latent, mla_latents_f64, mla_q_latent


def test_ds_rope_interleave_closed_form():
    x = torch.arange(64).float().reshape(1, 64)
    y = ds_rope_interleave(x)[0]
    assert y[:32].tolist() == list(range(0, 64, 2))
    assert y[32:].tolist() == list(range(1, 64, 2))


def _mla_case(T, H, seed):
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(T, H, 192, generator=g) * 2).bfloat16()
    w_uk = (torch.randn(H, 128, 512, generator=g) / 11).bfloat16()
    ckv = (torch.randn(T, 576, generator=g) * 3).bfloat16()
    w = (1 + 0.2 * torch.randn(512, generator=g)).bfloat16()
    return q, w_uk, ckv, w


def test_mla_position_zero_leaves_pe_interleaved_only():
    q, w_uk, ckv, w = _mla_case(3, 2, 1)
    cos, sin = rope_tables([0, 0, 0], 64)
    ql = mla_q_latent(q, w_uk, cos, sin)
    kl = mla_kv_latent(ckv, w, 1e-6, cos, sin)
    assert torch.equal(ql[..., 512:], ds_rope_interleave(q[..., 128:]))
    assert torch.equal(kl[:, 0, 512:], ds_rope_interleave(ckv[:, 512:]))


def test_mla_rope_pairs_keep_norm_and_relative_scores():
    """In float64: each rotated pair (j, 32 + j) of the interleaved pe keeps
    its norm, and the pe score q . k depends on the position difference."""
    q, w_uk, ckv, w = _mla_case(1, 1, 2)
    for p in (0, 5, 1000):
        ql, kl = mla_latents_f64(q, w_uk, ckv, w, 1e-6, [p])
        x = ds_rope_interleave(q[..., 128:].double())
        got = ql[..., 512:]
        assert torch.allclose(got[..., :32] ** 2 + got[..., 32:] ** 2, x[..., :32] ** 2 + x[..., 32:] ** 2)
    s = []
    for pq, pk in ((10, 3), (107, 100), (5007, 5000)):
        ql, _ = mla_latents_f64(q, w_uk, ckv, w, 1e-6, [pq])
        _, kl = mla_latents_f64(q, w_uk, ckv, w, 1e-6, [pk])
        s.append(float((ql[0, 0, 512:] * kl[0, 0, 512:]).sum()))
    assert max(s) - min(s) < 1e-9 * max(1.0, abs(s[0]))


def test_mla_bf16_restatement_tracks_float64():
    """The bf16 restatement is the float64 mathematics up to bf16 rounding:
    the W_UK product within one bf16 ulp (fp32 accumulation, one rounding),
    the norm and RoPE within a few ulps of each row's largest value."""
    T, H = 6, 4
    q, w_uk, ckv, w = _mla_case(T, H, 3)
    pos = [0, 1, 17, 300, 4095, 65000]
    cos, sin = rope_tables(pos, 64)
    ql = mla_q_latent(q, w_uk, cos, sin).double()
    kl = mla_kv_latent(ckv, w, 1e-6, cos, sin).double()
    el, ek = mla_latents_f64(q, w_uk, ckv, w, 1e-6, pos)
    absd = (ql[..., :512] - el[..., :512]).abs()
    assert bool((absd <= el[..., :512].abs() * 2.0 ** -8 + 1e-6).all())
    for got, exp in ((ql[..., 512:], el[..., 512:]), (kl, ek)):
        row = exp.abs().amax(dim=-1, keepdim=True)
        assert bool(((got - exp).abs() <= row * 2.0 ** -6).all())


def test_mla_v_up_is_the_non_absorbed_value_path():
    """Absorbed == non-absorbed for the value side (the identity the
    reference states at mla.py:80-84 and checks in
    scripts/verify_mla_absorb.py:114-141): with attention weights P over the
    latent rows ckv, mla_v_up(P ckv, W_UV) equals P V where V is built the
    non-absorbed way, straight from kv_b_proj: (ckv kv_b^T).view(T, H, nope +
    vd)[..., nope:].  A wrong head index or a transposed W_UV fails it; the
    bf16 restatement is within one bf16 ulp plus fp32 reassociation."""
    from oracle.pre_attention import mla_v_up
    from auto_infer_amd.attention.mla import build_absorb_weights
    g = torch.Generator().manual_seed(9)
    T, H, nope, vd, kvl, L = 5, 3, 128, 128, 512, 7
    kv_b = torch.randn(H * (nope + vd), kvl, generator=g, dtype=torch.float64) / 20
    ckv = torch.randn(L, kvl, generator=g, dtype=torch.float64)
    P = torch.softmax(torch.randn(T, H, L, generator=g, dtype=torch.float64), dim=-1)
    v = (ckv @ kv_b.T).view(L, H, nope + vd)[..., nope:]             # (L, H, vd)
    expect = torch.einsum("thl,lhv->thv", P, v)
    _, w_uv = build_absorb_weights(kv_b, H, nope, vd, kvl)
    o_latent = torch.einsum("thl,lk->thk", P, ckv)                      # (T, H, kvl)
    got = mla_v_up(o_latent, w_uv)
    assert torch.allclose(got, expect, rtol=1e-5, atol=1e-6)     # fp32 sums
    got16 = mla_v_up(o_latent.bfloat16(), w_uv.bfloat16()).double()
    exact = torch.einsum("thl,hvl->thv", o_latent.bfloat16().double(), w_uv.bfloat16().double())
    assert bool(((got16 - exact).abs() <= exact.abs() * 2.0 ** -8 + 1e-6).all())
