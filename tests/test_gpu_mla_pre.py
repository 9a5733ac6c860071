"""Absorbed-MLA pre-attention kernels (latent query, latent KV row) and the
W_UV value up-projection vs the bf16 torch restatement in
oracle/pre_attention.py.

Bars: the RoPE parts are bit-exact (the kernels round where the torch ops
round).  The normed latent is within one bf16 ulp of the row's largest value
(the fp32 sum of squares is added in another order) and bit-exact on at least
99% of values.  The W_UK product accumulates in fp32 and rounds once, as the
bf16 GEMM of the restatement does, so it is within one ulp of each value
(plus fp32 reassociation, far below that) and bit-exact on at least 99%.
"""
import pytest
import torch

from auto_infer_amd import ops
from oracle.pre_attention import mla_kv_latent, mla_q_latent, mla_v_up, rope_tables

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def case(T, H, seed, pos_hi=40000):
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(T, H, 192, generator=g) * 2).bfloat16()
    w_uk = (torch.randn(H, 128, 512, generator=g) / 11).bfloat16()
    ckv = (torch.randn(T, 576, generator=g) * 3).bfloat16()
    w = (1 + 0.2 * torch.randn(512, generator=g)).bfloat16()
    pos = torch.randint(0, pos_hi, (T,), generator=g)
    cos, sin = rope_tables(pos, 64)
    return q, w_uk, ckv, w, cos, sin


def close_to_one_ulp(got, exp, row_relative):
    diff = (got.float() - exp.float()).abs()
    if row_relative:
        bound = exp.float().abs().amax(dim=-1, keepdim=True) * 2.0 ** -7
    else:
        bound = exp.float().abs() * 2.0 ** -7 + 1e-6
    assert bool((diff <= bound).all()), diff.max().item()
    same = (got == exp).float().mean().item()
    print(f"bit-exact fraction {same:.5f}", flush=True)
    assert same >= 0.99


@pytest.mark.parametrize("T,H", [(1, 16), (7, 16), (64, 16), (33, 128), (300, 4)])
def test_q_latent_vs_oracle(T, H):
    q, w_uk, _, _, cos, sin = case(T, H, seed=T + H)
    got = ops.mla_q_latent(q.to(DEV), w_uk.transpose(1, 2).contiguous().to(DEV), cos.to(DEV),
                           sin.to(DEV)).cpu()
    exp = mla_q_latent(q, w_uk, cos, sin)
    assert torch.equal(got[..., 512:], exp[..., 512:])
    close_to_one_ulp(got[..., :512], exp[..., :512], row_relative=False)


@pytest.mark.parametrize("T", [1, 5, 64, 2049])
def test_kv_latent_vs_oracle(T):
    _, _, ckv, w, cos, sin = case(T, 1, seed=T)
    got = ops.mla_kv_latent(ckv.to(DEV), w.to(DEV), 1e-6, cos.to(DEV), sin.to(DEV)).cpu()
    exp = mla_kv_latent(ckv, w, 1e-6, cos, sin)
    assert got.shape == exp.shape == (T, 1, 576)
    assert torch.equal(got[..., 512:], exp[..., 512:])
    close_to_one_ulp(got[..., :512], exp[..., :512], row_relative=True)


def test_strided_inputs():
    """q as a view of a wider projection, ckv rows inside wider rows and
    cos/sin as views of wider tables give the same results."""
    T, H = 9, 8
    q, w_uk, ckv, w, cos, sin = case(T, H, seed=4)
    wide_q = torch.zeros(T, H, 200, dtype=torch.bfloat16)
    wide_q[..., :192] = q
    wide_ckv = torch.zeros(T, 640, dtype=torch.bfloat16)
    wide_ckv[:, :576] = ckv
    wide_c = torch.zeros(T, 1, 128, dtype=torch.bfloat16)
    wide_s = torch.zeros(T, 1, 128, dtype=torch.bfloat16)
    wide_c[..., :64] = cos
    wide_s[..., :64] = sin
    c, s = wide_c.to(DEV)[..., :64], wide_s.to(DEV)[..., :64]
    wt = w_uk.transpose(1, 2).contiguous().to(DEV)
    a = ops.mla_q_latent(wide_q.to(DEV)[..., :192], wt, c, s).cpu()
    b = ops.mla_q_latent(q.to(DEV), wt, cos.to(DEV), sin.to(DEV)).cpu()
    assert torch.equal(a, b)
    a = ops.mla_kv_latent(wide_ckv.to(DEV)[:, :576], w.to(DEV), 1e-6, c, s).cpu()
    b = ops.mla_kv_latent(ckv.to(DEV), w.to(DEV), 1e-6, cos.to(DEV), sin.to(DEV)).cpu()
    assert torch.equal(a, b)


def test_rejects_bad_shapes():
    q = torch.zeros(4, 16, 192, dtype=torch.bfloat16, device=DEV)
    cos = torch.zeros(4, 1, 64, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(ValueError, match="w_uk_t"):
        ops.mla_q_latent(q, torch.zeros(16, 128, 512, dtype=torch.bfloat16, device=DEV), cos, cos)
    with pytest.raises(ValueError, match="ckv_full"):
        ops.mla_kv_latent(torch.zeros(4, 512, dtype=torch.bfloat16, device=DEV),
                          torch.zeros(512, dtype=torch.bfloat16, device=DEV), 1e-6, cos, cos)


@pytest.mark.parametrize("T,H", [(1, 16), (7, 16), (64, 16), (65, 16), (300, 4), (200, 128),
                                 (2049, 16)])
def test_v_up_vs_oracle(T, H):
    """Decode / verify sizes and, beyond the rows the backend routes to it,
    long steps, with ragged last token tiles."""
    g = torch.Generator().manual_seed(T * 7 + H)
    o = (torch.randn(T, H, 512, generator=g) / 4).bfloat16()
    w_uv = (torch.randn(H, 128, 512, generator=g) / 11).bfloat16()
    got = ops.mla_v_up(o.to(DEV), w_uv.to(DEV)).cpu()
    close_to_one_ulp(got, mla_v_up(o, w_uv), row_relative=False)


def test_v_up_strided_views():
    """o_latent as the first 512 dims of (T, H, 576) rows and out as a view of
    the (T, H * 128) o_proj input give the same values as dense tensors."""
    T, H = 33, 16
    g = torch.Generator().manual_seed(5)
    wide = (torch.randn(T, H, 576, generator=g) / 4).bfloat16().to(DEV)
    w_uv = (torch.randn(H, 128, 512, generator=g) / 11).bfloat16().to(DEV)
    flat = torch.full((T, H * 128), 7.0, dtype=torch.bfloat16, device=DEV)
    ops.mla_v_up(wide, w_uv, out=flat.view(T, H, 128))
    dense = ops.mla_v_up(wide[..., :512].contiguous(), w_uv)
    assert torch.equal(flat.view(T, H, 128), dense)


def test_v_up_rejects_bad_shapes():
    o = torch.zeros(4, 16, 512, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(ValueError, match="w_uv"):
        ops.mla_v_up(o, torch.zeros(16, 512, 128, dtype=torch.bfloat16, device=DEV))
    with pytest.raises(ValueError, match="o_latent"):
        ops.mla_v_up(o[..., :256], torch.zeros(16, 128, 512, dtype=torch.bfloat16, device=DEV))
