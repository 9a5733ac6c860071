"""Fused pre-attention kernel (QK-RMSNorm + NeoX RoPE in place over the qkv
projection) vs the bf16 torch restatement in oracle/pre_attention.py.

Bars: without the norm, bit-exact (the kernel rounds where the torch ops
round); with the norm, within one bf16 ulp of the row's largest value (the
fp32 mean of squares is summed in a different order, which can move a normed
value by one ulp) and bit-exact on at least 99% of values; V is never
touched.
"""
import pytest
import torch

from auto_infer_amd import ops
from oracle.pre_attention import qk_norm_rope, rope_tables

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def case(T, hq, hkv, norm, seed, pos_hi=40000, d=128):
    g = torch.Generator().manual_seed(seed)
    qkv = (torch.randn(T, (hq + 2 * hkv) * d, generator=g) * 2).bfloat16()
    pos = torch.randint(0, pos_hi, (T,), generator=g)
    cos, sin = rope_tables(pos, d)
    wq = (1 + 0.2 * torch.randn(d, generator=g)).bfloat16() if norm else None
    wk = (1 + 0.2 * torch.randn(d, generator=g)).bfloat16() if norm else None
    return qkv, cos, sin, wq, wk


def gpu(qkv, hq, hkv, cos, sin, wq, wk, d=128):
    buf = qkv.to(DEV)
    q, k, v = ops.qk_norm_rope(buf, hq, hkv, cos.to(DEV), sin.to(DEV),
                               None if wq is None else wq.to(DEV),
                               None if wk is None else wk.to(DEV), 1e-6, head_dim=d)
    torch.cuda.synchronize()
    return q.cpu(), k.cpu(), v.cpu()


@pytest.mark.parametrize("T,hq,hkv", [(16, 16, 8), (2048, 28, 4), (32, 32, 8), (1, 64, 8),
                                      (7, 4, 2)])
@pytest.mark.parametrize("norm", [False, True])
@pytest.mark.parametrize("d", [128, 64])
def test_qk_norm_rope_vs_oracle(T, hq, hkv, norm, d):
    """head_dim 128 (Qwen2-7B / Qwen3) and 64 (Qwen2 / Qwen2.5 0.5B)."""
    qkv, cos, sin, wq, wk = case(T, hq, hkv, norm, seed=T + hq, d=d)
    gq, gk, gv = gpu(qkv, hq, hkv, cos, sin, wq, wk, d)
    eq, ek, ev = qk_norm_rope(qkv, hq, hkv, cos, sin, wq, wk, 1e-6)
    assert torch.equal(gv, ev)
    for got, exp in ((gq, eq), (gk, ek)):
        if not norm:
            assert torch.equal(got, exp)
        else:
            # a one-ulp difference in a normed input moves a rotated output by
            # up to one ulp of the row's largest values (cancellation aside)
            diff = (got.float() - exp.float()).abs()
            row_max = exp.float().abs().amax(dim=-1, keepdim=True)
            assert bool((diff <= row_max * 2.0 ** -7).all()), diff.max().item()
            same = (got == exp).float().mean().item()
            print(f"bit-exact fraction {same:.5f}", flush=True)
            assert same >= 0.99


def test_strided_tables_and_positions_zero():
    """cos/sin given as (T, 1, 128) views of wider tables; position 0 leaves
    q and k unchanged."""
    T, hq, hkv = 5, 8, 2
    qkv, _, _, _, _ = case(T, hq, hkv, False, seed=3)
    cos, sin = rope_tables([0] * T, 128)
    wide_c = torch.zeros(T, 1, 256, dtype=torch.bfloat16)
    wide_s = torch.zeros(T, 1, 256, dtype=torch.bfloat16)
    wide_c[..., :128] = cos
    wide_s[..., :128] = sin
    buf = qkv.to(DEV)
    q, k, v = ops.qk_norm_rope(buf, hq, hkv, wide_c.to(DEV)[..., :128], wide_s.to(DEV)[..., :128])
    torch.cuda.synchronize()
    assert torch.equal(buf.cpu(), qkv)


def test_rejects_bad_shapes():
    qkv = torch.zeros(4, (8 + 4) * 128, dtype=torch.bfloat16, device=DEV)
    cos = torch.zeros(4, 1, 128, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(ValueError):
        ops.qk_norm_rope(qkv, 8, 4, cos, cos)          # width != (Hq + 2 Hkv) x 128
    with pytest.raises(ValueError):
        ops.qk_norm_rope(qkv[:, :1024], 4, 2, cos[:, :, :64], cos[:, :, :64])


def test_unsupported_head_dim():
    qkv = torch.zeros(4, (8 + 4) * 96, dtype=torch.bfloat16, device=DEV)
    cos = torch.zeros(4, 1, 96, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(NotImplementedError):
        ops.qk_norm_rope(qkv, 8, 2, cos, cos, head_dim=96)
