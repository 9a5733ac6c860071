"""Torch helpers around the attention op (projections, norms, RoPE).

These run before/after the hot path and are plain PyTorch on the GPU; they
restate the reference's helpers so the backends produce the same sub-block
output: ``_lin`` (auto_infer/layers/attention/base.py:9-18, plain weights
only), ``rms_norm`` (auto_infer/layers/norm.py:5-8, npu_rms_norm: fp32
mean-square, scale by weight), ``rotate_half`` / ``ds_rope_interleave``
(auto_infer/layers/rotary_embedding/__init__.py:10-23).
"""
import torch


def lin(x, w, bias=None):
    if isinstance(w, tuple):
        raise NotImplementedError("W8A8 projections are outside the paged-attention path")
    out = x @ w.t()
    return out + bias if bias is not None else out


def rms_norm(x, weight, eps):
    xf = x.float()
    y = xf * torch.rsqrt(xf.pow(2).mean(dim=-1, keepdim=True) + eps)
    return (y * weight.float()).to(x.dtype)


def rotate_half(x):
    x1, x2 = x.chunk(2, dim=-1)
    return torch.cat((-x2, x1), dim=-1)


def ds_rope_interleave(x):
    d = x.shape[-1]
    return x.view(*x.shape[:-1], d // 2, 2).transpose(-1, -2).reshape(*x.shape[:-1], d)
