"""Torch-CPU restatement of the pre-attention steps of the GQA sub-block.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Reference: ``_GqaProjRopeMixin.attention`` (auto_infer/layers/attention/
gqa.py:27-49) splits the packed qkv projection into q (T, Hq, D), k (T, Hkv,
D) and v (gqa.py:15-17, 37-40); if the layer has q_norm/k_norm weights it
applies per-head RMSNorm to q and k (gqa.py:41-44, ``npu_rms_norm`` in
auto_infer/layers/norm.py:5-8: mean of squares in fp32, multiply by the
weight, result in the input dtype); then NeoX RoPE
``x * cos + rotate_half(x) * sin`` (gqa.py:45-46, rotate_half in
auto_infer/layers/rotary_embedding/__init__.py:10-13) with cos/sin of shape
(T, 1, D) (auto_infer/models/base.py:74-75, tables from
auto_infer/models/qwen2.py:170-176).  All of it runs as bf16 torch ops, so
``qk_norm_rope`` below does the same: every op rounds its result to bf16.

``qk_norm_rope_f64`` is the same mathematics in float64 with no rounding,
used to pin the bf16 restatement by identities (see tests/test_oracle_rope.py).
"""
import torch


def rms_norm(x, weight, eps):
    """norm.py:5-8: fp32 mean of squares over the last dim, scale by the
    weight, back to the input dtype."""
    xf = x.float()
    y = xf * torch.rsqrt(xf.pow(2).mean(dim=-1, keepdim=True) + eps)
    return (y * weight.float()).to(x.dtype)


def rotate_half(x):
    """rotary_embedding/__init__.py:10-13."""
    x1, x2 = x.chunk(2, dim=-1)
    return torch.cat((-x2, x1), dim=-1)


def rope_tables(positions, dim, base=10000.0, dtype=torch.bfloat16):
    """qwen2.py:170-176: NeoX cos/sin tables, (T, 1, dim) as base.py:74-75."""
    inv = 1.0 / (base ** (torch.arange(0, dim, 2, dtype=torch.float32) / dim))
    f = torch.outer(torch.as_tensor(positions).float(), inv)
    emb = torch.cat((f, f), dim=-1)
    return emb.cos().to(dtype)[:, None], emb.sin().to(dtype)[:, None]


def qk_norm_rope(qkv, num_q_heads, num_kv_heads, cos, sin, q_norm_weight=None,
                 k_norm_weight=None, eps=1e-6):
    """gqa.py:37-46 on a packed (T, (Hq + 2 Hkv) * D) bf16 projection.
    Returns (q, k, v) as (T, H, D) bf16 tensors."""
    T = qkv.shape[0]
    D = cos.shape[-1]
    q, k, v = qkv.split((num_q_heads * D, num_kv_heads * D, num_kv_heads * D), dim=-1)
    q = q.reshape(T, num_q_heads, D)
    k = k.reshape(T, num_kv_heads, D)
    v = v.reshape(T, num_kv_heads, D)
    if q_norm_weight is not None:
        q = rms_norm(q, q_norm_weight, eps)
        k = rms_norm(k, k_norm_weight, eps)
    cos = cos.reshape(T, 1, D)
    sin = sin.reshape(T, 1, D)
    q = q * cos + rotate_half(q) * sin
    k = k * cos + rotate_half(k) * sin
    return q, k, v


def qk_norm_rope_f64(qkv, num_q_heads, num_kv_heads, positions, q_norm_weight=None,
                     k_norm_weight=None, eps=1e-6, base=10000.0):
    """The same mathematics in float64 with exact angles (no bf16 rounding)."""
    T = qkv.shape[0]
    D = qkv.shape[1] // (num_q_heads + 2 * num_kv_heads)
    x = qkv.double()
    q, k, v = x.split((num_q_heads * D, num_kv_heads * D, num_kv_heads * D), dim=-1)
    q = q.reshape(T, num_q_heads, D)
    k = k.reshape(T, num_kv_heads, D)
    v = v.reshape(T, num_kv_heads, D)
    if q_norm_weight is not None:
        def nrm(t, w):
            return t * torch.rsqrt(t.pow(2).mean(dim=-1, keepdim=True) + eps) * w.double()
        q = nrm(q, q_norm_weight)
        k = nrm(k, k_norm_weight)
    inv = 1.0 / (base ** (torch.arange(0, D, 2, dtype=torch.float64) / D))
    f = torch.outer(torch.as_tensor(positions).double(), inv)
    emb = torch.cat((f, f), dim=-1)[:, None]
    q = q * emb.cos() + rotate_half(q) * emb.sin()
    k = k * emb.cos() + rotate_half(k) * emb.sin()
    return q, k, v


# ------------------------------------------------------------- absorbed MLA

def ds_rope_interleave(x):
    """rotary_embedding/__init__.py:15-23: the DeepSeek pe dims are stored
    interleaved; view (d/2, 2), transpose, flatten: out[j] = in[2j],
    out[d/2 + j] = in[2j + 1]."""
    d = x.shape[-1]
    return x.reshape(*x.shape[:-1], d // 2, 2).transpose(-1, -2).reshape(*x.shape[:-1], d)


def mla_kv_latent(ckv_full, norm_weight, eps, cos, sin, kv_lora_rank=512):
    """mla.py:97-111 on the kv_a_proj_with_mqa output (T, kvl + rope):
    k_latent = cat(rms_norm(ckv), rope(ds_rope_interleave(k_pe))), (T, 1,
    kvl + rope), every op rounding to bf16 as the reference's bf16 ops do."""
    T = ckv_full.shape[0]
    ckv, k_pe = ckv_full.split([kv_lora_rank, ckv_full.shape[1] - kv_lora_rank], dim=-1)
    ckv = rms_norm(ckv, norm_weight, eps)
    k_pe = ds_rope_interleave(k_pe.reshape(T, 1, -1))
    cos = cos.reshape(T, 1, -1)
    sin = sin.reshape(T, 1, -1)
    k_pe = k_pe * cos + rotate_half(k_pe) * sin
    return torch.cat([ckv.unsqueeze(1), k_pe], dim=-1)


def mla_q_latent(q, w_uk, cos, sin):
    """mla.py:93-107 on q (T, H, nope + rope): q_latent = cat(einsum(
    "tnp,npl->tnl", q_nope, W_UK), rope(ds_rope_interleave(q_pe))), (T, H,
    kvl + rope).  The einsum is a bf16 GEMM: fp32 products and sums, one
    rounding to bf16 (as the library GEMM it runs on)."""
    T, H, _ = q.shape
    nope = w_uk.shape[1]
    q_nope, q_pe = q.split([nope, q.shape[2] - nope], dim=-1)
    absorbed = torch.einsum("tnp,npl->tnl", q_nope.float(), w_uk.float()).to(q.dtype)
    q_pe = ds_rope_interleave(q_pe)
    cos = cos.reshape(T, 1, -1)
    sin = sin.reshape(T, 1, -1)
    q_pe = q_pe * cos + rotate_half(q_pe) * sin
    return torch.cat([absorbed, q_pe], dim=-1)


def mla_v_up(o_latent, w_uv):
    """mla.py:120-121: o = einsum("tnl,nvl->tnv", o_latent[..., :kvl], W_UV)
    for o_latent (T, H, >= kvl) and W_UV (H, vd, kvl).  A bf16 GEMM: fp32
    products and sums, one rounding to bf16."""
    kvl = w_uv.shape[2]
    return torch.einsum("tnl,nvl->tnv", o_latent[..., :kvl].float(), w_uv.float()).to(o_latent.dtype)


def mla_latents_f64(q, w_uk, ckv_full, norm_weight, eps, positions, kv_lora_rank=512,
                    base=10000.0):
    """q_latent and k_latent in float64 with exact angles (no rounding)."""
    T, H, _ = q.shape
    nope = w_uk.shape[1]
    x = q.double()
    q_nope, q_pe = x.split([nope, x.shape[2] - nope], dim=-1)
    rope = q_pe.shape[-1]
    inv = 1.0 / (base ** (torch.arange(0, rope, 2, dtype=torch.float64) / rope))
    f = torch.outer(torch.as_tensor(positions).double(), inv)
    emb = torch.cat((f, f), dim=-1)[:, None]

    def rot(t):
        t = ds_rope_interleave(t)
        return t * emb.cos() + rotate_half(t) * emb.sin()
    ql = torch.cat([torch.einsum("tnp,npl->tnl", q_nope, w_uk.double()), rot(q_pe)], dim=-1)
    c = ckv_full.double()
    ckv, k_pe = c.split([kv_lora_rank, c.shape[1] - kv_lora_rank], dim=-1)
    ckv = ckv * torch.rsqrt(ckv.pow(2).mean(dim=-1, keepdim=True) + eps) * norm_weight.double()
    kl = torch.cat([ckv.unsqueeze(1), rot(k_pe.reshape(T, 1, -1))], dim=-1)
    return ql, kl
