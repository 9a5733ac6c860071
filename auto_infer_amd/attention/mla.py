"""Absorbed-MLA paged attention backend on the gfx950 kernels.

``MlaHipBackend`` follows the reference's absorbed variant
(auto_infer/layers/attention/mla.py:76-122 ``mla_paged_absorbed``, selected
by ``MlaFIABackend(absorb=True)`` :221-241): it caches only the 576-wide
latent ``[rms_norm(ckv) (512), rope(k_pe) (64)]`` of each token as one
MQA-style KV head, projects the query into latent space with W_UK, attends
with V = K and applies W_UV to the first 512 outputs.  The reference stores
the latent in both a k and a v cache (mla.py:113); here
``alloc_kv_caches`` returns the same tensor twice, so both "caches" hold
the written rows while HBM holds and the kernel reads them once.
"""
import torch

from auto_infer_amd import ops
from auto_infer_amd.attention.base import AttentionBackend
from auto_infer_amd.attention.layers import ds_rope_interleave, rms_norm, rotate_half
from auto_infer_amd.attention.metadata import step_plan


def build_absorb_weights(kv_b_weight, num_heads, qk_nope, v_head_dim, kv_lora_rank):
    """Split kv_b_proj (nh*(nope+vd), kvl) into W_UK (nh, nope, kvl) and
    W_UV (nh, vd, kvl) (reference mla.py:67-73)."""
    W = kv_b_weight.view(num_heads, qk_nope + v_head_dim, kv_lora_rank)
    w_uk, w_uv = W.split([qk_nope, v_head_dim], dim=1)
    return w_uk.contiguous(), w_uv.contiguous()


class MlaHipBackend(AttentionBackend):

    def __init__(self, w: dict, *, num_heads: int, qk_nope: int, qk_rope: int,
                 v_head_dim: int, kv_lora_rank: int, q_lora_rank, rms_eps: float,
                 softmax_scale: float, num_layers: int, device, dtype, absorb: bool = True,
                 layer_prefix=None, fuse_pre_attention: bool = True):
        if kv_lora_rank != ops.MLA_LATENT or qk_rope != ops.MLA_ROPE:
            raise NotImplementedError(
                f"mla_hip supports latent 512 + rope 64, got {kv_lora_rank} + {qk_rope}")
        self.w = w
        self.num_heads = num_heads
        self.qk_nope = qk_nope
        self.qk_rope = qk_rope
        self.v_head_dim = v_head_dim
        self.kv_lora_rank = kv_lora_rank
        self.q_lora_rank = q_lora_rank
        self.rms_eps = rms_eps
        self.softmax_scale = softmax_scale
        self.num_layers = num_layers
        self.device = device
        self.dtype = dtype
        self.absorb = True      # the latent cache is the point of this family
        self.layer_prefix = layer_prefix or (lambda i: f"model.layers.{i}.")
        self._absorb_w = {}
        # With fuse_pre_attention, q_latent and k_latent each come from one
        # kernel (norm / interleave / RoPE / W_UK product / cat; bf16 rounding
        # where the torch ops round) when the shapes allow it (nope 128), and
        # the W_UV product after attention from a third (v_head_dim 128, up to
        # ops.MLA_V_UP_MAX_ROWS query rows; longer steps use the library GEMM).
        self.fuse_pre_attention = fuse_pre_attention

    def alloc_kv_caches(self, num_blocks: int, block_size: int) -> list:
        kd = self.kv_lora_rank + self.qk_rope
        caches = []
        for _ in range(self.num_layers):
            latent = torch.zeros((num_blocks, block_size, 1, kd), device=self.device,
                                 dtype=self.dtype)
            caches.append((latent, latent))
        return caches

    def _weights(self, layer_idx):
        """(W_UK, W_UV, W_UK transposed to (H, 512, nope) for the fused query
        kernel), split once per layer."""
        if layer_idx not in self._absorb_w:
            p = self.layer_prefix(layer_idx)
            w_uk, w_uv = build_absorb_weights(
                self.w[p + "self_attn.kv_b_proj.weight"], self.num_heads, self.qk_nope,
                self.v_head_dim, self.kv_lora_rank)
            self._absorb_w[layer_idx] = (w_uk, w_uv, w_uk.transpose(1, 2).contiguous())
        return self._absorb_w[layer_idx]

    def _fusable(self, q, ckv_full, ctx):
        T = q.shape[0]

        def rows(t):             # one 64-wide row per token, 8-byte accesses
            return (t is not None and t.dtype == torch.bfloat16 and t.is_cuda and t.numel() == T * 64
                    and t.stride(-1) == 1 and t.stride(0) % 4 == 0 and t.data_ptr() % 8 == 0)
        return (self.fuse_pre_attention and self.qk_nope == 128 and q.dtype == torch.bfloat16
                and q.is_cuda and q.stride(-1) == 1 and q.stride(0) % 8 == 0 and q.stride(1) % 8 == 0
                and q.data_ptr() % 16 == 0 and ckv_full.stride(-1) == 1
                and ckv_full.stride(0) % 8 == 0 and ckv_full.data_ptr() % 16 == 0
                and rows(getattr(ctx, "cos", None)) and rows(getattr(ctx, "sin", None)))

    def attention(self, layer_idx: int, x: torch.Tensor, ctx) -> torch.Tensor:
        w = self.w
        p = self.layer_prefix(layer_idx)
        T = x.shape[0]
        nh, nope, rope, vd, kvl = (self.num_heads, self.qk_nope, self.qk_rope,
                                   self.v_head_dim, self.kv_lora_rank)
        if self.q_lora_rank is None:
            q = x @ w[p + "self_attn.q_proj.weight"].t()
        else:
            q = rms_norm(x @ w[p + "self_attn.q_a_proj.weight"].t(),
                         w[p + "self_attn.q_a_layernorm.weight"], self.rms_eps)
            q = q @ w[p + "self_attn.q_b_proj.weight"].t()
        q = q.view(T, nh, nope + rope)
        ckv_full = x @ w[p + "self_attn.kv_a_proj_with_mqa.weight"].t()
        w_uk, w_uv, w_uk_t = self._weights(layer_idx)
        fused = self._fusable(q, ckv_full, ctx)
        if fused:
            q_latent = ops.mla_q_latent(q, w_uk_t, ctx.cos, ctx.sin)
            k_latent = ops.mla_kv_latent(ckv_full, w[p + "self_attn.kv_a_layernorm.weight"],
                                         self.rms_eps, ctx.cos, ctx.sin)
        else:
            q_nope, q_pe = q.split([nope, rope], dim=-1)
            ckv, k_pe = ckv_full.split([kvl, rope], dim=-1)
            ckv = rms_norm(ckv, w[p + "self_attn.kv_a_layernorm.weight"], self.rms_eps)
            k_pe = k_pe.reshape(T, 1, rope)
            q_pe = ds_rope_interleave(q_pe)
            k_pe = ds_rope_interleave(k_pe)
            q_pe = q_pe * ctx.cos + rotate_half(q_pe) * ctx.sin
            k_pe = k_pe * ctx.cos + rotate_half(k_pe) * ctx.sin
            q_latent = torch.cat([torch.einsum("tnp,npl->tnl", q_nope, w_uk), q_pe],
                                 dim=-1).contiguous()
            k_latent = torch.cat([ckv.unsqueeze(1), k_pe], dim=-1).contiguous()
        self._write_kv(layer_idx, k_latent, None, ctx)
        o_latent = self._attn(layer_idx, q_latent, k_latent, None, ctx)
        if fused and vd == 128 and T * nh <= ops.MLA_V_UP_MAX_ROWS:
            o = ops.mla_v_up(o_latent, w_uv)
        else:
            o = torch.einsum("tnl,nvl->tnv", o_latent, w_uv)
        return o.reshape(T, nh * vd) @ w[p + "self_attn.o_proj.weight"].t()

    def _write_kv(self, layer_idx, k, v, ctx) -> None:
        latent, _ = ctx.kv_caches[layer_idx]
        ops.write_kv(k, None, latent, None, ctx.slot_mapping)

    def _attn(self, layer_idx, q, k, v, ctx) -> torch.Tensor:
        latent, _ = ctx.kv_caches[layer_idx]
        plan = step_plan(ctx, self.num_heads, 1, self.kv_lora_rank, latent.shape[1])
        return ops.paged_attention_mla(q, latent, plan, self.softmax_scale)
