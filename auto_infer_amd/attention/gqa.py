"""GQA paged attention backend on the gfx950 kernels.

``GqaHipBackend`` is a drop-in for the reference's ``GqaFIABackend``
(auto_infer/layers/attention/gqa.py:52-94): same constructor arguments,
same KV-cache layout ``(2, num_blocks, block_size, n_kv, head_dim)`` per
layer (gqa.py:69-74), same sub-block math around the op pair (packed qkv
projection, optional Qwen3 QK-RMSNorm, NeoX RoPE, o_proj; gqa.py:27-49) and
the same op-pair seam ``_write_kv`` / ``_attn``.  Only the op pair differs:
the KV slot write and the split-K paged attention run as HIP kernels.
The backend is graph-capturable (no host sync, no allocation in ``_attn``
once the step's plan exists), so it serves both the "paged" and "graph"
modes.  With ``kv_layout="nz"`` it also takes the caches of the reference's
graph-mode backend (``GraphGqaBackend``, gqa.py:134-226): per layer a (k, v)
pair of (num_blocks, block_size, n_kv, head_dim) tensors whose memory is the
16-wide fractal NZ layout (viewed (num_blocks, n_kv * head_dim / 16,
block_size, 16) by npu_scatter_pa_kv_cache and FIA-v2, gqa.py:202-226).
"""
import torch

from auto_infer_amd import ops
from auto_infer_amd.attention.base import AttentionBackend
from auto_infer_amd.attention.layers import lin, rms_norm, rotate_half
from auto_infer_amd.attention.metadata import step_plan


class GqaHipBackend(AttentionBackend):

    def __init__(self, n_q_heads: int, n_kv_heads: int, head_dim: int, scale: float,
                 num_layers: int, device, dtype, w: dict = None, layer_prefix=None,
                 rms_eps=None, fuse_kv_write: bool = True, fuse_pre_attention: bool = True,
                 kv_layout: str = "nd"):
        self.n_q_heads = n_q_heads
        self.n_kv_heads = n_kv_heads
        self.head_dim = head_dim
        self.scale = scale
        self.num_layers = num_layers
        self.device = device
        self.dtype = dtype
        self.w = w
        self.layer_prefix = layer_prefix or (lambda i: f"model.layers.{i}.")
        self.rms_eps = rms_eps
        # With fuse_kv_write, _write_kv defers the slot write to the attention
        # kernel of the following _attn (same cache contents, one launch less);
        # attention() always calls the two in that order.  The kernel writes
        # each new row at the slot its request's block table gives its
        # position, so the write is deferred only for contexts that declare
        # their slot_mapping equal to those slots
        # (ctx.aia_slots_from_block_table, set by this package's packers);
        # any other slot_mapping is written as given, by its own launch.
        self.fuse_kv_write = fuse_kv_write
        # With fuse_pre_attention, the split / QK-RMSNorm / RoPE steps run as
        # one in-place kernel over the qkv projection (bf16 rounding where the
        # torch ops round); q, k, v are then strided views of it.
        self.fuse_pre_attention = fuse_pre_attention
        if kv_layout not in ops.KV_LAYOUTS:
            raise ValueError(f"kv_layout must be one of {sorted(ops.KV_LAYOUTS)}")
        self.kv_layout = kv_layout
        self._pending = None

    def alloc_kv_caches(self, num_blocks: int, block_size: int) -> list:
        if self.kv_layout == "nz":      # GraphGqaBackend.alloc_kv_caches (gqa.py:195-204)
            shape = (num_blocks, block_size, self.n_kv_heads, self.head_dim)
            return [(torch.zeros(shape, device=self.device, dtype=self.dtype),
                     torch.zeros(shape, device=self.device, dtype=self.dtype))
                    for _ in range(self.num_layers)]
        shape = (2, num_blocks, block_size, self.n_kv_heads, self.head_dim)
        return [torch.zeros(shape, device=self.device, dtype=self.dtype)
                for _ in range(self.num_layers)]

    def _write(self, k, v, kc, vc, slot_mapping):
        if self.kv_layout == "nz":
            ops.write_kv_nz(k, v, kc, vc, slot_mapping)
        else:
            ops.write_kv(k, v, kc, vc, slot_mapping)

    def attention(self, layer_idx: int, x: torch.Tensor, ctx) -> torch.Tensor:
        T = x.shape[0]
        n_q, n_kv, hd = self.n_q_heads, self.n_kv_heads, self.head_dim
        w = self.w
        p = self.layer_prefix(layer_idx) + "self_attn."
        qkv = lin(x, w[p + "qkv_proj.weight"], w.get(p + "qkv_proj.bias"))
        qn = w.get(p + "q_norm.weight")
        if self._fusable(qkv, ctx):
            q, k, v = ops.qk_norm_rope(qkv, n_q, n_kv, ctx.cos, ctx.sin, qn,
                                       w.get(p + "k_norm.weight") if qn is not None else None,
                                       self.rms_eps if self.rms_eps is not None else 1e-6,
                                       head_dim=hd)
        else:
            q, k, v = qkv.split((n_q * hd, n_kv * hd, n_kv * hd), dim=-1)
            q = q.view(T, n_q, hd)
            k = k.view(T, n_kv, hd)
            v = v.view(T, n_kv, hd)
            if qn is not None:
                q = rms_norm(q, qn, self.rms_eps)
                k = rms_norm(k, w[p + "k_norm.weight"], self.rms_eps)
            q = q * ctx.cos + rotate_half(q) * ctx.sin
            k = k * ctx.cos + rotate_half(k) * ctx.sin
        self._write_kv(layer_idx, k, v, ctx)
        o = self._attn(layer_idx, q, k, v, ctx).reshape(T, n_q * hd)
        return lin(o, w[p + "o_proj.weight"])

    def _fusable(self, qkv, ctx):
        T = qkv.shape[0]
        def aligned(t):          # 16-byte accesses: 8-element strides, 16-byte base
            return t.stride(0) % 8 == 0 and t.data_ptr() % 16 == 0
        hd = self.head_dim
        return (self.fuse_pre_attention and hd in (128, 64) and qkv.dtype == torch.bfloat16
                and qkv.is_cuda and qkv.stride(-1) == 1 and aligned(qkv)
                and all(t.dtype == torch.bfloat16 and t.numel() == T * hd and t.stride(-1) == 1
                        and aligned(t) for t in (ctx.cos, ctx.sin)))

    def _write_kv(self, layer_idx: int, k: torch.Tensor, v: torch.Tensor, ctx) -> None:
        cache = ctx.kv_caches[layer_idx]
        if (self.fuse_kv_write and getattr(ctx, "aia_slots_from_block_table", False)
                and k.shape[0] == ctx.slot_mapping.shape[0]):
            self._pending = (layer_idx, id(ctx), k, v)
            return
        self._write(k, v, cache[0], cache[1], ctx.slot_mapping)

    def _attn(self, layer_idx: int, q, k, v, ctx) -> torch.Tensor:
        cache = ctx.kv_caches[layer_idx]
        plan = step_plan(ctx, self.n_q_heads, self.n_kv_heads, self.head_dim, cache[0].shape[1])
        pending, self._pending = self._pending, None
        if pending is not None and pending[:2] == (layer_idx, id(ctx)):
            return ops.paged_attention_gqa(q, cache[0], cache[1], plan, self.scale,
                                           key_new=pending[2], value_new=pending[3],
                                           kv_layout=self.kv_layout)
        if pending is not None:      # a deferred write for another call: do it now
            lay, _, pk, pv = pending
            c = ctx.kv_caches[lay]
            self._write(pk, pv, c[0], c[1], ctx.slot_mapping)
        return ops.paged_attention_gqa(q, cache[0], cache[1], plan, self.scale,
                                       kv_layout=self.kv_layout)
