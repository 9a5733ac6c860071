"""The attention seam and step context, mirrored from the reference.

``AttentionBackend`` has exactly the reference's abstract surface
(auto_infer/layers/attention/base.py:21-38): ``alloc_kv_caches`` and
``attention``.  ``ForwardContext`` has the reference's fields
(auto_infer/forward_context.py:9-23); the packer in
``auto_infer_amd.packing`` additionally attaches device copies of the
metadata as extra attributes, which the dataclass allows.
"""
from abc import ABC, abstractmethod
from dataclasses import dataclass

import torch


class AttentionBackend(ABC):
    """Owns the whole attention sub-block of one layer."""

    @abstractmethod
    def alloc_kv_caches(self, num_blocks: int, block_size: int) -> list:
        """Per-layer KV cache list (backend-specific shape/dtype/device)."""
        raise NotImplementedError

    @abstractmethod
    def attention(self, layer_idx: int, x: torch.Tensor, ctx) -> torch.Tensor:
        """x: normed hidden (T, hidden); returns (T, hidden) ready to add to
        the residual."""
        raise NotImplementedError


@dataclass
class ForwardContext:
    token_ids: torch.Tensor
    positions: torch.Tensor
    slot_mapping: torch.Tensor
    block_table: torch.Tensor
    cu_seqlens_q: list
    seqlens_kv: list
    attn_mask: torch.Tensor
    attn_backend: AttentionBackend
    kv_caches: list
    is_decode: bool
    cos: torch.Tensor | None = None
    sin: torch.Tensor | None = None
    active_token_mask: torch.Tensor | None = None
