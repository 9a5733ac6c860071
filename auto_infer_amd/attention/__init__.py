"""Attention-backend families ``gqa_hip`` / ``gqa_hip_nz`` / ``mla_hip`` for the reference's
registry seam; importing this package registers them."""
from auto_infer_amd.attention.base import AttentionBackend, ForwardContext  # noqa: F401
from auto_infer_amd.attention.registry import (  # noqa: F401
    GQA_FAMILY, GQA_NZ_FAMILY, MLA_FAMILY, build_attention_backend, build_mtp_attention_backend,
    register_attention_family, register_into, register_mtp_attention_family)
