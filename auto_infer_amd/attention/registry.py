"""Attention-family registry with the reference's API and error behaviour.

Mirrors auto_infer/layers/attention/registry.py: ``register_attention_family``
(:11-16), ``register_mtp_attention_family`` (:19-28), ``build_attention_backend``
(:119-136) and ``build_mtp_attention_backend`` (:139-157), same validation,
exception types and message stems.  The families this package adds are
``"gqa_hip"`` and ``"mla_hip"`` (and MTP ``"gqa_hip"``), plus ``"gqa_hip_nz"``
(and MTP ``"gqa_hip_nz"``): the same GQA backend over the two-tensor, 16-wide
NZ KV caches of the reference's graph mode (``GraphGqaBackend``,
gqa.py:192-211), for runners that hand the caches to other NZ consumers.  ``register_into``
installs the same builders into another registry -- the reference's own --
which is how a maintainer plugs them in without touching its dispatcher.
"""
from typing import Callable

AttentionBuilder = Callable[[object, str], object]
MtpAttentionBuilder = Callable[[object, str, str], object]
_FAMILIES: dict = {}
_MTP_FAMILIES: dict = {}

GQA_FAMILY = "gqa_hip"
MLA_FAMILY = "mla_hip"
GQA_NZ_FAMILY = "gqa_hip_nz"


def register_attention_family(name: str, builder: AttentionBuilder) -> None:
    if not name:
        raise ValueError("attention family name must not be empty")
    if name in _FAMILIES:
        raise ValueError(f"attention family already registered: {name}")
    _FAMILIES[name] = builder


def register_mtp_attention_family(name: str, builder: MtpAttentionBuilder) -> None:
    if not name:
        raise ValueError("MTP attention family name must not be empty")
    if name in _MTP_FAMILIES:
        raise ValueError(f"MTP attention family already registered: {name}")
    _MTP_FAMILIES[name] = builder


def _paged_only(family, mode):
    if mode == "dense":
        raise NotImplementedError(
            f"{family} is a paged-KV family; dense bring-up uses the reference's "
            f"full-softmax backends")


def _gqa_hip(model, mode: str, kv_layout: str = "nd", family: str = GQA_FAMILY):
    from auto_infer_amd.attention.gqa import GqaHipBackend
    _paged_only(family, mode)
    cfg = model.cfg
    return GqaHipBackend(
        n_q_heads=model.n_q_local, n_kv_heads=model.n_kv_local, head_dim=cfg.head_dim,
        scale=cfg.head_dim ** -0.5, num_layers=cfg.num_layers, device=model.device,
        dtype=model.dtype, w=model.w, layer_prefix=model.layer_prefix,
        rms_eps=getattr(cfg, "rms_eps", None), kv_layout=kv_layout)


def _gqa_hip_nz(model, mode: str):
    return _gqa_hip(model, mode, "nz", GQA_NZ_FAMILY)


def _mla_hip(model, mode: str):
    from auto_infer_amd.attention.mla import MlaHipBackend
    _paged_only(MLA_FAMILY, mode)
    cfg = model.cfg
    return MlaHipBackend(
        model.w, num_heads=cfg.num_heads, qk_nope=cfg.qk_nope, qk_rope=cfg.qk_rope,
        v_head_dim=cfg.v_head_dim, kv_lora_rank=cfg.kv_lora_rank,
        q_lora_rank=cfg.q_lora_rank, rms_eps=cfg.rms_eps,
        softmax_scale=model._softmax_scale, num_layers=cfg.num_layers,
        device=model.device, dtype=model.dtype, layer_prefix=model.layer_prefix)


def _gqa_hip_mtp(model, mode: str, prefix: str, kv_layout: str = "nd"):
    from auto_infer_amd.attention.gqa import GqaHipBackend
    cfg = model.cfg
    return GqaHipBackend(
        n_q_heads=model.n_q_local, n_kv_heads=model.n_kv_local, head_dim=cfg.head_dim,
        scale=cfg.head_dim ** -0.5, num_layers=1, device=model.device, dtype=model.dtype,
        w=model.w, layer_prefix=lambda _: prefix, rms_eps=getattr(cfg, "rms_eps", None),
        kv_layout=kv_layout)


def _gqa_hip_nz_mtp(model, mode: str, prefix: str):
    return _gqa_hip_mtp(model, mode, prefix, "nz")


BUILDERS = {GQA_FAMILY: _gqa_hip, MLA_FAMILY: _mla_hip, GQA_NZ_FAMILY: _gqa_hip_nz}
MTP_BUILDERS = {GQA_FAMILY: _gqa_hip_mtp, GQA_NZ_FAMILY: _gqa_hip_nz_mtp}


def register_into(register_family=register_attention_family,
                  register_mtp_family=register_mtp_attention_family):
    """Register this package's families through the given registration
    functions (defaults: this module's own registry)."""
    for name, builder in BUILDERS.items():
        register_family(name, builder)
    for name, builder in MTP_BUILDERS.items():
        register_mtp_family(name, builder)


register_into()


def build_attention_backend(model, mode: str, num_blocks: int = 0, block_size: int = 0):
    if mode not in {"dense", "paged", "graph"}:
        raise ValueError(f"unsupported attention mode: {mode}")
    family = model.ATTENTION_FAMILY
    try:
        builder = _FAMILIES[family]
    except KeyError:
        choices = ", ".join(sorted(_FAMILIES))
        raise KeyError(
            f"unregistered attention family: {family}; registered families: {choices}"
        ) from None
    backend = builder(model, mode)
    return backend, backend.alloc_kv_caches(num_blocks, block_size)


def build_mtp_attention_backend(model, mode: str, prefix: str, num_blocks: int = 0,
                                block_size: int = 0):
    if mode not in {"paged", "graph"}:
        raise ValueError(f"unsupported MTP attention mode: {mode}")
    family = model.ATTENTION_FAMILY
    try:
        builder = _MTP_FAMILIES[family]
    except KeyError:
        raise NotImplementedError(
            f"{family} MTP attention does not support {mode} mode") from None
    backend = builder(model, mode, prefix)
    return backend, backend.alloc_kv_caches(num_blocks, block_size)
