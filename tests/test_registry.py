"""The drop-in boundary on the CPU: registry contract (same API, errors and
message stems as the reference's registry) and KV-cache allocation shapes."""
from types import SimpleNamespace

import pytest
import torch

from auto_infer_amd.attention import base, registry
from auto_infer_amd.attention.gqa import GqaHipBackend
from auto_infer_amd.attention.mla import MlaHipBackend


def test_abc_surface_is_exactly_alloc_and_attention():
    assert base.AttentionBackend.__abstractmethods__ == frozenset({"alloc_kv_caches", "attention"})
    with pytest.raises(TypeError):
        base.AttentionBackend()
    assert issubclass(GqaHipBackend, base.AttentionBackend)
    assert issubclass(MlaHipBackend, base.AttentionBackend)


def test_forward_context_fields_match_the_reference():
    names = [f for f in base.ForwardContext.__dataclass_fields__]
    assert names == ["token_ids", "positions", "slot_mapping", "block_table", "cu_seqlens_q",
                     "seqlens_kv", "attn_mask", "attn_backend", "kv_caches", "is_decode",
                     "cos", "sin", "active_token_mask"]


def test_families_registered_at_import():
    assert registry.GQA_FAMILY in registry._FAMILIES
    assert registry.MLA_FAMILY in registry._FAMILIES
    assert registry.GQA_FAMILY in registry._MTP_FAMILIES


def test_duplicate_and_empty_names_rejected():
    with pytest.raises(ValueError, match="already registered"):
        registry.register_attention_family("gqa_hip", lambda m, mode: None)
    with pytest.raises(ValueError, match="must not be empty"):
        registry.register_attention_family("", lambda m, mode: None)
    with pytest.raises(ValueError, match="already registered"):
        registry.register_mtp_attention_family("gqa_hip", lambda m, mode, p: None)


def test_unknown_family_and_bad_mode():
    with pytest.raises(KeyError, match="unregistered attention family: nope"):
        registry.build_attention_backend(SimpleNamespace(ATTENTION_FAMILY="nope"), "paged")
    with pytest.raises(ValueError, match="unsupported attention mode"):
        registry.build_attention_backend(SimpleNamespace(ATTENTION_FAMILY="gqa_hip"), "eager")
    with pytest.raises(ValueError, match="unsupported MTP attention mode"):
        registry.build_mtp_attention_backend(SimpleNamespace(ATTENTION_FAMILY="gqa_hip"),
                                             "dense", "p.")


def test_mla_mtp_fails_explicitly():
    with pytest.raises(NotImplementedError, match="mla_hip.*MTP.*graph"):
        registry.build_mtp_attention_backend(SimpleNamespace(ATTENTION_FAMILY="mla_hip"),
                                             "graph", "model.mtp.", 5, 16)


def _gqa_model():
    return SimpleNamespace(
        ATTENTION_FAMILY="gqa_hip", cfg=SimpleNamespace(head_dim=128, num_layers=3, rms_eps=1e-6),
        n_q_local=16, n_kv_local=8, device=torch.device("cpu"), dtype=torch.bfloat16, w={},
        layer_prefix=lambda i: f"model.layers.{i}.")


def test_gqa_builder_and_cache_layout():
    backend, caches = registry.build_attention_backend(_gqa_model(), "paged", 10, 32)
    assert isinstance(backend, GqaHipBackend)
    assert backend.scale == 128 ** -0.5
    assert len(caches) == 3
    for c in caches:
        assert c.shape == (2, 10, 32, 8, 128) and c.dtype == torch.bfloat16
    backend, _ = registry.build_attention_backend(_gqa_model(), "graph", 2, 16)
    assert isinstance(backend, GqaHipBackend)
    with pytest.raises(NotImplementedError, match="paged-KV family"):
        registry.build_attention_backend(_gqa_model(), "dense", 2, 16)


def test_gqa_nz_family_allocates_graph_mode_caches():
    """gqa_hip_nz allocates what GraphGqaBackend.alloc_kv_caches does
    (gqa.py:192-201): per layer two (num_blocks, block_size, n_kv, head_dim)
    tensors."""
    model = _gqa_model()
    model.ATTENTION_FAMILY = "gqa_hip_nz"
    backend, caches = registry.build_attention_backend(model, "graph", 10, 32)
    assert isinstance(backend, GqaHipBackend) and backend.kv_layout == "nz"
    assert len(caches) == 3
    for kc, vc in caches:
        assert kc.shape == vc.shape == (10, 32, 8, 128) and kc is not vc
    backend, caches = registry.build_mtp_attention_backend(model, "graph", "model.mtp.", 5, 16)
    assert backend.kv_layout == "nz" and caches[0][0].shape == (5, 16, 8, 128)
    with pytest.raises(ValueError, match="kv_layout"):
        GqaHipBackend(16, 8, 128, 0.1, 1, torch.device("cpu"), torch.bfloat16, kv_layout="nhd")


def test_gqa_mtp_builds_one_layer_with_prefix():
    backend, caches = registry.build_mtp_attention_backend(_gqa_model(), "paged",
                                                           "model.mtp_layers.0.", 5, 16)
    assert backend.num_layers == 1 and len(caches) == 1
    assert backend.layer_prefix(0) == "model.mtp_layers.0."


def test_mla_builder_aliases_one_latent_cache():
    cfg = SimpleNamespace(num_heads=16, qk_nope=128, qk_rope=64, v_head_dim=128,
                          kv_lora_rank=512, q_lora_rank=None, rms_eps=1e-6, num_layers=2)
    model = SimpleNamespace(ATTENTION_FAMILY="mla_hip", cfg=cfg, w={}, _softmax_scale=0.07,
                            device=torch.device("cpu"), dtype=torch.bfloat16,
                            layer_prefix=lambda i: f"model.layers.{i}.")
    backend, caches = registry.build_attention_backend(model, "paged", 6, 128)
    assert isinstance(backend, MlaHipBackend) and backend.softmax_scale == 0.07
    for k, v in caches:
        assert k.shape == (6, 128, 1, 576) and k is v


def test_register_into_another_registry():
    """How a maintainer installs the families into the reference's registry."""
    seen, seen_mtp = {}, {}

    def reg(name, builder):
        if name in seen:
            raise ValueError(f"attention family already registered: {name}")
        seen[name] = builder

    registry.register_into(reg, lambda n, b: seen_mtp.__setitem__(n, b))
    assert set(seen) == {"gqa_hip", "mla_hip", "gqa_hip_nz"}
    assert set(seen_mtp) == {"gqa_hip", "gqa_hip_nz"}
