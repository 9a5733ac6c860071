"""The C-ABI library loads and exports every symbol the header declares (CPU)."""
import ctypes
import os
import re

import pytest

from auto_infer_amd import _native

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    names = set()
    for fn in os.listdir(os.path.join(ROOT, "include")):
        if fn.endswith(".h"):
            text = open(os.path.join(ROOT, "include", fn)).read()
            names |= set(re.findall(r"^\s*(?:const\s+)?\w+\*?\s+\*?(aia_\w+)\s*\(", text, re.M))
    return names


def test_header_declares_the_binding_table():
    assert declared_symbols() == set(_native.SIGNATURES)


def test_library_exports_all_declared_symbols():
    if not os.path.exists(_native.LIB_PATH):
        pytest.fail(f"library not built: {_native.LIB_PATH}")
    lib = ctypes.CDLL(_native.LIB_PATH)
    for name in declared_symbols():
        assert hasattr(lib, name), name


def test_version_and_error_reporting_without_gpu():
    lib = _native.load()
    assert lib.aia_version() >= 100
    # argument validation happens before any device call
    rc = lib.aia_attn_workspace_bytes(4, 4, 3, 2, 128, 0, ctypes.byref(ctypes.c_int64()))
    assert rc == _native.AIA_ERR_INVALID
    assert "multiple" in _native.last_error()
    with pytest.raises(ValueError, match="multiple"):
        _native.check(rc, "aia_attn_workspace_bytes")


def test_workspace_query():
    out = ctypes.c_int64(0)
    _native.call("aia_attn_workspace_bytes", 16, 16, 16, 8, 128, 0, ctypes.byref(out))
    assert out.value > 0
    # sized for the range count asked for: the default 256 ranges of a
    # config-1 step need tens of MB, the maximum range count far more
    big = ctypes.c_int64(0)
    _native.call("aia_attn_workspace_bytes", 16, 16, 16, 8, 128, 16384, ctypes.byref(big))
    assert out.value < 64 << 20 < big.value


def test_argument_validation_of_the_fused_kernels_without_gpu():
    """Bad arguments are rejected before any device call, with the mapped
    exception types."""
    lib = _native.load()
    vp = ctypes.c_void_p
    # qk norm + rope: head_dim other than 128 and 64 is unsupported
    rc = lib.aia_qk_norm_rope(vp(16), 1024, 4, 4, 2, 96, vp(16), 96, vp(16), 96, None, None,
                              ctypes.c_float(1e-6), None)
    assert rc == _native.AIA_ERR_UNSUPPORTED
    with pytest.raises(NotImplementedError, match="head_dim"):
        _native.check(rc, "aia_qk_norm_rope")
    # norm weights go together
    rc = lib.aia_qk_norm_rope(vp(16), 1024, 4, 4, 2, 128, vp(16), 128, vp(16), 128, vp(16), None,
                              ctypes.c_float(1e-6), None)
    assert rc == _native.AIA_ERR_INVALID and "together" in _native.last_error()
    # MTP compaction: gear limits
    for gear in (0, 65):
        rc = lib.aia_mtp_compact(*([vp(16)] * 4), 8, vp(16), vp(16), vp(16), vp(16), gear, 2, 8,
                                 vp(16), vp(16), 8, vp(16), vp(16), vp(16), None)
        assert rc == _native.AIA_ERR_INVALID and "gear" in _native.last_error()
    # paged GQA: the scale must be positive
    rc = lib.aia_paged_attention_gqa(vp(16), 2048, 128, vp(16), vp(16), vp(16), 16, vp(16),
                                     vp(16), 1, 1, 16, 8, 128, 16, 4, ctypes.c_float(0.0),
                                     vp(16), 2048, 128, None, None, 0, 0, 0, 0, vp(16), 1 << 20,
                                     None)
    assert rc == _native.AIA_ERR_INVALID and "scale" in _native.last_error()
    # the pool's slots must be addressable by the int32 slot_mapping
    rc = lib.aia_paged_attention_gqa(vp(16), 2048, 128, vp(16), vp(16), vp(16), 16, vp(16),
                                     vp(16), 1, 1, 16, 8, 128, 256, 1 << 23, ctypes.c_float(0.1),
                                     vp(16), 2048, 128, None, None, 0, 0, 0, 0, vp(16), 1 << 20,
                                     None)
    assert rc == _native.AIA_ERR_INVALID and "int32 slot range" in _native.last_error()
    rc = lib.aia_paged_attention_mla(vp(16), 16 * 576, 576, vp(16), vp(16), 16, vp(16), vp(16),
                                     1, 1, 16, 512, 64, 256, 1 << 23, ctypes.c_float(0.1),
                                     vp(16), 16 * 512, 512, 0, 0, vp(256), 1 << 20, None)
    assert rc == _native.AIA_ERR_INVALID and "int32 slot range" in _native.last_error()
    # the workspace must be 256-byte aligned
    rc = lib.aia_attn_plan(vp(256), vp(256), vp(256), 16, 16, 1, 1, 16, 8, 128, 0, vp(256 + 16),
                           1 << 30, None)
    assert rc == _native.AIA_ERR_INVALID and "256-byte" in _native.last_error()
    # absorbed-MLA latents: rows of 576 with 16-byte alignment
    rc = lib.aia_mla_kv_latent(vp(16), 500, 4, vp(16), ctypes.c_float(1e-6), vp(16), 64, vp(16),
                               64, vp(16), 576, None)
    assert rc == _native.AIA_ERR_INVALID and "576" in _native.last_error()
    rc = lib.aia_mla_kv_latent(vp(8), 576, 4, vp(16), ctypes.c_float(1e-6), vp(16), 64, vp(16),
                               64, vp(16), 576, None)
    assert rc == _native.AIA_ERR_INVALID
    rc = lib.aia_mla_q_latent(vp(16), 16 * 192, 192, 4, 0, vp(16), vp(16), 64, vp(16), 64,
                              vp(16), 16 * 576, 576, None)
    assert rc == _native.AIA_ERR_INVALID and "sizes" in _native.last_error()
    rc = lib.aia_mla_q_latent(vp(16), 16 * 192, 100, 4, 16, vp(16), vp(16), 64, vp(16), 64,
                              vp(16), 16 * 576, 576, None)
    assert rc == _native.AIA_ERR_INVALID and "alignment" in _native.last_error()
    # no tokens: nothing to do, whatever the pointers
    assert lib.aia_mla_q_latent(None, 0, 0, 0, 16, None, None, 0, None, 0, None, 0, 0, None) == 0


def test_error_messages_are_per_thread():
    """aia_last_error() is thread local: two host threads failing with
    different arguments at the same time each read their own message."""
    import threading
    lib = _native.load()
    errs = []

    def worker(hq):
        out = ctypes.c_int64()
        for _ in range(2000):
            rc = lib.aia_attn_workspace_bytes(4, 4, hq, 2, 128, 0, ctypes.byref(out))
            msg = _native.last_error()
            if rc != _native.AIA_ERR_INVALID or f"num_q_heads {hq} " not in msg:
                errs.append((hq, rc, msg))
                return

    ts = [threading.Thread(target=worker, args=(hq,)) for hq in (3, 5, 7)]
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    assert not errs, errs[:3]
