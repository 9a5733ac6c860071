"""ctypes binding of the C ABI in include/auto_infer_amd.h.

The HIP library is the only compute path: if it is missing or fails to
load, every op raises ``NativeLibraryError`` -- there is no CPU fallback.
Status codes map to the Python exception types the reference raises for
the same conditions (ValueError for bad arguments and gear / capacity
overflow, NotImplementedError for unsupported shapes, RuntimeError for HIP
failures).
"""
import ctypes
import os
import threading

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_lib",
                        "libautoinfer_amd.so")

AIA_OK = 0
AIA_ERR_INVALID = -1
AIA_ERR_HIP = -2
AIA_ERR_CAPACITY = -3
AIA_ERR_UNSUPPORTED = -4

c_i32, c_i64, c_f32, c_vp = ctypes.c_int32, ctypes.c_int64, ctypes.c_float, ctypes.c_void_p

# name -> argtypes; every symbol declared in include/auto_infer_amd.h
SIGNATURES = {
    "aia_version": [],
    "aia_last_error": [],
    "aia_kv_write": [c_vp, c_i64, c_vp, c_i64, c_vp, c_vp, c_vp, c_i32, c_i32, c_i32,
                     c_i64, c_vp],
    "aia_kv_write_nz": [c_vp, c_i64, c_vp, c_i64, c_vp, c_vp, c_vp, c_i32, c_i32, c_i32, c_i64,
                        c_vp],
    "aia_attn_workspace_bytes": [c_i32, c_i32, c_i32, c_i32, c_i32, c_i32,
                                 ctypes.POINTER(c_i64)],
    "aia_attn_workspace_layout": [c_i32, c_i32, c_i32, c_i32, c_i32, c_i32,
                                  ctypes.POINTER(c_i64), c_i32],
    "aia_attn_plan": [c_vp, c_vp, c_vp, c_i32, c_i32, c_i32, c_i32, c_i32, c_i32, c_i32, c_i32,
                      c_vp, c_i64, c_vp],
    "aia_paged_attention_gqa": [c_vp, c_i64, c_i64, c_vp, c_vp, c_vp, c_i32, c_vp, c_vp,
                                c_i32, c_i32, c_i32, c_i32, c_i32, c_i32, c_i32, c_f32,
                                c_vp, c_i64, c_i64, c_vp, c_vp, c_i64, c_i64, c_i32, c_i32,
                                c_vp, c_i64, c_vp],
    "aia_paged_attention_gqa_noalloc": [c_vp, c_i64, c_i64, c_vp, c_vp, c_vp, c_i32, c_vp,
                                        c_vp, c_i32, c_i32, c_i32, c_i32, c_i32, c_i32, c_i32,
                                        c_f32, c_vp, c_i64, c_i64, c_vp, c_vp, c_i64, c_i64,
                                        c_i32, c_i32, c_vp],
    "aia_noalloc_scratch_bytes": [ctypes.POINTER(c_i64)],
    "aia_paged_attention_mla": [c_vp, c_i64, c_i64, c_vp, c_vp, c_i32, c_vp, c_vp, c_i32,
                                c_i32, c_i32, c_i32, c_i32, c_i32, c_i32, c_f32, c_vp,
                                c_i64, c_i64, c_i32, c_i32, c_vp, c_i64, c_vp],
    "aia_pack_rows": [c_vp, c_vp, c_i32, c_vp, c_vp, c_i32, c_vp, c_i64, c_vp, c_i64, c_vp,
                      c_i32, c_i32, c_i32, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp,
                      c_i32, c_i32, c_vp],
    "aia_pack_rows_inline": [c_vp, c_i32, c_i32, c_i32, c_vp, c_i64, c_vp, c_i64, c_i32, c_i32,
                             c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_i32, c_i32, c_vp],
    "aia_splice_tokens": [c_vp, c_i32, c_vp, c_i64, c_vp],
    "aia_qk_norm_rope": [c_vp, c_i64, c_i32, c_i32, c_i32, c_i32, c_vp, c_i64, c_vp, c_i64,
                         c_vp, c_vp, c_f32, c_vp],
    "aia_mla_kv_latent": [c_vp, c_i64, c_i32, c_vp, c_f32, c_vp, c_i64, c_vp, c_i64, c_vp, c_i64,
                          c_vp],
    "aia_mla_q_latent": [c_vp, c_i64, c_i64, c_i32, c_i32, c_vp, c_vp, c_i64, c_vp, c_i64, c_vp,
                         c_i64, c_i64, c_vp],
    "aia_mla_v_up": [c_vp, c_i64, c_i64, c_i32, c_i32, c_vp, c_vp, c_i64, c_i64, c_vp],
    "aia_mtp_compact": [c_vp, c_vp, c_vp, c_vp, c_i64, c_vp, c_vp, c_vp, c_vp, c_i32, c_i32,
                        c_i32, c_vp, c_vp, c_i64, c_vp, c_vp, c_vp, c_vp],
}


class NativeLibraryError(RuntimeError):
    """The gfx950 HIP library is not built or could not be loaded."""


_lock = threading.Lock()
_lib = None


def load():
    """Load the shared library once (after torch, so both share one HIP runtime)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        import torch  # noqa: F401  -- torch's HIP runtime must be loaded first
        if not os.path.exists(LIB_PATH):
            raise NativeLibraryError(
                f"{LIB_PATH} is missing; build it with "
                "`python -m auto_infer_amd.csrc.build` (hipcc, gfx950)")
        try:
            lib = ctypes.CDLL(LIB_PATH)
        except OSError as exc:
            raise NativeLibraryError(f"cannot load {LIB_PATH}: {exc}") from exc
        for name, argtypes in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = argtypes
            fn.restype = ctypes.c_char_p if name == "aia_last_error" else ctypes.c_int
        _lib = lib
        return lib


def last_error():
    return load().aia_last_error().decode(errors="replace")


def check(rc, what):
    if rc == AIA_OK:
        return
    msg = f"{what}: {last_error()}"
    if rc in (AIA_ERR_INVALID, AIA_ERR_CAPACITY):
        raise ValueError(msg)
    if rc == AIA_ERR_UNSUPPORTED:
        raise NotImplementedError(msg)
    raise RuntimeError(msg)


_addr = {}


def address(name):
    """Address of an exported entry point, for native callers."""
    a = _addr.get(name)
    if a is None:
        a = _addr[name] = ctypes.cast(getattr(load(), name), ctypes.c_void_p).value
    return a


def call(name, *args):
    check(getattr(load(), name)(*args), name)
