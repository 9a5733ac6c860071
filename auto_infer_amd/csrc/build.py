"""Compile the gfx950 HIP sources into the package's C-ABI shared library.

Usage: ``python -m auto_infer_amd.csrc.build`` (or ``build()`` from Python).
Output: ``auto_infer_amd/_lib/libautoinfer_amd.so``, the packer's host
extension ``auto_infer_amd/_hostpack*.so`` and the bench's HBM probes
``auto_infer_amd/_lib/libaia_probes.so`` (not part of the product ABI).
Always recompiles.
"""
import os
import subprocess
import sys
import sysconfig

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.dirname(HERE)
ROOT = os.path.dirname(PKG)
OUT_DIR = os.path.join(PKG, "_lib")
LIB = os.path.join(OUT_DIR, "libautoinfer_amd.so")
PROBES = os.path.join(OUT_DIR, "libaia_probes.so")
SOURCES = ["core.hip", "kv_write.hip", "paged_attention.hip", "noalloc.hip", "pack.hip", "qk_rope.hip",
           "mtp_compact.hip", "mla_pre.hip"]

HIPCC_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
    "-munsafe-fp-atomics",
    # keep the compiler from emitting packed-fp32 VALU ops
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def hipcc():
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    return os.path.join(rocm, "bin", "hipcc")


HOSTPACK = os.path.join(PKG, "_hostpack" + sysconfig.get_config_var("EXT_SUFFIX"))


def build_hostpack(verbose=False):
    """The packer's native host loop, upload staging and pack launch
    (CPython extension, g++)."""
    tmp = HOSTPACK + ".tmp"
    # links the HIP runtime by SONAME: loaded after torch, it is torch's
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    cmd = ["g++", "-O2", "-std=c++17", "-shared", "-fPIC", "-Wall", "-D__HIP_PLATFORM_AMD__",
           "-I", sysconfig.get_paths()["include"], "-I", os.path.join(rocm, "include"),
           os.path.join(HERE, "hostpack.cpp"), "-o", tmp, "-L", os.path.join(rocm, "lib"),
           "-lamdhip64"]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, HOSTPACK)
    return HOSTPACK


def build(verbose=False):
    build_hostpack(verbose)
    os.makedirs(OUT_DIR, exist_ok=True)
    srcs = [os.path.join(HERE, s) for s in SOURCES]
    tmp = LIB + ".tmp"
    cmd = [hipcc(), *HIPCC_FLAGS, "-I", os.path.join(ROOT, "include"), "-I", HERE,
           *srcs, "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB)
    tmp = PROBES + ".tmp"
    cmd = [hipcc(), *HIPCC_FLAGS, os.path.join(HERE, "probes.hip"), "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, PROBES)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
