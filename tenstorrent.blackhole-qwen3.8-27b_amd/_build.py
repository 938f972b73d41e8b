"""Builds libqwen_mlp.so in-tree with hipcc for gfx950 (one object per source, then one link).

Every build stamps the library with ``source_hash()`` (a digest of the kernel sources and the C
header); ``qmlp_version()`` reports it, and the ctypes loader refuses a library whose stamp is not
the digest of the sources beside it.
"""
import hashlib
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG_DIR, "csrc")
OBJ_DIR = os.path.join(PKG_DIR, "_build")
LIB_NAME = "libqwen_mlp.so"
LIB_PATH = os.path.join(PKG_DIR, LIB_NAME)
SOURCES = ["qmlp_abi.hip", "qmlp_pack.hip", "qmlp_prep.hip", "qmlp_gemv.hip", "qmlp_stream.hip",
           "qmlp_tiled.hip", "qmlp_noalloc.hip"]
ARCH = "gfx950"
INCLUDE_DIR = os.path.join(os.path.dirname(PKG_DIR), "include")


def source_files():
    """The files whose bytes decide the library: csrc/*.hip, csrc/*.h and include/*.h."""
    out = []
    for d, exts in ((CSRC, (".hip", ".h")), (INCLUDE_DIR, (".h",))):
        if os.path.isdir(d):
            out += [os.path.join(d, n) for n in sorted(os.listdir(d)) if n.endswith(exts)]
    return out


def source_hash():
    """sha256 (first 16 hex digits) over the library's sources, each as its name then its bytes."""
    h = hashlib.sha256()
    for path in source_files():
        with open(path, "rb") as f:
            h.update(os.path.basename(path).encode() + b"\0" + f.read() + b"\0")
    return h.hexdigest()[:16]

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    # Keep the compiler from forming packed-fp32 instructions.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _hipcc():
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    return os.path.join(rocm, "bin", "hipcc")


def _compile(src, extra, verbose):
    obj = os.path.join(OBJ_DIR, os.path.splitext(src)[0] + ".o")
    cmd = [_hipcc(), *HIPCC_FLAGS, *extra, "-c", os.path.join(CSRC, src), "-o", obj]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature; drop that noise.
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{err}")
    if err.strip() and verbose:
        print(err, file=sys.stderr)
    return obj


def build_library(verbose=False, extra_flags=()):
    """Compile every source and link LIB_PATH.  Always rebuilds (a build check must compile)."""
    os.makedirs(OBJ_DIR, exist_ok=True)
    srcs = [s for s in SOURCES if os.path.exists(os.path.join(CSRC, s))]
    stamp = [f'-DQMLP_SOURCE_HASH="{source_hash()}"']
    with ThreadPoolExecutor(max_workers=min(len(srcs), 8)) as ex:
        objs = list(ex.map(lambda s: _compile(s, stamp + list(extra_flags), verbose), srcs))
    tmp = LIB_PATH + ".tmp"
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build_library(verbose="-v" in sys.argv))
