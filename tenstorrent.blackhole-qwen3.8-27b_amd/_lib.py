"""ctypes binding of libqwen_mlp.so (the C ABI in include/qwen_mlp.h).

The library is built in-tree by ``_build.py``.  There is no fallback: if the shared library is
missing, every entry point raises, and so does a library whose source stamp (``qmlp_version()``)
is not the digest of the sources beside it (a binary built from other sources).
"""
import ctypes
import importlib.util
import os

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG_DIR, "libqwen_mlp.so")

FMT_BF16 = 0
FMT_BFP8 = 1
FMT_BF4 = 2
FORMATS = {"bf16": FMT_BF16, "bfp8": FMT_BFP8, "bf4": FMT_BF4}

QMLP_OK = 0
OUT_F32 = 1
RESIDUAL_F32 = 2
WS_COUNTER_BYTES = 524288  # QMLP_WS_COUNTER_BYTES
SCRATCH_BYTES = 33554432  # QMLP_SCRATCH_BYTES
E_SHAPE, E_ALIGN, E_FORMAT, E_LAUNCH, E_WORKSPACE, E_NULL, E_DEVICE = -1, -2, -3, -4, -5, -6, -7
_VALUE_ERRORS = {E_SHAPE, E_ALIGN, E_FORMAT, E_WORKSPACE, E_NULL}

# name -> (restype, argtypes); mirrors include/qwen_mlp.h
_P, _I, _SZ, _U32P, _DP = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_void_p
SIGNATURES = {
    "qmlp_last_error": (ctypes.c_char_p, []),
    "qmlp_version": (ctypes.c_char_p, []),
    "qmlp_quantize_bfp8": (_I, [_P, _I, _I, _P, _P, _U32P, _P]),
    "qmlp_quantize_bf4": (_I, [_P, _I, _I, _P, _P, _U32P, _P]),
    "qmlp_packed_bytes": (_SZ, [_I, _I, _I]),
    "qmlp_pack": (_I, [_P, _P, _I, _I, _I, _P, _SZ, _P]),
    "qmlp_packed_info": (_I, [_P, _I, _I, _I, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_uint32), _P]),
    "qmlp_unpack_bfp8": (_I, [_P, _I, _I, _P, _P, _P]),
    "qmlp_unpack_bf4": (_I, [_P, _I, _I, _P, _P, _P]),
    "qmlp_dequant_packed": (_I, [_P, _I, _I, _I, _P, _P]),
    "qmlp_forward": (_I, [_P, _P, _P, _P, _P, _P, _P, _SZ, _I, _I, _I, _I, _P]),
    "qmlp_forward_ex": (_I, [_P, _P, _P, _P, _P, _P, _P, _SZ, _I, _I, _I, _I, _I, _P]),
    "qmlp_workspace_bytes": (_SZ, [_I, _I, _I, _I]),
    "qmlp_workspace_init": (_I, [_P, _SZ, _P]),
    "qmlp_plan_stream": (_I, [_I, _I, _I, ctypes.POINTER(ctypes.c_int)]),
    "qmlp_set_profile_events": (_I, [_P, _I]),
    "qmlp_plan_split": (_I, [_I, _I, _I, _I, _I, ctypes.POINTER(ctypes.c_int)]),
    "qmlp_forward_rmsnorm": (_I, [_P, _P, ctypes.c_float, _P, _P, _P, _P, _P, _SZ, _I, _I, _I, _I, _I, _P]),
    "qmlp_forward_noalloc": (_I, [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _P]),
}

_lib = None


class QmlpError(RuntimeError):
    """A library call failed at run time (launch or device error)."""

    def __init__(self, code, message):
        super().__init__(f"qwen_mlp error {code}: {message}")
        self.code = code


def _build_module():
    spec = importlib.util.spec_from_file_location("_qmlp_build", os.path.join(PKG_DIR, "_build.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def tree_source_hash():
    """Digest of the kernel sources in this tree (what a build now would stamp)."""
    return _build_module().source_hash()


def library_source_hash(handle=None):
    """The source digest stamped into the loaded library ("unstamped" if it has none)."""
    version = (handle or lib()).qmlp_version().decode()
    return version.rsplit("src=", 1)[1] if "src=" in version else "unstamped"


def lib():
    """Load libqwen_mlp.so (raises if it has not been built, or was built from other sources)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it with __graft_entry__.build()")
        handle = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        built, tree = library_source_hash(handle), tree_source_hash()
        if built != tree:
            raise RuntimeError(f"{LIB_PATH} was built from other sources (library src={built}, tree src={tree}): "
                               "rebuild it with __graft_entry__.build()")
        _lib = handle
    return _lib


def last_error():
    return lib().qmlp_last_error().decode()


def check(rc, what):
    """Raise ValueError for argument errors, QmlpError for run-time errors."""
    if rc == QMLP_OK:
        return
    msg = last_error()
    if rc in _VALUE_ERRORS:
        raise ValueError(f"{what}: {msg} (code {rc})")
    raise QmlpError(rc, f"{what}: {msg}")


def ptr(t):
    """Device pointer of a torch tensor (None -> null)."""
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream_handle(stream=None):
    import torch

    s = stream if stream is not None else torch.cuda.current_stream()
    return ctypes.c_void_p(s.cuda_stream)
