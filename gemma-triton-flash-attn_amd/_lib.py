"""ctypes binding of the C ABI declared in include/gfa.h (libgfa.so, built in-tree).

torch is imported first on purpose: both torch's bundled HIP runtime and libgfa.so
carry the SONAME libamdhip64.so.7, so loading libgfa.so after torch makes it bind to the
runtime torch already owns, and torch's hipStream_t handles are valid in our launches.
There is no fallback: if the library is missing or does not load, every entry point
raises.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch  # noqa: F401  (must precede the CDLL load, see module docstring)

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("GFA_LIBRARY", os.path.join(_HERE, "libgfa.so"))

GFA_DTYPE_FP16 = 0
GFA_DTYPE_BF16 = 1
GFA_BWD_DQ = 1
GFA_BWD_DKV = 2

STATUS_NAMES = {
    0: "GFA_OK",
    1: "GFA_ERR_INVALID_ARGUMENT",
    2: "GFA_ERR_UNSUPPORTED",
    3: "GFA_ERR_WORKSPACE",
    4: "GFA_ERR_LAUNCH",
}

# GFA_VERSION of include/gfa.h whose struct layouts FwdArgs / BwdArgs below mirror. A library
# built from other sources reads another prefix of the argument structs (an older one ignores the
# segment, soft-cap and dropout fields), so load() refuses it instead of computing wrong results.
ABI_VERSION = 106

EXPORTED = ("gfa_fwd", "gfa_bwd", "gfa_bwd_noalloc", "gfa_bwd_workspace_size", "gfa_bwd_workspace_bytes",
            "gfa_bwd_ds_limit", "gfa_config", "gfa_last_error", "gfa_version", "gfa_set_runtime_scheduling")
NOALLOC_SCRATCH_BYTES = 64 << 20  # GFA_NOALLOC_SCRATCH_BYTES


class GfaError(RuntimeError):
    """Non-zero status from the native library."""

    def __init__(self, status: int, message: str):
        super().__init__(f"{STATUS_NAMES.get(status, status)}: {message}")
        self.status = status


class Strides(ctypes.Structure):
    _fields_ = [("batch", ctypes.c_int64), ("head", ctypes.c_int64), ("row", ctypes.c_int64)]


class FwdArgs(ctypes.Structure):
    _fields_ = [
        ("q", ctypes.c_void_p), ("k", ctypes.c_void_p), ("v", ctypes.c_void_p),
        ("o", ctypes.c_void_p), ("lse", ctypes.c_void_p),
        ("q_strides", Strides), ("k_strides", Strides), ("v_strides", Strides), ("o_strides", Strides),
        ("batch", ctypes.c_int32), ("heads_q", ctypes.c_int32), ("heads_kv", ctypes.c_int32),
        ("seq_len", ctypes.c_int32), ("head_dim", ctypes.c_int32),
        ("causal", ctypes.c_int32), ("window", ctypes.c_int32), ("scale", ctypes.c_float),
        ("dtype", ctypes.c_int32), ("block_kv", ctypes.c_int32), ("lse_ld", ctypes.c_int32),
        ("stream", ctypes.c_void_p), ("seg_lo", ctypes.c_void_p), ("seg_hi", ctypes.c_void_p),
        ("softcap", ctypes.c_float), ("dropout_p", ctypes.c_float), ("dropout_seed", ctypes.c_uint64),
    ]


class BwdArgs(ctypes.Structure):
    _fields_ = [
        ("q", ctypes.c_void_p), ("k", ctypes.c_void_p), ("v", ctypes.c_void_p),
        ("o", ctypes.c_void_p), ("dout", ctypes.c_void_p),
        ("lse", ctypes.c_void_p), ("delta", ctypes.c_void_p),
        ("dq", ctypes.c_void_p), ("dk", ctypes.c_void_p), ("dv", ctypes.c_void_p),
        ("q_strides", Strides), ("k_strides", Strides), ("v_strides", Strides), ("o_strides", Strides),
        ("do_strides", Strides), ("dq_strides", Strides), ("dk_strides", Strides), ("dv_strides", Strides),
        ("batch", ctypes.c_int32), ("heads_q", ctypes.c_int32), ("heads_kv", ctypes.c_int32),
        ("seq_len", ctypes.c_int32), ("head_dim", ctypes.c_int32),
        ("causal", ctypes.c_int32), ("window", ctypes.c_int32), ("scale", ctypes.c_float),
        ("dtype", ctypes.c_int32), ("q_splits", ctypes.c_int32), ("lse_ld", ctypes.c_int32),
        ("stages", ctypes.c_int32),
        ("workspace", ctypes.c_void_p), ("workspace_bytes", ctypes.c_size_t),
        ("stream", ctypes.c_void_p), ("seg_lo", ctypes.c_void_p), ("seg_hi", ctypes.c_void_p),
        ("softcap", ctypes.c_float), ("dropout_p", ctypes.c_float), ("dropout_seed", ctypes.c_uint64),
    ]


class ConfigInfo(ctypes.Structure):
    _fields_ = [(name, ctypes.c_int32) for name in (
        "head_dim", "fwd_block_q", "fwd_block_kv", "fwd_waves", "dq_block_q", "dq_block_kv", "dq_waves",
        "dkv_block_kv", "dkv_block_q", "dkv_waves", "q_splits")]

    def as_dict(self) -> dict:
        return {name: int(getattr(self, name)) for name, _ in self._fields_}


_lib = None
_lock = threading.Lock()


def load() -> ctypes.CDLL:
    """Load libgfa.so once and declare the prototypes. Raises if it is missing."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"libgfa.so not found at {LIB_PATH}; build it with "
                "`python gemma-triton-flash-attn_amd/build.py` (or __graft_entry__.build())")
        lib = ctypes.CDLL(LIB_PATH)
        lib.gfa_fwd.argtypes = [ctypes.POINTER(FwdArgs)]
        lib.gfa_fwd.restype = ctypes.c_int
        lib.gfa_bwd.argtypes = [ctypes.POINTER(BwdArgs)]
        lib.gfa_bwd.restype = ctypes.c_int
        lib.gfa_bwd_noalloc.argtypes = [ctypes.POINTER(BwdArgs)]
        lib.gfa_bwd_noalloc.restype = ctypes.c_int
        lib.gfa_bwd_workspace_size.argtypes = [ctypes.c_int32] * 8
        lib.gfa_bwd_workspace_size.restype = ctypes.c_size_t
        lib.gfa_bwd_workspace_bytes.argtypes = [ctypes.POINTER(BwdArgs)]
        lib.gfa_bwd_workspace_bytes.restype = ctypes.c_size_t
        lib.gfa_bwd_ds_limit.argtypes = [ctypes.c_int64]
        lib.gfa_bwd_ds_limit.restype = ctypes.c_int64
        lib.gfa_config.argtypes = [ctypes.c_int32] * 5 + [ctypes.POINTER(ConfigInfo)]
        lib.gfa_config.restype = ctypes.c_int
        lib.gfa_last_error.argtypes = []
        lib.gfa_last_error.restype = ctypes.c_char_p
        lib.gfa_version.argtypes = []
        lib.gfa_version.restype = ctypes.c_int
        lib.gfa_set_runtime_scheduling.argtypes = [ctypes.c_int32]
        lib.gfa_set_runtime_scheduling.restype = ctypes.c_int
        built = int(lib.gfa_version())
        if built != ABI_VERSION:
            raise RuntimeError(
                f"{LIB_PATH} reports GFA_VERSION {built}, but this binding mirrors version {ABI_VERSION}; "
                "rebuild it with `python gemma-triton-flash-attn_amd/build.py` (or __graft_entry__.build())")
        _lib = lib
        return lib


def check(status: int) -> None:
    if status != 0:
        msg = load().gfa_last_error().decode(errors="replace")
        raise GfaError(status, msg)


def set_runtime_scheduling(enable: bool) -> bool:
    """Switch the run-time work distribution of the head_dim-512 grids on or off (process-wide;
    results are bitwise the same either way). Returns the previous setting."""
    return bool(load().gfa_set_runtime_scheduling(1 if enable else 0))


def set_bwd_ds_limit(nbytes: int) -> int:
    """Largest dS store (bytes) the materialised backward may use; 0 switches that form off.
    Process-wide; returns the previous limit."""
    return int(load().gfa_bwd_ds_limit(int(nbytes)))


def bwd_ds_limit() -> int:
    return int(load().gfa_bwd_ds_limit(-1))


def strides_of(t) -> Strides:
    s = t.stride()
    return Strides(s[0], s[1], s[2])


def config(batch: int, heads_q: int, heads_kv: int, seq_len: int, head_dim: int) -> dict:
    info = ConfigInfo()
    check(load().gfa_config(batch, heads_q, heads_kv, seq_len, head_dim, ctypes.byref(info)))
    return info.as_dict()


def bwd_workspace_size(batch, heads_q, heads_kv, seq_len, head_dim, causal, window, q_splits=0) -> int:
    return int(load().gfa_bwd_workspace_size(batch, heads_q, heads_kv, seq_len, head_dim, int(causal), window,
                                             q_splits))
