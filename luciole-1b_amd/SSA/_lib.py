"""ctypes binding of libssa_mi355x.so (declared in include/ssa_mi355x.h).

The library is built in-tree by ``SSA/_build.py`` (``__graft_entry__.build()``).
If it is missing, ``lib()`` raises: there is no CPU or PyTorch fallback.
"""

from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

# SSA_MI355X_LIB overrides the library path (e.g. to compare two builds).
LIB_PATH = Path(os.environ.get("SSA_MI355X_LIB", str(Path(__file__).resolve().parent / "libssa_mi355x.so")))

SSA_OK = 0
SSA_ERR_NULL_POINTER = 1
SSA_ERR_SHAPE = 2
SSA_ERR_HEAD_DIM = 3
SSA_ERR_DTYPE = 4
SSA_ERR_ALIGNMENT = 5
SSA_ERR_LAUNCH = 6
SSA_ERR_CU_SEQLENS = 7
SSA_ERR_SCRATCH = 8

SSA_DTYPE_BF16 = 0
SSA_DTYPE_FP16 = 1
SSA_DTYPE_FP32 = 2

# Every exported symbol of include/ssa_mi355x.h.
EXPORTED_SYMBOLS = (
    "ssa_abi_version",
    "ssa_status_string",
    "ssa_bwd_partials_count",
    "ssa_bwd_ds_workspace_bytes",
    "ssa_fwd",
    "ssa_bwd",
    "ssa_bwd_preprocess",
    "ssa_bwd_dkdv",
    "ssa_bwd_dq",
    "ssa_bwd_reduce",
    "ssa_bwd_noalloc",
    "ssa_varlen_fwd",
    "ssa_varlen_bwd",
    "ssa_varlen_bwd_ds_workspace_bytes",
    "ssa_decode_num_splits",
    "ssa_decode_workspace_bytes",
    "ssa_decode",
    "ssa_rope",  # include/ssa_decoder_ops.h
    "ssa_rmsnorm_workspace_floats",
    "ssa_rmsnorm_fwd",
    "ssa_rmsnorm_bwd",
    "ssa_swiglu",
    "ssa_cross_entropy",
)

ABI_VERSION = 6


class Tensor4(ctypes.Structure):
    _fields_ = [
        ("ptr", ctypes.c_void_p),
        ("stride_b", ctypes.c_int64),
        ("stride_h", ctypes.c_int64),
        ("stride_s", ctypes.c_int64),
    ]


class FwdArgs(ctypes.Structure):
    _fields_ = [
        ("q", Tensor4),
        ("k", Tensor4),
        ("v", Tensor4),
        ("out", Tensor4),
        ("m", ctypes.c_void_p),
        ("ssa_n", ctypes.c_void_p),
        ("ssa_b", ctypes.c_void_p),
        ("batch", ctypes.c_int32),
        ("heads_q", ctypes.c_int32),
        ("heads_kv", ctypes.c_int32),
        ("seqlen", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("dtype", ctypes.c_int32),
        ("causal", ctypes.c_int32),
        ("softmax_scale", ctypes.c_float),
    ]


class BwdArgs(ctypes.Structure):
    _fields_ = [
        ("q", Tensor4),
        ("k", Tensor4),
        ("v", Tensor4),
        ("out", Tensor4),
        ("dout", Tensor4),
        ("dq", Tensor4),
        ("dk", Tensor4),
        ("dv", Tensor4),
        ("m", ctypes.c_void_p),
        ("delta", ctypes.c_void_p),
        ("partials", ctypes.c_void_p),
        ("dn", ctypes.c_void_p),
        ("db", ctypes.c_void_p),
        ("ssa_n", ctypes.c_void_p),
        ("ssa_b", ctypes.c_void_p),
        ("batch", ctypes.c_int32),
        ("heads_q", ctypes.c_int32),
        ("heads_kv", ctypes.c_int32),
        ("seqlen", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("dtype", ctypes.c_int32),
        ("causal", ctypes.c_int32),
        ("softmax_scale", ctypes.c_float),
        ("ds_workspace", ctypes.c_void_p),
    ]


class RopeArgs(ctypes.Structure):
    """ssa_rope_args of include/ssa_decoder_ops.h."""

    _fields_ = [
        ("x", ctypes.c_void_p),
        ("x_stride_s", ctypes.c_int64),
        ("x_stride_b", ctypes.c_int64),
        ("x_stride_h", ctypes.c_int64),
        ("y", ctypes.c_void_p),
        ("cos", ctypes.c_void_p),
        ("sin", ctypes.c_void_p),
        ("seqlen", ctypes.c_int32),
        ("batch", ctypes.c_int32),
        ("heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("dtype", ctypes.c_int32),
        ("inverse", ctypes.c_int32),
    ]


class RmsNormFwdArgs(ctypes.Structure):
    """ssa_rmsnorm_fwd_args of include/ssa_decoder_ops.h."""

    _fields_ = [
        ("x", ctypes.c_void_p),
        ("weight", ctypes.c_void_p),
        ("y", ctypes.c_void_p),
        ("rstd", ctypes.c_void_p),
        ("rows", ctypes.c_int32),
        ("hidden", ctypes.c_int32),
        ("out_dtype", ctypes.c_int32),
        ("eps", ctypes.c_float),
    ]


class RmsNormBwdArgs(ctypes.Structure):
    """ssa_rmsnorm_bwd_args of include/ssa_decoder_ops.h."""

    _fields_ = [
        ("x", ctypes.c_void_p),
        ("weight", ctypes.c_void_p),
        ("dy", ctypes.c_void_p),
        ("rstd", ctypes.c_void_p),
        ("dx", ctypes.c_void_p),
        ("dweight", ctypes.c_void_p),
        ("workspace", ctypes.c_void_p),
        ("rows", ctypes.c_int32),
        ("hidden", ctypes.c_int32),
        ("dy_dtype", ctypes.c_int32),
    ]


class SwigluArgs(ctypes.Structure):
    """ssa_swiglu_args of include/ssa_decoder_ops.h."""

    _fields_ = [
        ("z", ctypes.c_void_p),
        ("dh", ctypes.c_void_p),
        ("out", ctypes.c_void_p),
        ("rows", ctypes.c_int32),
        ("ffn", ctypes.c_int32),
        ("dtype", ctypes.c_int32),
        ("backward", ctypes.c_int32),
    ]


class CrossEntropyArgs(ctypes.Structure):
    """ssa_cross_entropy_args of include/ssa_decoder_ops.h."""

    _fields_ = [
        ("logits", ctypes.c_void_p),
        ("labels", ctypes.c_void_p),
        ("loss", ctypes.c_void_p),
        ("lse", ctypes.c_void_p),
        ("scale", ctypes.c_void_p),
        ("dlogits", ctypes.c_void_p),
        ("rows", ctypes.c_int32),
        ("vocab", ctypes.c_int32),
        ("dtype", ctypes.c_int32),
        ("backward", ctypes.c_int32),
    ]


class VarlenFwdArgs(ctypes.Structure):
    _fields_ = [("dense", FwdArgs), ("cu_seqlens", ctypes.c_void_p), ("total_tokens", ctypes.c_int32)]


class VarlenBwdArgs(ctypes.Structure):
    _fields_ = [("dense", BwdArgs), ("cu_seqlens", ctypes.c_void_p), ("total_tokens", ctypes.c_int32)]


class DecodeArgs(ctypes.Structure):
    _fields_ = [
        ("q", Tensor4),
        ("k_cache", Tensor4),
        ("v_cache", Tensor4),
        ("out", Tensor4),
        ("m", ctypes.c_void_p),
        ("cache_seqlens", ctypes.c_void_p),
        ("ssa_n", ctypes.c_void_p),
        ("ssa_b", ctypes.c_void_p),
        ("batch", ctypes.c_int32),
        ("heads_q", ctypes.c_int32),
        ("heads_kv", ctypes.c_int32),
        ("capacity", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("dtype", ctypes.c_int32),
        ("num_splits", ctypes.c_int32),
        ("softmax_scale", ctypes.c_float),
        ("workspace", ctypes.c_void_p),
    ]


_lock = threading.Lock()
_lib = None


def _declare(lib: ctypes.CDLL) -> None:
    lib.ssa_abi_version.restype = ctypes.c_int32
    lib.ssa_abi_version.argtypes = []
    lib.ssa_status_string.restype = ctypes.c_char_p
    lib.ssa_status_string.argtypes = [ctypes.c_int32]
    lib.ssa_bwd_partials_count.restype = ctypes.c_int64
    lib.ssa_bwd_partials_count.argtypes = [ctypes.c_int32, ctypes.c_int32, ctypes.c_int32]
    lib.ssa_bwd_ds_workspace_bytes.restype = ctypes.c_int64
    lib.ssa_bwd_ds_workspace_bytes.argtypes = [ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32]
    lib.ssa_varlen_bwd_ds_workspace_bytes.restype = ctypes.c_int64
    lib.ssa_varlen_bwd_ds_workspace_bytes.argtypes = [ctypes.c_int32] * 5
    for name, argt in (("ssa_fwd", FwdArgs), ("ssa_bwd", BwdArgs), ("ssa_bwd_preprocess", BwdArgs),
                       ("ssa_bwd_dkdv", BwdArgs), ("ssa_bwd_dq", BwdArgs), ("ssa_bwd_reduce", BwdArgs),
                       ("ssa_bwd_noalloc", BwdArgs)):
        fn = getattr(lib, name)
        fn.restype = ctypes.c_int32
        fn.argtypes = [ctypes.POINTER(argt), ctypes.c_void_p]
    for name, argt in (("ssa_varlen_fwd", VarlenFwdArgs), ("ssa_varlen_bwd", VarlenBwdArgs),
                       ("ssa_decode", DecodeArgs), ("ssa_rope", RopeArgs), ("ssa_rmsnorm_fwd", RmsNormFwdArgs),
                       ("ssa_rmsnorm_bwd", RmsNormBwdArgs), ("ssa_swiglu", SwigluArgs),
                       ("ssa_cross_entropy", CrossEntropyArgs)):
        fn = getattr(lib, name)
        fn.restype = ctypes.c_int32
        fn.argtypes = [ctypes.POINTER(argt), ctypes.c_void_p]
    i32 = ctypes.c_int32
    lib.ssa_decode_num_splits.restype = ctypes.c_int32
    lib.ssa_decode_num_splits.argtypes = [i32, i32, i32, i32, i32]
    lib.ssa_rmsnorm_workspace_floats.restype = ctypes.c_int64
    lib.ssa_rmsnorm_workspace_floats.argtypes = [i32, i32]
    lib.ssa_decode_workspace_bytes.restype = ctypes.c_int64
    lib.ssa_decode_workspace_bytes.argtypes = [i32, i32, i32, i32, i32, i32]


def lib() -> ctypes.CDLL:
    """Load (once) and return the library; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"SSA HIP library not found at {LIB_PATH}; build it with "
                    "`python luciole-1b_amd/SSA/_build.py` (or __graft_entry__.build())."
                )
            handle = ctypes.CDLL(str(LIB_PATH))
            _declare(handle)
            ver = handle.ssa_abi_version()
            if ver != ABI_VERSION:
                raise RuntimeError(f"libssa_mi355x ABI version {ver}, expected {ABI_VERSION}")
            _lib = handle
    return _lib


def status_text(status: int) -> str:
    return lib().ssa_status_string(int(status)).decode()


def check(status: int, what: str) -> None:
    """Map a library status to a Python exception."""
    if status == SSA_OK:
        return
    msg = f"{what}: {status_text(status)} (status {status})"
    if status in (SSA_ERR_SHAPE, SSA_ERR_HEAD_DIM, SSA_ERR_DTYPE, SSA_ERR_ALIGNMENT, SSA_ERR_CU_SEQLENS,
                  SSA_ERR_SCRATCH):
        raise ValueError(msg)
    raise RuntimeError(msg)
