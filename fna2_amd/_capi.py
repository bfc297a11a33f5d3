"""ctypes binding of the C ABI in ``include/fna2.h`` (``libfna2_hip.so``).

This is the Python-side binding of the drop-in boundary: the launchers in
``flash_naylis_attn.py`` fill the argument structs from torch tensors (device
pointers, element strides, sizes) and call ``fna2_fwd`` / ``fna2_bwd`` on
torch's current HIP stream.  torch only provides memory and the stream.

There is no fallback: if the library is missing, ``lib()`` raises.
"""
from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

LIB_PATH = Path(os.environ.get("FNA2_LIB", Path(__file__).resolve().parent / "libfna2_hip.so"))

FNA2_BF16 = 1
FNA2_F16 = 2
FNA2_F32 = 3

STATUS = {
    0: "FNA2_OK",
    -1: "FNA2_E_NULL",
    -2: "FNA2_E_DTYPE",
    -3: "FNA2_E_HEAD_DIM",
    -4: "FNA2_E_RANK",
    -5: "FNA2_E_HEADS",
    -6: "FNA2_E_SHAPE",
    -7: "FNA2_E_STRIDE",
    -8: "FNA2_E_SEQLENS",
    -9: "FNA2_E_WORKSPACE",
    -10: "FNA2_E_LAUNCH",
    -11: "FNA2_E_DEVICE",
    -12: "FNA2_E_SCALE",
    -13: "FNA2_E_ALIAS",
    -14: "FNA2_E_SCRATCH",
}
# Contract violations surface as AssertionError, like the reference's asserts
# (FNA2/flash_naylis_attn.py:718-720, :778, :1419-1427); the rest as RuntimeError.
_ASSERT_CODES = {-1, -2, -3, -4, -5, -6, -7, -8, -12, -13}


class Tensor(ctypes.Structure):
    _fields_ = [
        ("ptr", ctypes.c_void_p),
        ("stride_b", ctypes.c_int64),
        ("stride_s", ctypes.c_int64),
        ("stride_h", ctypes.c_int64),
    ]


class Problem(ctypes.Structure):
    _fields_ = [
        ("dtype", ctypes.c_int32),
        ("varlen", ctypes.c_int32),
        ("batch", ctypes.c_int32),
        ("seqlen_q", ctypes.c_int32),
        ("seqlen_k", ctypes.c_int32),
        ("total_q", ctypes.c_int32),
        ("total_k", ctypes.c_int32),
        ("heads", ctypes.c_int32),
        ("heads_kv", ctypes.c_int32),
        ("heads_graph", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("rank", ctypes.c_int32),
        ("causal", ctypes.c_int32),
        ("softmax_scale", ctypes.c_float),
        ("cu_seqlens_q", ctypes.c_void_p),
        ("cu_seqlens_k", ctypes.c_void_p),
    ]


class FwdArgs(ctypes.Structure):
    _fields_ = [
        ("p", Problem),
        ("q", Tensor),
        ("k", Tensor),
        ("v", Tensor),
        ("r_q", Tensor),
        ("r_k", Tensor),
        ("graph_scale", ctypes.c_void_p),
        ("out", Tensor),
        ("lse", Tensor),
        ("workspace", ctypes.c_void_p),
        ("workspace_bytes", ctypes.c_size_t),
        ("events", ctypes.c_void_p),
        ("plan", ctypes.c_void_p),
        ("plan_bytes", ctypes.c_size_t),
        ("plan_filled", ctypes.c_int32),
    ]


FWD_EVENTS = 2
BWD_EVENTS = 4
DECODE_EVENTS = 2


class BwdArgs(ctypes.Structure):
    _fields_ = [
        ("p", Problem),
        ("q", Tensor),
        ("k", Tensor),
        ("v", Tensor),
        ("r_q", Tensor),
        ("r_k", Tensor),
        ("graph_scale", ctypes.c_void_p),
        ("out", Tensor),
        ("lse", Tensor),
        ("dout", Tensor),
        ("delta", Tensor),
        ("dq", Tensor),
        ("dk", Tensor),
        ("dv", Tensor),
        ("dr_q", Tensor),
        ("dr_k", Tensor),
        ("d_graph_scale", ctypes.c_void_p),
        ("workspace", ctypes.c_void_p),
        ("workspace_bytes", ctypes.c_size_t),
        ("events", ctypes.c_void_p),
        ("plan", ctypes.c_void_p),
        ("plan_bytes", ctypes.c_size_t),
    ]


class RopeArgs(ctypes.Structure):
    _fields_ = [
        ("dtype", ctypes.c_int32),
        ("total_tokens", ctypes.c_int32),
        ("heads_q", ctypes.c_int32),
        ("heads_k", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("nseq", ctypes.c_int32),
        ("sign", ctypes.c_int32),
        ("cu_seqlens", ctypes.c_void_p),
        ("inv_freq", ctypes.c_void_p),
        ("q", Tensor),
        ("k", Tensor),
        ("q_out", Tensor),
        ("k_out", Tensor),
        ("norm_q", ctypes.c_void_p),
        ("norm_k", ctypes.c_void_p),
        ("norm_eps", ctypes.c_float),
    ]


class RopeBwdArgs(ctypes.Structure):
    _fields_ = [
        ("fwd", RopeArgs),
        ("dq_out", Tensor),
        ("dk_out", Tensor),
        ("dq", Tensor),
        ("dk", Tensor),
        ("dnorm_q", ctypes.c_void_p),
        ("dnorm_k", ctypes.c_void_p),
        ("workspace", ctypes.c_void_p),
        ("workspace_bytes", ctypes.c_size_t),
    ]


class DecodeArgs(ctypes.Structure):
    _fields_ = [
        ("batch", ctypes.c_int32),
        ("heads", ctypes.c_int32),
        ("heads_kv", ctypes.c_int32),
        ("heads_graph", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("rank", ctypes.c_int32),
        ("max_seqlen_k", ctypes.c_int32),
        ("num_splits", ctypes.c_int32),
        ("softmax_scale", ctypes.c_float),
        ("seqlens_k", ctypes.c_void_p),
        ("q", Tensor),
        ("r_q", Tensor),
        ("k_cache", Tensor),
        ("v_cache", Tensor),
        ("rk_cache", Tensor),
        ("graph_scale", ctypes.c_void_p),
        ("out", Tensor),
        ("lse", Tensor),
        ("workspace", ctypes.c_void_p),
        ("workspace_bytes", ctypes.c_size_t),
        ("events", ctypes.c_void_p),
    ]


# Every symbol the header declares, with its ctypes signature.
SIGNATURES = {
    "fna2_version": (ctypes.c_int, []),
    "fna2_status_string": (ctypes.c_char_p, [ctypes.c_int]),
    "fna2_check_fwd": (ctypes.c_int, [ctypes.POINTER(FwdArgs)]),
    "fna2_check_bwd": (ctypes.c_int, [ctypes.POINTER(BwdArgs)]),
    "fna2_fwd_workspace_bytes": (ctypes.c_size_t, [ctypes.POINTER(Problem)]),
    "fna2_bwd_workspace_bytes": (ctypes.c_size_t, [ctypes.POINTER(Problem)]),
    "fna2_plan_bytes": (ctypes.c_size_t, [ctypes.POINTER(Problem)]),
    "fna2_fwd": (ctypes.c_int, [ctypes.POINTER(FwdArgs), ctypes.c_void_p]),
    "fna2_fwd_noalloc": (ctypes.c_int, [ctypes.POINTER(FwdArgs), ctypes.c_void_p]),
    "fna2_fwd_noalloc_max_bytes": (ctypes.c_size_t, []),
    "fna2_bwd": (ctypes.c_int, [ctypes.POINTER(BwdArgs), ctypes.c_void_p]),
    "fna2_check_rope": (ctypes.c_int, [ctypes.POINTER(RopeArgs)]),
    "fna2_rope_varlen": (ctypes.c_int, [ctypes.POINTER(RopeArgs), ctypes.c_void_p]),
    "fna2_rope_bwd_workspace_bytes": (ctypes.c_size_t, [ctypes.POINTER(RopeArgs)]),
    "fna2_check_rope_bwd": (ctypes.c_int, [ctypes.POINTER(RopeBwdArgs)]),
    "fna2_rope_bwd": (ctypes.c_int, [ctypes.POINTER(RopeBwdArgs), ctypes.c_void_p]),
    "fna2_check_decode": (ctypes.c_int, [ctypes.POINTER(DecodeArgs)]),
    "fna2_decode_num_splits": (ctypes.c_int, [ctypes.POINTER(DecodeArgs)]),
    "fna2_decode_workspace_bytes": (ctypes.c_size_t, [ctypes.POINTER(DecodeArgs)]),
    "fna2_decode": (ctypes.c_int, [ctypes.POINTER(DecodeArgs), ctypes.c_void_p]),
}

_lib = None
_lock = threading.Lock()


def lib() -> ctypes.CDLL:
    """Load ``libfna2_hip.so`` (once).  Raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"FNA2 HIP library not found at {LIB_PATH}; build it with "
                    "`python -m fna2_amd.build` (hipcc, gfx950)")
            handle = ctypes.CDLL(str(LIB_PATH))
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype = res
                fn.argtypes = args
            _lib = handle
    return _lib


def available() -> bool:
    try:
        lib()
        return True
    except (RuntimeError, OSError):
        return False


class FNA2Error(RuntimeError):
    pass


def raise_for(status: int, what: str) -> None:
    if status == 0:
        return
    name = STATUS.get(status, str(status))
    msg = f"{what}: {name}: {lib().fna2_status_string(status).decode()}"
    if status in _ASSERT_CODES:
        raise AssertionError(msg)
    raise FNA2Error(msg)


def empty_tensor() -> Tensor:
    return Tensor(None, 0, 0, 0)
