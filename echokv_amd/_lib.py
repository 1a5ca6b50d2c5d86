"""ctypes binding of ``libechokv.so`` (the C ABI in ``include/echokv.h``).

Python passes raw device pointers, element strides, the layout struct and the
current HIP stream; every call returns an error code that becomes an
exception here. There is no other implementation to fall back to: without
the built library (``python -m echokv_amd.build``) every device entry point
raises.
"""

from __future__ import annotations

import ctypes as C
from ctypes import byref  # noqa: F401  (re-exported for callers)
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "libechokv.so"

F32, F16, BF16 = 0, 1, 2
DECODE_BATCH_INVARIANT = 1
DTYPES = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16}

EXPORTS = (
    "echokv_error_string", "echokv_write_tokens", "echokv_finalize_k", "echokv_write_step", "echokv_seal_groups",
    "echokv_gather", "echokv_write_headers",
    "echokv_store_blocks", "echokv_decode", "echokv_decode_static", "echokv_prefill", "echokv_prefill_dense",
    "echokv_prefill_dense_workspace", "echokv_prefill_own_group",
    "echokv_dequant_dense", "echokv_canary_kl", "echokv_decode_workspace_rows",
)


class Layout(C.Structure):
    _fields_ = [
        ("num_kv_heads", C.c_int32), ("head_size", C.c_int32), ("block_size", C.c_int32),
        ("k_group", C.c_int32), ("v_group", C.c_int32), ("chunks_per_page", C.c_int32),
        ("num_blocks", C.c_int64), ("page_stride", C.c_int64),
        ("o_v_scale", C.c_int64), ("o_v_min", C.c_int64), ("o_k_scale", C.c_int64), ("o_k_min", C.c_int64),
        ("o_data", C.c_int64), ("chunk_bytes", C.c_int64),
    ]


class Residual(C.Structure):
    _fields_ = [
        ("ptr", C.c_void_p), ("dtype", C.c_int32), ("rows", C.c_int32),
        ("s0", C.c_int64), ("s1", C.c_int64), ("s2", C.c_int64),
    ]


P = C.c_void_p
I32, I64, FL = C.c_int32, C.c_int64, C.c_float
LP, RP = C.POINTER(Layout), C.POINTER(Residual)

_SIGS = {
    "echokv_write_tokens": [LP, P, P, I64, I64, P, I64, I64, I32, P, I64, I64, RP, P, I64, I64, P],
    "echokv_finalize_k": [LP, P, P, I64, I64, I32, P, P, I64, RP, P],
    "echokv_write_step": [LP, P, P, I64, I64, P, I64, I64, I32, P, I64, I64, P, P, I64, RP, P, I64, I64, P],
    "echokv_seal_groups": [LP, P, P, I64, RP, P],
    "echokv_gather": [LP, P, P, P, RP, P, P, I64, P, P, P],
    "echokv_write_headers": [P, I32, I64, P, I64, P, P],
    "echokv_store_blocks": [LP, P, P, I64, P, P, I32, P],
    "echokv_decode": [LP, P, P, P, RP, P, I64, I64, I32, I32, P, P, I64, P, P, I64, FL, I32, I32, I32, P, I32, P, P,
                      P, I64, I64, I32, P],
    "echokv_decode_static": [LP, P, P, P, RP, P, I64, I64, I32, I32, P, P, I64, P, P, I64, FL, I32, I32, I32, P, I32,
                             P, I64, I64, I32, P],
    "echokv_prefill": [LP, P, P, P, RP, P, I64, I64, I32, I32, P, I64, I64, I32, P, I64, I32, P, I64, FL, I32, P, P],
    "echokv_prefill_own_group": [LP, P, P, P, RP, P, I64, I64, I32, I32, P, I64, I64, I32, P, I64, P, I64, P, I64, I64,
                                 P, P, I64, I64, I32, FL, P],
    "echokv_prefill_dense": [LP, P, P, P, RP, P, I64, I64, I32, I32, P, I64, I64, I32, P, I64, P, I64, I32, P, I64,
                             P, I64, FL, I32, P, P],
    "echokv_dequant_dense": [LP, P, P, P, RP, P, I64, P, I64, P, P, I64, I64, I32, P],
    "echokv_canary_kl": [P, I32, I64, I64, I64, P, I64, I64, I64, I32, I32, I32, I32, I32, I32, I32, I32, I32, FL, P, P,
                         P],
}

_lib = None


def lib() -> C.CDLL:
    """The loaded library; raises if it was not built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build the HIP extension first (python -m echokv_amd.build)"
            )
        l = C.CDLL(str(LIB_PATH))
        l.echokv_error_string.restype = C.c_char_p
        l.echokv_error_string.argtypes = [C.c_int]
        for name, args in _SIGS.items():
            fn = getattr(l, name)
            fn.argtypes = args
            fn.restype = C.c_int
        l.echokv_prefill_dense_workspace.argtypes = [LP, I64]
        l.echokv_prefill_dense_workspace.restype = C.c_int64
        l.echokv_decode_workspace_rows.argtypes = [LP, I32, I32, I64, I32, I32]
        l.echokv_decode_workspace_rows.restype = C.c_int64
        _lib = l
    return _lib


def call(name: str, *args) -> None:
    rc = getattr(lib(), name)(*args)
    if rc != 0:
        msg = lib().echokv_error_string(rc).decode()
        raise RuntimeError(f"{name}: {msg} (code {rc})")


def dtype_code(t: torch.Tensor) -> int:
    try:
        return DTYPES[t.dtype]
    except KeyError:
        raise RuntimeError(f"unsupported dtype {t.dtype}") from None


def ptr(t: torch.Tensor | None):
    return None if t is None else t.data_ptr()


def stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def require_device(*ts: torch.Tensor) -> None:
    """The kernels run on the GPU only; CPU tensors are an error, never a fallback."""
    for t in ts:
        if t is not None and t.device.type != "cuda":
            raise RuntimeError(f"EchoKV kernels need device tensors, got a {t.device} tensor")


def residual(res: torch.Tensor) -> Residual:
    if res.stride(3) != 1:
        raise ValueError("residual rows must be contiguous along head_dim")
    return Residual(res.data_ptr(), dtype_code(res), res.shape[0], res.stride(0), res.stride(1), res.stride(2))
