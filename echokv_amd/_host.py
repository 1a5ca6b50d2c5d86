"""ctypes binding of ``libechokv_host.so``: the native host planner and chunk pools
(``include/echokv_host.h``, ``echokv_amd/host/plan.cpp``). CPU only; built with g++ by
``echokv_amd.build``. There is no Python fallback: without the library the store's
host side raises."""

from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

LIB_PATH = Path(__file__).resolve().parent / "libechokv_host.so"

OK, EINVAL, ESLOTS = 0, 1, 2
STEP, RES_FREE, RES_SLOTS, KREF_POS, KREF_FILL, KREF_WINDOW, NUM_BLOCKS = range(7)
FILL, LAST, CUM = range(3)

EXPORTS = (
    "ekh_planner_new", "ekh_planner_free", "ekh_plan", "ekh_commit", "ekh_planner_state", "ekh_residual_free_list",
    "ekh_sealed_mask", "ekh_block_array", "ekh_pool_new", "ekh_pool_free", "ekh_pool_open", "ekh_pool_seal_row",
    "ekh_pool_counters", "ekh_pool_reset_counters", "ekh_pool_tags", "ekh_pool_free_list", "ekh_pool_live",
    "ekh_stepper_new", "ekh_stepper_free", "ekh_stepper_run", "ekh_host_slots",
)


class PlanView(C.Structure):
    _fields_ = [(n, C.c_int64) for n in ("step", "n_rows", "n_fin", "n_evict", "n_open", "n_touched", "n_res_map",
                                         "n_grp_map", "stage_len")] + [
        ("stage", C.POINTER(C.c_int64)), ("evict", C.POINTER(C.c_int64)), ("open", C.POINTER(C.c_int64)),
        ("touched", C.POINTER(C.c_int64))]


class Batch(C.Structure):
    """``ekh_batch``: one step's batch (pointers to int32 query starts / lengths, int64 slots)."""

    _fields_ = [("num_reqs", C.c_int64), ("num_tokens", C.c_int64), ("query_start", C.c_void_p),
                ("seq_lens", C.c_void_p), ("slot_mapping", C.c_void_p)]


_STEP_WORDS = ("step", "len", "o_canary", "o_mask", "o_dec", "o_tok", "o_fin", "o_res", "o_grp", "o_open", "o_hdr", "o_seal",
               "rows_dec", "rows_tok", "rows_fin", "n_dec", "n_tokens", "n_fin", "n_res", "n_grp", "n_open",
               "n_seal", "n_canary", "decode_only", "graph_rows")


class StepView(C.Structure):
    """``ekh_step_view``: where each part of a step image sits."""

    _fields_ = [(n, C.c_int64) for n in _STEP_WORDS] + [
        ("canary_ctx", C.c_double), ("n_prefill", C.c_int64), ("prefill", C.POINTER(C.c_int64)),
        ("n_victims", C.c_int64), ("victims", C.POINTER(C.c_int64)), ("image", C.POINTER(C.c_int64))]


P, I32, I64, PI64, PU8 = C.c_void_p, C.c_int32, C.c_int64, C.POINTER(C.c_int64), C.POINTER(C.c_uint8)
_SIGS = {
    "ekh_planner_new": ([I64, I32, I32, I32, I32], P),
    "ekh_planner_free": ([P], None),
    "ekh_plan": ([P, PI64, I64, C.POINTER(PlanView)], C.c_int),
    "ekh_commit": ([P, I64, PI64, I64], C.c_int),
    "ekh_planner_state": ([P, I32], I64),
    "ekh_residual_free_list": ([P, PI64, I64], I64),
    "ekh_sealed_mask": ([P, I64], I32),
    "ekh_block_array": ([P, I32], PI64),
    "ekh_pool_new": ([P, I32], P),
    "ekh_pool_free": ([P], None),
    "ekh_pool_open": ([P, PI64, I64, I32, PI64, I64, PU8, PI64, PI64], C.c_int),
    "ekh_pool_seal_row": ([P, PI64, PI64], I64),
    "ekh_pool_counters": ([P, PI64], None),
    "ekh_pool_reset_counters": ([P], None),
    "ekh_pool_tags": ([P], PI64),
    "ekh_pool_free_list": ([P, PI64, I64], I64),
    "ekh_pool_live": ([P, PI64], None),
    "ekh_stepper_new": ([P, C.POINTER(P), I32, I64, I32], P),
    "ekh_stepper_free": ([P], None),
    "ekh_stepper_run": ([P, C.POINTER(Batch), P, I32, P, I64, C.POINTER(StepView)], C.c_int),
    "ekh_host_slots": ([C.POINTER(Batch), P, I64, I64, I64, P, I64, I32, P], C.c_int),
}

_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is missing: build it first (python -m echokv_amd.build)")
        l = C.CDLL(str(LIB_PATH))
        for name, (args, res) in _SIGS.items():
            fn = getattr(l, name)
            fn.argtypes = args
            fn.restype = res
        _lib = l
    return _lib


def i64p(a: np.ndarray):
    """Pointer to a C-contiguous int64 array."""
    return a.ctypes.data_as(PI64)


def as_i64(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.int64).reshape(-1))


def copy_i64(ptr, n: int) -> np.ndarray:
    """A numpy copy of ``n`` int64 values at ``ptr`` (native memory that a later call reuses)."""
    if n == 0:
        return np.zeros(0, np.int64)
    return np.ctypeslib.as_array(ptr, shape=(n,)).copy()


def view_i64(ptr, n: int, owner) -> np.ndarray:
    """A writable numpy view of ``n`` int64 values of native memory owned by
    ``owner``; the view keeps ``owner`` (and so the memory) alive."""
    buf = (C.c_int64 * n).from_address(C.addressof(ptr.contents))
    buf._owner = owner
    return np.frombuffer(buf, dtype=np.int64)
