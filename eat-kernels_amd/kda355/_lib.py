"""ctypes binding of libkda355.so (the C ABI declared in include/kda355.h).

The library is loaded from this directory only.  There is no fallback: if it is missing, every entry point raises.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libkda355.so"
NOALLOC_LIB_PATH = Path(__file__).resolve().parent / "libkda355_noalloc.so"

P = ctypes.c_void_p
I32 = ctypes.c_int32
I64 = ctypes.c_int64
U32 = ctypes.c_uint32
F32 = ctypes.c_float

EINVAL = -1
ELAUNCH = -2

REC_NORMALIZE_QK = 1
REC_RAW_GATE = 2
REC_RAW_BETA = 4
REC_PER_TOKEN = 8
REC_SLOT0_RESERVED = 16
REC_WRITE_SLOT0_RESERVED = 32


class KdaRecurrentArgs(ctypes.Structure):
    _fields_ = [
        ("q", P), ("k", P), ("v", P), ("g", P), ("beta", P), ("A_log", P), ("dt_bias", P),
        ("read_pool", P), ("write_pool", P), ("read_idx", P), ("num_accepted", P), ("write_idx", P), ("out", P),
        ("qkv_row_stride", I64), ("g_row_stride", I64), ("beta_row_stride", I64), ("out_row_stride", I64),
        ("read_slot_stride", I64), ("read_slots", I64), ("write_slot_stride", I64), ("write_slots", I64),
        ("B", I32), ("S", I32), ("H", I32), ("read_idx_stride", I32),
        ("scale", F32), ("lower_bound", F32), ("flags", U32), ("reserved", I32),
    ]


class KdaSpecCommitArgs(ctypes.Structure):
    _fields_ = [
        ("scratch", P), ("pool", P), ("scratch_idx", P), ("pool_idx", P), ("num_accepted", P),
        ("scratch_slot_stride", I64), ("scratch_slots", I64), ("pool_slot_stride", I64), ("pool_slots", I64),
        ("B", I32), ("S", I32), ("H", I32), ("flags", U32),
    ]


class KdaDecodeArgs(ctypes.Structure):
    _fields_ = [
        ("mixed_qkv", P), ("conv_state", P), ("conv_weight", P), ("gate", P), ("beta", P), ("out_gate", P),
        ("A_log", P), ("dt_bias", P), ("norm_weight", P), ("ssm_state", P), ("state_indices", P),
        ("num_accepted", P), ("out", P),
        ("mixed_row_stride", I64), ("gate_row_stride", I64), ("beta_row_stride", I64), ("out_gate_row_stride", I64),
        ("out_row_stride", I64),
        ("conv_slot_stride", I64), ("conv_tap_stride", I64), ("conv_slots", I64), ("ssm_slot_stride", I64),
        ("ssm_slots", I64),
        ("B", I32), ("S", I32), ("H", I32), ("conv_taps", I32),
        ("norm_eps", F32), ("lower_bound", F32), ("flags", U32), ("reserved", I32),
        ("workspace", P),
    ]


class KdaPrefillPlanIn(ctypes.Structure):
    _fields_ = [
        ("cu_seqlens", P), ("ck_offsets", P), ("N", I32), ("H", I32), ("ck_every", I32), ("num_cus", I32),
        ("flags", U32), ("reserved", I32),
    ]


class KdaPrefillPlan(ctypes.Structure):
    _fields_ = [
        ("T", I64), ("N", I32), ("H", I32), ("num_chunks", I32), ("num_chains", I32), ("max_chain_chunks", I32),
        ("ck_every", I32), ("table_words", I64), ("workspace_bytes", I64), ("ck_rows", I64), ("magic", U32),
        ("flags", U32), ("num_pieces", I32), ("num_split", I32), ("num_fix_tasks", I32), ("num_ck_tasks", I32),
        ("chunk_grid", I32), ("chunk32", I32),
    ]


class KdaPrefillArgs(ctypes.Structure):
    _fields_ = [
        ("q", P), ("k", P), ("v", P), ("g", P), ("beta", P), ("A_log", P), ("dt_bias", P),
        ("out", P),
        ("state_pool", P), ("state_idx", P), ("has_initial_state", P),
        ("initial_state", P), ("final_state", P),
        ("ck_pool", P), ("ck_idx", P),
        ("tables", P), ("workspace", P),
        ("qkv_row_stride", I64), ("g_row_stride", I64), ("beta_row_stride", I64), ("out_row_stride", I64),
        ("state_slot_stride", I64), ("state_slots", I64), ("ck_slot_stride", I64), ("ck_slots", I64),
        ("T", I64), ("N", I32), ("H", I32),
        ("scale", F32), ("lower_bound", F32), ("flags", U32), ("ck_dtype", I32),
        ("plan", ctypes.POINTER(KdaPrefillPlan)),
    ]


_lib = None
_noalloc = None


def lib():
    """The loaded library; raises RuntimeError when it has not been built (no CPU or torch fallback exists)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"kda355: native library not built: {LIB_PATH} "
                               "(run __graft_entry__.build() or `make -C eat-kernels_amd/csrc`)")
        L = ctypes.CDLL(str(LIB_PATH))
        L.kda355_recurrent_launch.argtypes = [ctypes.POINTER(KdaRecurrentArgs), P]
        L.kda355_recurrent_launch.restype = ctypes.c_int
        L.kda355_spec_commit_launch.argtypes = [ctypes.POINTER(KdaSpecCommitArgs), P]
        L.kda355_spec_commit_launch.restype = ctypes.c_int
        L.kda355_decode_launch.argtypes = [ctypes.POINTER(KdaDecodeArgs), P]
        L.kda355_decode_launch.restype = ctypes.c_int
        L.kda355_prefill_plan.argtypes = [ctypes.POINTER(KdaPrefillPlanIn), ctypes.POINTER(KdaPrefillPlan), P, I64]
        L.kda355_prefill_plan.restype = ctypes.c_int
        L.kda355_prefill_workspace_bytes.argtypes = [ctypes.POINTER(KdaPrefillPlan)]
        L.kda355_prefill_workspace_bytes.restype = I64
        L.kda355_prefill_launch.argtypes = [ctypes.POINTER(KdaPrefillArgs), P]
        L.kda355_prefill_launch.restype = ctypes.c_int
        L.kda355_last_error.restype = ctypes.c_char_p
        L.kda355_version.restype = ctypes.c_int
        _lib = L
    return _lib


def noalloc_lib():
    """libkda355_noalloc.so (kda355_prefill_launch_noalloc and its static device scratch), loaded on first use only: a
    process that never calls the no-allocation entry point never holds the scratch."""
    global _noalloc
    if _noalloc is None:
        lib()
        if not NOALLOC_LIB_PATH.exists():
            raise RuntimeError(f"kda355: native library not built: {NOALLOC_LIB_PATH} "
                               "(run __graft_entry__.build() or `make -C eat-kernels_amd/csrc`)")
        L = ctypes.CDLL(str(NOALLOC_LIB_PATH))
        L.kda355_prefill_launch_noalloc.argtypes = [ctypes.POINTER(KdaPrefillArgs), P]
        L.kda355_prefill_launch_noalloc.restype = ctypes.c_int
        _noalloc = L
    return _noalloc


def check(rc: int, what: str):
    if rc == 0:
        return
    msg = lib().kda355_last_error().decode(errors="replace")
    if rc == EINVAL:
        raise ValueError(f"{what}: {msg}")
    raise RuntimeError(f"{what}: {msg} (status {rc})")


def exported_symbols():
    """Names declared in include/kda355.h that the library must export."""
    return ["kda355_recurrent_launch", "kda355_spec_commit_launch", "kda355_decode_launch", "kda355_prefill_plan",
            "kda355_prefill_workspace_bytes", "kda355_prefill_launch", "kda355_prefill_launch_noalloc",
            "kda355_last_error", "kda355_version"]


NOALLOC_SYMBOLS = ("kda355_prefill_launch_noalloc",)  # exported by libkda355_noalloc.so, the rest by libkda355.so


NOALLOC_SCRATCH_BYTES = 256 << 20  # KDA355_NOALLOC_SCRATCH_BYTES
