"""ctypes binding of ``_lib/libmoe_mi355x.so`` (C ABI in include/moe_mi355x.h).

There is no fallback: if the library is missing, every entry point raises.
"""
from __future__ import annotations

import ctypes
from ctypes import c_int32, c_size_t, c_uint32, c_void_p, POINTER
from pathlib import Path

import os

# MOE_MI355X_LIB names another build of the same library (A/B measurements of
# a variant without replacing the in-tree one); the default is the in-tree build.
LIB_PATH = Path(os.environ.get("MOE_MI355X_LIB") or
                Path(__file__).resolve().parent / "_lib" / "libmoe_mi355x.so")

MOE_OK, MOE_EINVAL, MOE_EDEVICE, MOE_ESPACE = 0, -1, -2, -3
WEIGHTS_BF16, WEIGHTS_W4G128, WEIGHTS_W4G128_FOLD = 0, 1, 2
IDS_INT32, IDS_INT64 = 0, 1
ROUTE_FIXED, ROUTE_LOGITS = 0, 1
STATUS_BAD_ID, STATUS_BAD_WEIGHT, STATUS_BAD_LOGIT, STATUS_DIRTY_COUNTERS, STATUS_STALLED = 1, 2, 4, 8, 16


class MoeDesc(ctypes.Structure):
    _fields_ = [("T", c_int32), ("H", c_int32), ("I", c_int32), ("E", c_int32), ("K", c_int32),
                ("weight_format", c_int32), ("id_dtype", c_int32), ("route_mode", c_int32),
                ("renormalize", c_int32), ("token_block", c_int32),
                ("x", c_void_p), ("logits", c_void_p), ("ids", c_void_p), ("weights", c_void_p),
                ("gate_up", c_void_p), ("w4_words", c_void_p), ("w4_scales", c_void_p),
                ("down", c_void_p), ("out", c_void_p), ("workspace", c_void_p),
                ("workspace_bytes", c_size_t)]


class MoeLayout(ctypes.Structure):
    _fields_ = [(name, c_size_t) for name in
                ("status", "counts", "offsets", "ranks", "map", "row_route", "row_token", "tasks",
                 "num_tasks", "counters", "partials", "act", "routed", "total")] + \
               [("task_capacity", c_int32), ("token_block", c_int32), ("launches", c_int32),
                ("fast_path", c_int32)]


STATIC_WORKSPACE_BYTES = 16 << 20  # MOE_STATIC_WORKSPACE_BYTES

GQA_MAX_SEGMENTS = 4


class GqaDesc(ctypes.Structure):
    _fields_ = [("T", c_int32), ("Hq", c_int32), ("Hkv", c_int32), ("D", c_int32),
                ("num_segments", c_int32), ("len", c_int32 * GQA_MAX_SEGMENTS),
                ("q", c_void_p), ("out", c_void_p),
                ("k", c_void_p * GQA_MAX_SEGMENTS), ("v", c_void_p * GQA_MAX_SEGMENTS),
                ("k_stride", ctypes.c_int64 * GQA_MAX_SEGMENTS),
                ("v_stride", ctypes.c_int64 * GQA_MAX_SEGMENTS),
                ("scale", ctypes.c_float), ("workspace", c_void_p), ("workspace_bytes", c_size_t)]


# name -> (restype, argtypes); the complete exported ABI of include/*.h.
SIGNATURES = {
    "moe_abi_version": (c_int32, []),
    "moe_last_error": (ctypes.c_char_p, []),
    "moe_workspace_layout": (c_int32, [POINTER(MoeDesc), POINTER(MoeLayout)]),
    "moe_plan_create": (c_int32, [POINTER(c_void_p), POINTER(MoeDesc)]),
    "moe_plan_run": (c_int32, [c_void_p, c_void_p]),
    "moe_plan_run_stage": (c_int32, [c_void_p, c_int32, c_void_p]),
    "moe_plan_read_status": (c_int32, [c_void_p, c_void_p, POINTER(c_uint32)]),
    "moe_plan_reset_counters": (c_int32, [c_void_p, c_void_p]),
    "moe_forward_static": (c_int32, [POINTER(MoeDesc), c_void_p]),
    "moe_plan_layout": (c_int32, [c_void_p, POINTER(MoeLayout)]),
    "moe_plan_destroy": (None, [c_void_p]),
    "moe_w4_quantize": (c_int32, [c_void_p, c_int32, c_int32, c_int32, c_void_p, c_void_p]),
    "moe_w4_tiled_words_bytes": (c_size_t, [c_int32, c_int32, c_int32]),
    "moe_w4_tiled_scales_bytes": (c_size_t, [c_int32, c_int32, c_int32]),
    "moe_w4_tile": (c_int32, [c_void_p, c_void_p, c_int32, c_int32, c_int32, c_void_p, c_void_p]),
    "moe_w4_dequantize": (c_int32, [c_void_p, c_void_p, c_int32, c_int32, c_int32, c_void_p,
                                    c_void_p]),
    "gqa_seg_workspace_bytes": (c_int32, [POINTER(GqaDesc), POINTER(c_size_t)]),
    "gqa_seg_plan_create": (c_int32, [POINTER(c_void_p), POINTER(GqaDesc)]),
    "gqa_seg_plan_run": (c_int32, [c_void_p, c_void_p]),
    "gqa_seg_plan_destroy": (None, [c_void_p]),
}

_LIB = None


def lib():
    """Load the HIP library once; raise if it has not been built."""
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"HIP library {LIB_PATH} is not built; run "
                               "`python -m llm_gpu_kernels_amd.build`")
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        if handle.moe_abi_version() != 2:
            raise RuntimeError("libmoe_mi355x ABI version mismatch")
        _LIB = handle
    return _LIB


def last_error() -> str:
    msg = lib().moe_last_error()
    return msg.decode() if msg else ""


def check(rc: int, what: str):
    """Map C ABI return codes to the reference's exception types."""
    if rc == MOE_OK:
        return
    msg = f"{what}: {last_error()}"
    if rc in (MOE_EINVAL, MOE_ESPACE):
        raise ValueError(msg)
    raise RuntimeError(msg)
