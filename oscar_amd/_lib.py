"""ctypes binding of liboscar_amd.so (the C ABI declared in include/oscar_amd.h).

This is the binding a maintainer adds to the reference's Python backend to reach
the HIP kernels.  Loading fails loudly when the library is missing: there is no
CPU fallback in this package.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "liboscar_amd.so"

OSCAR_F32, OSCAR_F16, OSCAR_BF16 = 0, 1, 2
STAGE_NONE, STAGE_INVALIDATE, STAGE_WRITE = 0, 1, 2
WORK_INTS = 8
GROUP_INTS = 8
ABI_VERSION = 3
DECODE_STATIC_MAX_ITEMS = 512

vp = C.c_void_p
i32, i64, f32 = C.c_int32, C.c_int64, C.c_float


class Cache(C.Structure):
    _fields_ = [("k", vp), ("v", vp), ("num_blocks", i64), ("block_size", i64),
                ("num_kv_heads", i64), ("head_dim", i64), ("k_stride", i64 * 3),
                ("v_stride", i64 * 3)]


class Staging(C.Structure):
    _fields_ = [("stage_k", vp), ("stage_v", vp), ("owner", vp), ("rows", i64)]


class StoreArgs(C.Structure):
    _fields_ = [
        ("key", vp), ("value", vp), ("kv_dtype", i32), ("num_tokens", i64),
        ("key_stride_token", i64), ("value_stride_token", i64),
        ("query", vp), ("num_q_heads", i64), ("query_stride_token", i64),
        ("rk", vp), ("rv", vp), ("k_clip_ratio", f32), ("v_clip_ratio", f32),
        ("slot_mapping", vp), ("cache", Cache),
        ("stage_mode", i32), ("staging", Staging),
        ("query_start_loc", vp), ("seq_lens", vp), ("num_reqs", i32),
        ("recent_tokens", i32), ("sink_tokens_eff", i32),
        ("query_rot", vp), ("key_rot", vp), ("value_rot", vp),
        ("slot_claims", vp), ("seat_claims", vp), ("epoch_counter", vp),
        ("workspace", vp), ("workspace_bytes", i64), ("arrivals", vp),
    ]


class RotateArgs(C.Structure):
    _fields_ = [("x", vp), ("x_dtype", i32), ("rows", i64), ("x_stride_row", i64),
                ("r", vp), ("transpose", i32), ("out", vp), ("out_dtype", i32),
                ("out_stride_row", i64), ("head_dim", i64)]


class Plan(C.Structure):
    _fields_ = [("num_items", i32), ("num_groups", i32), ("partial_bytes", i64),
                ("max_group_items", i32), ("reserved", i32)]


class AttnArgs(C.Structure):
    _fields_ = [
        ("q", vp), ("num_tokens", i64), ("num_q_heads", i64), ("q_stride_token", i64),
        ("k_new", vp), ("v_new", vp), ("kv_new_stride_token", i64),
        ("cache", Cache), ("block_table", vp), ("block_table_stride", i64),
        ("query_start_loc", vp), ("seq_lens", vp), ("num_reqs", i32),
        ("staging", C.POINTER(Staging)), ("scale", f32),
        ("items", vp), ("num_items", i32), ("groups", vp), ("num_groups", i32),
        ("workspace", vp), ("workspace_bytes", i64), ("max_group_items", i32),
        ("out_rot", vp), ("lse", vp), ("phases", i32), ("q_dtype", i32),
        ("block_table_rows", i64), ("block_table_cols", i64),
    ]


class PrefillArgs(C.Structure):
    _fields_ = [
        ("q", vp), ("q_stride_token", i64), ("k", vp), ("v", vp), ("kv_stride_token", i64),
        ("num_tokens", i64), ("num_q_heads", i64), ("num_kv_heads", i64), ("head_dim", i64),
        ("history", i64), ("cache", Cache), ("block_table_row", vp),
        ("staging", C.POINTER(Staging)), ("scale", f32), ("out", vp),
        ("out_stride_token", i64), ("lse", vp), ("workspace", vp), ("workspace_bytes", i64),
        ("q_dtype", i32), ("block_table_cols", i64),
    ]


class StepArgs(C.Structure):
    _fields_ = [
        ("query", vp), ("key", vp), ("value", vp), ("kv_stride_token", i64),
        ("num_tokens", i64), ("num_q_heads", i64), ("q_dtype", i32), ("stage_mode", i32),
        ("slot_mapping", vp), ("cache", Cache), ("block_table", vp), ("block_table_stride", i64),
        ("staging", C.POINTER(Staging)), ("sink_tokens_eff", i32), ("recent_tokens", i32),
        ("rk", vp), ("rv", vp), ("k_clip_ratio", f32), ("v_clip_ratio", f32), ("scale", f32),
        ("target_items", i32), ("host_query_start_loc", vp), ("host_seq_lens", vp),
        ("num_reqs", i32), ("reserved", i32), ("output", vp),
        ("slot_claims", vp), ("seat_claims", vp), ("epoch_counter", vp),
        ("store_workspace", vp), ("store_workspace_bytes", i64), ("arrivals", vp),
        ("workspace", vp), ("workspace_bytes", i64), ("workspace_needed", i64),
        ("block_table_rows", i64), ("block_table_cols", i64),
    ]


STEP_NOT_DECODE = 1

# name -> (restype, argtypes); every symbol declared in include/oscar_amd.h
SIGNATURES = {
    "oscar_abi_version": (C.c_int, []),
    "oscar_last_error": (C.c_char_p, []),
    "oscar_store_workspace_bytes_v1": (i64, [i64, i64, i64]),
    "oscar_store_v1": (C.c_int, [C.POINTER(StoreArgs), vp]),
    "oscar_rotate_v1": (C.c_int, [C.POINTER(RotateArgs), vp]),
    "oscar_attn_plan_v1": (C.c_int, [C.POINTER(i32), C.POINTER(i32), i32, i32, i32, i32, i32,
                                     i32, i32, i32, i32, C.POINTER(i32), i32, C.POINTER(i32), i32,
                                     C.POINTER(Plan)]),
    "oscar_attn_decode_v1": (C.c_int, [C.POINTER(AttnArgs), vp]),
    "oscar_decode_write_v1": (C.c_int, [C.POINTER(StoreArgs), C.POINTER(AttnArgs), vp]),
    "oscar_attn_decode_static_v1": (C.c_int, [C.POINTER(AttnArgs), vp]),
    "oscar_prefill_workspace_bytes_v1": (i64, [i64, i64, i64]),
    "oscar_prefill_workspace_bytes_v2": (i64, [i64, i64, i64, i64, i64]),
    "oscar_prefill_plan_v1": (C.c_int, [i64, i64, i64, i64, C.POINTER(i32), i32]),
    "oscar_attn_prefill_v1": (C.c_int, [C.POINTER(PrefillArgs), vp]),
    "oscar_context_create_v1": (C.c_int, [i32, C.POINTER(vp)]),
    "oscar_context_destroy_v1": (C.c_int, [vp]),
    "oscar_step_workspace_bytes_v1": (i64, [i64, i64, i64, i64, i64]),
    "oscar_decode_step_v1": (C.c_int, [vp, C.POINTER(StepArgs), vp]),
}

_LIB = None


class OscarLibraryError(RuntimeError):
    pass


def load() -> C.CDLL:
    """Load the HIP library once; raise if it has not been built."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not LIB_PATH.exists():
        raise OscarLibraryError(
            f"{LIB_PATH} is missing: build it with `python -m oscar_amd.build` "
            "(no CPU fallback exists for the OSCAR HIP path)")
    lib = C.CDLL(str(LIB_PATH))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if lib.oscar_abi_version() != ABI_VERSION:
        raise OscarLibraryError("liboscar_amd.so ABI version mismatch")
    _LIB = lib
    return lib


EINVAL = -22


def check(status: int, what: str) -> None:
    """Raise for a nonzero status: ValueError for rejected arguments (-22, where the
    reference's own checks raise ValueError, e.g. streaming_attention.py:32-65),
    RuntimeError for anything else (launch or allocation failures)."""
    if status != 0:
        msg = load().oscar_last_error().decode(errors="replace")
        cls = ValueError if status == EINVAL else RuntimeError
        raise cls(f"{what} failed ({status}): {msg}")
