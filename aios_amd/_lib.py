"""ctypes binding of libaios_attn.so (the C ABI declared in include/aios_attn.h).

The library is loaded lazily on first use.  There is no fallback: if the
shared library is missing or fails to load, every call raises.
"""
from __future__ import annotations

import ctypes
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libaios_attn.so"

AIOS_OK = 0
AIOS_ERR_INVALID = 1
AIOS_ERR_UNSUPPORTED = 2
AIOS_ERR_WORKSPACE = 3
AIOS_ERR_LAUNCH = 4

PHASE_PREFILL = 0
PHASE_DECODE = 1
PROLOGUE_NONE = 0
PROLOGUE_ADD_RMSNORM = 1
EPILOGUE_NONE = 0
EPILOGUE_SILU_MUL = 1

# Every symbol include/aios_attn.h declares.
# Size of the built-in partial-state array of aios_attn_decode_noalloc
# (AIOS_DECODE_NOALLOC_MAX_BYTES in include/aios_attn.h).
DECODE_NOALLOC_MAX_BYTES = 8 << 20

EXPORTED_SYMBOLS = (
    "aios_last_error",
    "aios_version",
    "aios_kv_append",
    "aios_attn_plan",
    "aios_attn_prefill",
    "aios_attn_decode",
    "aios_attn_append_decode",
    "aios_attn_append_decode_rope",
    "aios_attn_decode_noalloc",
    "aios_build_indices",
    "aios_rmsnorm",
    "aios_qk_norm_rope",
    "aios_cg_step_begin",
    "aios_cg_step_end",
    "aios_cg_step_prepare",
    "aios_silu_mul",
    "aios_linear_rows",
    "aios_linear_rows_ex",
    "aios_greedy_select",
    "aios_attnres_mix",
    "aios_attnres_mix_ex",
    "aios_stateless_uniforms",
    "aios_sample",
)


class AttnPlan(ctypes.Structure):
    """Mirror of ``aios_attn_plan_t``."""

    _fields_ = [
        ("phase", ctypes.c_int32),
        ("batch_size", ctypes.c_int32),
        ("num_qo_heads", ctypes.c_int32),
        ("num_kv_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("group", ctypes.c_int32),
        ("total_q", ctypes.c_int32),
        ("total_kv", ctypes.c_int32),
        ("max_q_len", ctypes.c_int32),
        ("max_kv_len", ctypes.c_int32),
        ("prefix_len", ctypes.c_int32),
        ("prefix_chunk_len", ctypes.c_int32),
        ("num_prefix_chunks", ctypes.c_int32),
        ("cascade_rows", ctypes.c_int32),
        ("cascade_mgroups", ctypes.c_int32),
        ("suffix_split_len", ctypes.c_int32),
        ("num_suffix_splits", ctypes.c_int32),
        ("suffix_tpg", ctypes.c_int32),
        ("num_parts", ctypes.c_int32),
        ("prefill_q_tile", ctypes.c_int32),
        ("num_q_tiles", ctypes.c_int32),
        ("stage_mask", ctypes.c_int32),
        ("min_kv_len", ctypes.c_int32),
        ("suffix_parts_per_item", ctypes.c_int32),
        ("ws_parts_o", ctypes.c_int64),
        ("ws_parts_lse", ctypes.c_int64),
        ("ws_bytes", ctypes.c_int64),
    ]

    def as_dict(self) -> dict:
        return {name: getattr(self, name) for name, _ in self._fields_}


_lock = threading.Lock()
_lib: ctypes.CDLL | None = None

_vp = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_f32 = ctypes.c_float


def _declare(lib: ctypes.CDLL) -> None:
    lib.aios_last_error.restype = ctypes.c_char_p
    lib.aios_last_error.argtypes = []
    lib.aios_version.restype = ctypes.c_char_p
    lib.aios_version.argtypes = []
    lib.aios_kv_append.restype = ctypes.c_int
    lib.aios_kv_append.argtypes = [
        _vp, _vp, _i64, _i64, _vp, _vp, _i64, _vp, _i64, _i64, _i64, _i32, _vp,
    ]
    lib.aios_attn_plan.restype = ctypes.c_int
    lib.aios_attn_plan.argtypes = [
        _i32, _vp, _vp, _i32, _i32, _i32, _i32, _i32, _i32, _i64, _i32, _i32,
        ctypes.POINTER(AttnPlan),
    ]
    lib.aios_attn_prefill.restype = ctypes.c_int
    lib.aios_attn_prefill.argtypes = [
        ctypes.POINTER(AttnPlan), _vp, _i64, _vp, _vp, _i64, _vp, _vp, _vp, _vp, _f32, _vp,
    ]
    lib.aios_attn_decode.restype = ctypes.c_int
    lib.aios_attn_decode.argtypes = [
        ctypes.POINTER(AttnPlan), _vp, _i64, _vp, _vp, _i64, _vp, _vp, _vp, _vp, _i64, _f32, _vp,
    ]
    lib.aios_attn_decode_noalloc.restype = ctypes.c_int
    lib.aios_attn_decode_noalloc.argtypes = [
        ctypes.POINTER(AttnPlan), _vp, _i64, _vp, _vp, _i64, _vp, _vp, _vp, _f32, _vp,
    ]
    lib.aios_attn_append_decode.restype = ctypes.c_int
    lib.aios_attn_append_decode.argtypes = [
        ctypes.POINTER(AttnPlan), _vp, _i64, _vp, _i64, _vp, _i64, _vp, _vp, _vp, _i64, _vp, _vp,
        _vp, _vp, _i64, _f32, _vp,
    ]
    lib.aios_attn_append_decode_rope.restype = ctypes.c_int
    lib.aios_attn_append_decode_rope.argtypes = [
        ctypes.POINTER(AttnPlan), _vp, _i64, _vp, _i64, _vp, _i64, _vp, _vp, _vp, _i64, _vp, _vp,
        _vp, _vp, _vp, _vp, _i64, _vp, _f32, _vp, _vp, _i64, _f32, _vp,
    ]
    lib.aios_build_indices.restype = ctypes.c_int
    lib.aios_build_indices.argtypes = [_vp, _i64, _vp, _vp, _i32, _i32, _vp, _vp]
    lib.aios_rmsnorm.restype = ctypes.c_int
    lib.aios_rmsnorm.argtypes = [_vp, _i64, _vp, _i64, _vp, _vp, _i64, _i64, _i32, _f32, _vp]
    lib.aios_cg_step_begin.restype = ctypes.c_int
    lib.aios_cg_step_begin.argtypes = [_vp, _vp, _i32, _i32, _vp, _vp, _i64, _i32, _vp, _vp]
    lib.aios_cg_step_prepare.restype = ctypes.c_int
    lib.aios_cg_step_prepare.argtypes = [_vp, _vp, _i32, _i32, _vp, _vp, _i64, _i32, _vp, _vp,
                                         _vp, _i32, _vp, _vp, _vp, _i64, _i32, _vp, _vp]
    lib.aios_cg_step_end.restype = ctypes.c_int
    lib.aios_cg_step_end.argtypes = [_vp, _i32, _vp, _vp, _i64, _vp, _vp, _vp, _i64, _i32, _vp,
                                     _vp, _vp, _vp, _vp, _vp]
    lib.aios_qk_norm_rope.restype = ctypes.c_int
    lib.aios_qk_norm_rope.argtypes = [_vp, _i64, _i64, _i32, _i32, _i32, _vp, _vp, _vp, _vp, _i64,
                                      _vp, _vp, _vp, _f32, _vp]
    lib.aios_silu_mul.restype = ctypes.c_int
    lib.aios_silu_mul.argtypes = [_vp, _i64, _i64, _i32, _vp, _i64, _vp]
    lib.aios_linear_rows.restype = ctypes.c_int
    lib.aios_linear_rows.argtypes = [_vp, _i64, _vp, _i64, _vp, _i64, _i64, _i64, _i64, _vp]
    lib.aios_linear_rows_ex.restype = ctypes.c_int
    lib.aios_linear_rows_ex.argtypes = [_vp, _i64, _vp, _i64, _vp, _i64, _i64, _i64, _i64, _i32,
                                        _vp, _i64, _vp, _f32, _vp, _i64, _i32, _vp]
    lib.aios_greedy_select.restype = ctypes.c_int
    lib.aios_greedy_select.argtypes = [_vp, _i64, _i32, _i32, _i32, _vp, _vp, _vp]
    lib.aios_stateless_uniforms.restype = ctypes.c_int
    lib.aios_stateless_uniforms.argtypes = [_vp, _i32, _i32, _vp, _vp]
    lib.aios_sample.restype = ctypes.c_int
    lib.aios_sample.argtypes = [_vp, _i64, _i32, _i32, _i32, _f32, _i32, _f32, _vp, _i64, _i32,
                                _vp, _vp, _i32, _i32, _vp, _i32, _vp, _vp, _vp]
    lib.aios_attnres_mix.restype = ctypes.c_int
    lib.aios_attnres_mix.argtypes = [_vp, _i32, _i64, _i32, _vp, _vp, _f32, _vp, _vp, _vp]
    lib.aios_attnres_mix_ex.restype = ctypes.c_int
    lib.aios_attnres_mix_ex.argtypes = [_vp, _i32, _i64, _i32, _vp, _vp, _vp, _vp, _f32, _vp, _vp,
                                        _vp]


def lib() -> ctypes.CDLL:
    """Return the loaded library, loading it on first use (raises if absent)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"{LIB_PATH.name} is not built; run `python -m aios_amd.build` "
                    "(the gfx950 HIP backend has no fallback path)"
                )
            handle = ctypes.CDLL(str(LIB_PATH))
            _declare(handle)
            _lib = handle
    return _lib


def check(status: int, what: str) -> None:
    """Turn a non-zero status into the exception type the reference raises."""
    if status == AIOS_OK:
        return
    msg = lib().aios_last_error().decode(errors="replace")
    if status in (AIOS_ERR_INVALID, AIOS_ERR_UNSUPPORTED):
        raise ValueError(msg or f"{what} failed")
    raise RuntimeError(f"{what}: {msg} (status {status})")
