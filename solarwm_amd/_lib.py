"""ctypes binding of libsolarkv.so (the C ABI declared in include/solarkv.h).

The library is loaded from the package directory only (it is built in-tree by
``solarwm_amd.build``).  There is no fallback implementation: if the library is missing every
entry point raises, so a product path can never silently run on the CPU.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libsolarkv.so"

SKV_F32 = 0
SKV_BF16 = 1
SKV_FP8_E4M3 = 2
SKV_F16 = 3

SKV_MASK_NONE = 0
SKV_MASK_CHUNK_CAUSAL = 1

SKV_OK = 0
SKV_E_ARG = -1
SKV_E_UNSUPPORTED = -2
SKV_E_LAUNCH = -3

SKV_MAX_APPEND_FRAMES = 64
SKV_MAX_FRAMES = 256
SKV_MAX_SEGMENTS = 64
SKV_NOALLOC_SCRATCH_BYTES = 68157440

# Every symbol include/solarkv.h declares, with (restype, argtypes).
_i32, _i64, _f32, _vp = ctypes.c_int, ctypes.c_int64, ctypes.c_float, ctypes.c_void_p
_i32p = ctypes.POINTER(ctypes.c_int32)


class AppendDesc(ctypes.Structure):
    """``skv_append_desc`` (include/solarkv.h), field for field."""

    _fields_ = [
        ("k_new", _vp), ("v_new", _vp), ("src_dtype", _i32),
        ("src_sb", _i64), ("src_st", _i64), ("src_sh", _i64), ("src_frame0", _i32),
        ("k_pool", _vp), ("v_pool", _vp), ("k_scale", _vp), ("v_scale", _vp),
        ("pool_dtype", _i32), ("n_slots", _i32), ("dst_slots", _i32p),
        ("n_frames", _i32), ("batch", _i32), ("heads", _i32), ("head_dim", _i32),
        ("frame_tokens", _i32),
        ("k_inv_rms", _vp), ("k_rms_stride_b", _i64), ("k_norm_weight", _vp),
        ("kr_pool", _vp), ("rope_hw", _vp), ("grid_h", _i32), ("grid_w", _i32),
        ("vx_pool", _vp), ("kv_xform", _vp), ("workspace", _vp), ("workspace_bytes", _i64),
        ("kr_scale", _vp), ("vx_scale", _vp),
    ]


class AttentionDesc(ctypes.Structure):
    """``skv_attention_desc`` (include/solarkv.h), field for field."""

    _fields_ = [
        ("q", _vp), ("q_dtype", _i32), ("q_sb", _i64), ("q_st", _i64), ("q_sh", _i64),
        ("k_pool", _vp), ("v_pool", _vp), ("k_scale", _vp), ("v_scale", _vp),
        ("pool_dtype", _i32), ("n_slots", _i32), ("frame_slots", _i32p),
        ("n_frames", _i32), ("batch", _i32), ("heads", _i32), ("head_dim", _i32),
        ("q_len", _i32), ("frame_tokens", _i32),
        ("softmax_scale", _f32), ("mask_mode", _i32), ("q_pos0", _i64), ("chunk_tokens", _i64),
        ("out", _vp), ("out_sb", _i64), ("out_st", _i64), ("out_sh", _i64),
        ("q_inv_rms", _vp), ("q_rms_stride_b", _i64), ("q_norm_weight", _vp),
        ("rope_hw", _vp), ("grid_h", _i32), ("grid_w", _i32), ("rope_t", _vp), ("n_qframes", _i32),
        ("q_xform_t", _vp), ("q_xform_s", _vp), ("out_xform", _vp), ("frame_lens", _i32p),
        ("workspace", _vp), ("workspace_bytes", _i64),
        ("seg_rows", _i32p), ("seg_frames", _i32p), ("n_segments", _i32),
    ]


class H3XformDesc(ctypes.Structure):
    """``skv_h3_xform_desc`` (include/solarkv.h), field for field."""

    _fields_ = [
        ("x", _vp), ("x_sb", _i64), ("x_st", _i64), ("x_sh", _i64),
        ("out", _vp), ("out_sb", _i64), ("out_st", _i64), ("out_sh", _i64),
        ("batch", _i32), ("rows", _i32), ("heads", _i32), ("head_dim", _i32),
        ("cos", _vp), ("sin", _vp), ("table_dtype", _i32), ("table_stride", _i64),
        ("matrix", _vp), ("matrix_dtype", _i32), ("matrix_sb", _i64), ("matrix_st", _i64),
    ]


class LaunchPlan(ctypes.Structure):
    """``skv_launch_plan`` (include/solarkv.h): the launch skv_attention_ex would make."""

    _fields_ = [
        ("waves_per_group", _i32), ("split", _i32), ("n_workgroups", _i32), ("n_qtiles", _i32),
        ("workspace_bytes", _i64), ("key_tiles", _i32),
    ]


SIGNATURES: dict[str, tuple] = {
    "skv_version": (_i32, []),
    "skv_last_error": (ctypes.c_char_p, []),
    "skv_append": (
        _i32,
        [_vp, _vp, _i32, _i64, _i64, _i64, _i32, _vp, _vp, _vp, _vp, _i32, _i32, _i32p, _i32,
         _i32, _i32, _i32, _i32, _vp],
    ),
    "skv_gather": (
        _i32,
        [_vp, _vp, _i32, _i32, _i32p, _i32, _i32, _i32, _i32, _i32, _vp, _vp, _i64, _i64, _i64,
         _vp],
    ),
    "skv_attention": (
        _i32,
        [_vp, _i32, _i64, _i64, _i64, _vp, _vp, _vp, _vp, _i32, _i32, _i32p, _i32, _i32, _i32,
         _i32, _i32, _i32, _f32, _i32, _i64, _i64, _vp, _i64, _i64, _i64, _vp],
    ),
    "skv_append_rope": (
        _i32,
        [_vp, _vp, _i32, _i64, _i64, _i64, _i32, _vp, _vp, _i32, _i32, _i32p, _i32, _i32, _i32,
         _i32, _i32, _vp, _vp, _i32, _i32, _vp],
    ),
    "skv_attention_rope": (
        _i32,
        [_vp, _i32, _i64, _i64, _i64, _vp, _vp, _i32, _i32, _i32p, _i32, _i32, _i32, _i32, _i32,
         _i32, _f32, _i32, _i64, _i64, _vp, _i64, _i64, _i64, _vp, _i32, _i32, _vp, _i32, _vp],
    ),
    "skv_append_prope": (
        _i32,
        [_vp, _vp, _i32, _i64, _i64, _i64, _i32, _vp, _vp, _i32, _i32, _i32p, _i32, _i32, _i32,
         _i32, _i32, _vp, _vp, _vp, _i32, _i32, _vp, _vp],
    ),
    "skv_attention_prope": (
        _i32,
        [_vp, _i32, _i64, _i64, _i64, _vp, _vp, _i32, _i32, _i32p, _i32, _i32, _i32, _i32, _i32,
         _i32, _f32, _i32, _i64, _i64, _vp, _i64, _i64, _i64, _vp, _i32, _i32, _vp, _vp, _vp,
         _i32, _vp],
    ),
    "skv_rms_rows": (
        _i32,
        [_vp, _i32, _i64, _i64, _i64, _i32, _i32, _i32, _i32, _f32, _vp, _vp],
    ),
    "skv_append_ex": (_i32, [ctypes.POINTER(AppendDesc), _vp]),
    "skv_attention_ex": (_i32, [ctypes.POINTER(AttentionDesc), _vp]),
    "skv_attention_plan": (_i32, [ctypes.POINTER(AttentionDesc), ctypes.POINTER(LaunchPlan)]),
    "skv_attention_ex_noalloc": (_i32, [ctypes.POINTER(AttentionDesc), _vp]),
    "skv_noalloc_init": (_i32, []),
    "skv_append_workspace_size": (_i32, [ctypes.POINTER(AppendDesc), ctypes.POINTER(_i64)]),
    "skv_h3_rope_prope": (_i32, [ctypes.POINTER(H3XformDesc), _vp]),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


class SolarKVError(RuntimeError):
    """A libsolarkv entry point returned a non-zero status."""

    def __init__(self, fn: str, status: int, message: str):
        super().__init__(f"{fn} failed with status {status}: {message}")
        self.fn = fn
        self.status = status
        self.message = message


def load() -> ctypes.CDLL:
    """Load libsolarkv.so once per process; raise if it is absent."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise ImportError(
                f"{LIB_PATH} is not built; run `python -m solarwm_amd.build` "
                "(there is no CPU fallback for the KV-cache kernels)"
            )
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = lib
        return lib


def check(fn: str, status: int) -> None:
    if status != SKV_OK:
        msg = load().skv_last_error().decode(errors="replace")
        if status in (SKV_E_ARG, SKV_E_UNSUPPORTED):
            raise ValueError(f"{fn}: {msg}")
        raise SolarKVError(fn, status, msg)


def int32_array(values) -> ctypes.Array:
    vals = [int(v) for v in values]
    return (ctypes.c_int32 * max(1, len(vals)))(*vals)
