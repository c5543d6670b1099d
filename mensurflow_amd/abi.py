"""ctypes binding of the C ABI in ``include/mfr_rocm.h`` (``_lib/libmfr_rocm.so``).

This is a thin, loud binding: loading fails with an ImportError naming the missing library,
every nonzero status raises the exception the reference would throw (``ValueError`` for
``std::invalid_argument``, ``RuntimeError`` for ``std::runtime_error``, ``NotImplementedError``
for an unsupported layout), and there is no CPU fallback anywhere.
"""
from __future__ import annotations

import ctypes
import os

_PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_PKG, "_lib", "libmfr_rocm.so")

MFR_OK = 0
MFR_E_INVALID = 1
MFR_E_RUNTIME = 2
MFR_E_UNSUPPORTED = 3
MFR_E_NO_DEVICE = 4

ACT_NONE = 0
ACT_GELU_TANH = 1
ACT_GELU_ERF = 2

EW_ADD = 0
EW_MUL = 1
EW_SCAL = 2
EW_SUB = 3

TILE_AUTO = 0
TILE_256x256 = 1
TILE_128x128 = 2
TILE_128x64 = 3
TILE_64x128 = 4
TILE_64x64 = 5
TILE_THIN = 6
TILE_PANEL = 7
TILE_COUNT = 8
GEMM_CAUSAL = 1  # mfr_gemm_desc.flags: C(i, j) = -inf wherever j > i (panel path only)
STAGE_AUTO = 0
STAGE_NEVER = 1
STAGE_ALWAYS = 2
MAX_SPLITS = 64

MAX_BATCH_DIMS = 4
MAX_COPY_DIMS = 8
SGEMM_SCRATCH_BYTES = 64 << 20  # MFR_SGEMM_SCRATCH_BYTES: mfr_sgemm_noalloc's fixed scratch

_i64 = ctypes.c_int64
_i32 = ctypes.c_int32
_vp = ctypes.c_void_p
_f32 = ctypes.c_float
_size = ctypes.c_size_t


class GemmDesc(ctypes.Structure):
    """mfr_gemm_desc (include/mfr_rocm.h)."""

    _fields_ = [
        ("m", _i64), ("n", _i64), ("k", _i64),
        ("batch_dims", _i32), ("act", _i32),
        ("batch", _i64 * MAX_BATCH_DIMS),
        ("a", _vp), ("a_rs", _i64), ("a_cs", _i64), ("a_bs", _i64 * MAX_BATCH_DIMS),
        ("b", _vp), ("b_rs", _i64), ("b_cs", _i64), ("b_bs", _i64 * MAX_BATCH_DIMS),
        ("c", _vp), ("c_rs", _i64), ("c_bs", _i64 * MAX_BATCH_DIMS),
        ("c0", _vp), ("c0_rs", _i64), ("c0_bs", _i64 * MAX_BATCH_DIMS),
        ("bias", _vp),
        ("alpha", _f32), ("beta", _f32),
        ("tile", _i32), ("stage", _i32), ("splits", _i32), ("flags", _i32),
    ]


class AttentionDesc(ctypes.Structure):
    """mfr_attention_desc (include/mfr_rocm.h)."""

    _fields_ = [
        ("lq", _i64), ("lk", _i64), ("d", _i64),
        ("batch_dims", _i32), ("causal", _i32),
        ("batch", _i64 * MAX_BATCH_DIMS),
        ("q", _vp), ("q_rs", _i64), ("q_bs", _i64 * MAX_BATCH_DIMS),
        ("k", _vp), ("k_rs", _i64), ("k_bs", _i64 * MAX_BATCH_DIMS),
        ("v", _vp), ("v_rs", _i64), ("v_bs", _i64 * MAX_BATCH_DIMS),
        ("out", _vp), ("out_rs", _i64), ("out_bs", _i64 * MAX_BATCH_DIMS),
        ("mask", _vp), ("mask_rs", _i64), ("mask_cs", _i64), ("mask_bs", _i64 * MAX_BATCH_DIMS),
        ("scale", _f32), ("reserved", _i32),
    ]


# name -> (restype, argtypes). Every symbol the header declares is here; tests check that the
# library exports each of them.
SIGNATURES = {
    "mfr_last_error": (ctypes.c_char_p, []),
    "mfr_get_device_count": (ctypes.c_int, [ctypes.POINTER(ctypes.c_int)]),
    "mfr_get_device_info": (ctypes.c_int, [ctypes.c_int, ctypes.c_char_p, _size,
                                           ctypes.POINTER(_size), ctypes.POINTER(ctypes.c_int),
                                           ctypes.POINTER(ctypes.c_int)]),
    "mfr_malloc": (ctypes.c_int, [ctypes.c_int, _size, ctypes.POINTER(_vp)]),
    "mfr_free": (ctypes.c_int, [ctypes.c_int, _vp]),
    "mfr_stream_create": (ctypes.c_int, [ctypes.c_int, ctypes.POINTER(_vp)]),
    "mfr_stream_wrap": (ctypes.c_int, [ctypes.c_int, _vp, ctypes.POINTER(_vp)]),
    "mfr_stream_destroy": (ctypes.c_int, [_vp]),
    "mfr_stream_sync": (ctypes.c_int, [_vp]),
    "mfr_stream_handle": (_vp, [_vp]),
    "mfr_stream_device": (ctypes.c_int, [_vp]),
    "mfr_memcpy_h2d": (ctypes.c_int, [_vp, _vp, _vp, _size]),
    "mfr_memcpy_d2h": (ctypes.c_int, [_vp, _vp, _vp, _size]),
    "mfr_memcpy_d2d": (ctypes.c_int, [_vp, _vp, _vp, _size]),
    "mfr_event_create": (ctypes.c_int, [ctypes.POINTER(_vp)]),
    "mfr_event_destroy": (ctypes.c_int, [_vp]),
    "mfr_event_record": (ctypes.c_int, [_vp, _vp]),
    "mfr_event_elapsed_ms": (ctypes.c_int, [_vp, _vp, ctypes.POINTER(_f32)]),
    "mfr_sgemm": (ctypes.c_int, [_vp, ctypes.POINTER(GemmDesc)]),
    "mfr_sgemm_noalloc": (ctypes.c_int, [_vp, ctypes.POINTER(GemmDesc)]),
    "mfr_sgemm_plan": (ctypes.c_int, [ctypes.c_int, ctypes.POINTER(GemmDesc),
                                      ctypes.POINTER(_i32), ctypes.POINTER(_i32),
                                      ctypes.POINTER(_i32), ctypes.POINTER(_i32)]),
    "mfr_sgemm_rm": (ctypes.c_int, [_vp, ctypes.c_int, ctypes.c_int, _i64, _i64, _i64, _f32, _vp,
                                    _i64, _vp, _i64, _f32, _vp, _vp, _i64]),
    "mfr_sgemv": (ctypes.c_int, [_vp, ctypes.c_int, _i64, _i64, _f32, _vp, _i64, _vp, _f32, _vp,
                                 _vp]),
    "mfr_smatvec": (ctypes.c_int, [_vp, _i64, _i64, _vp, _i64, _vp, _vp]),
    "mfr_sdot": (ctypes.c_int, [_vp, _i64, _vp, _vp, _vp]),
    "mfr_bias_act": (ctypes.c_int, [_vp, _vp, _vp, _vp, _i64, _i64, ctypes.c_int]),
    "mfr_where": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, _i64]),
    "mfr_where_nd": (ctypes.c_int, [_vp, _i32, ctypes.POINTER(_i64), _vp, ctypes.POINTER(_i64),
                                    _vp, ctypes.POINTER(_i64), _vp, ctypes.POINTER(_i64), _vp]),
    "mfr_softmax": (ctypes.c_int, [_vp, _vp, _vp, _i64, _i64, _i64]),
    "mfr_argmax": (ctypes.c_int, [_vp, _vp, _vp, _i64, _i64]),
    "mfr_elementwise": (ctypes.c_int, [_vp, ctypes.c_int, _vp, _vp, _f32, _vp, _i64]),
    "mfr_attention": (ctypes.c_int, [_vp, ctypes.POINTER(AttentionDesc)]),
    "mfr_strided_copy": (ctypes.c_int, [_vp, _vp, _vp, _i32, _i32, ctypes.POINTER(_i64),
                                        ctypes.POINTER(_i64)]),
    "mfr_fill": (ctypes.c_int, [_vp, _vp, _i32, _i64, ctypes.c_uint64]),
}

_lib = None


def load() -> ctypes.CDLL:
    """The loaded library; raises ImportError if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"{LIB_PATH} is missing: build it with `python -m mensurflow_amd.build` "
            "(there is no CPU fallback)")
    lib = ctypes.CDLL(LIB_PATH)
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    _lib = lib
    return lib


def last_error() -> str:
    msg = load().mfr_last_error()
    return msg.decode() if msg else ""


def check(status: int, what: str = "") -> None:
    """Raise the exception the reference would throw for a nonzero status."""
    if status == MFR_OK:
        return
    message = last_error() or f"{what} failed with status {status}"
    if status == MFR_E_INVALID:
        raise ValueError(message)
    if status == MFR_E_UNSUPPORTED:
        raise NotImplementedError(message)
    raise RuntimeError(message)
