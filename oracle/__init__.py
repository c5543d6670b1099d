"""CPU oracle for mensurflow's fp32 BLAS hot path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import this package: it is the checker the HIP kernels are compared against, never the thing
measured or shipped. The product (``mensurflow_amd``) never imports it.

Two libraries are wrapped:

* ``liboracle.so`` -- the C restatement of the reference's CPU path (``oracle.c``); each
  function cites the reference file:line it follows.
* ``_ref/libmfref.so`` -- the reference's own CPU kernels compiled from their sources
  (``Makefile``, target ``ref``), present when it was built in a container that holds the
  reference. Used to pin the restatement and as the CPU baseline.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "liboracle.so")
REF_SO = os.path.join(HERE, "_ref", "libmfref.so")

_f32p = ctypes.POINTER(ctypes.c_float)
_f64p = ctypes.POINTER(ctypes.c_double)
_i64 = ctypes.c_int64
_u64 = ctypes.c_uint64
_u8p = ctypes.POINTER(ctypes.c_uint8)
_i64p = ctypes.POINTER(ctypes.c_int64)
_u32p = ctypes.POINTER(ctypes.c_uint32)
_vp = ctypes.c_void_p


def build() -> None:
    """Compile liboracle.so (and _ref/libmfref.so where the reference is present)."""
    subprocess.run(["make", "-s", "-C", HERE, "all"], check=True)


def _ptr(array: np.ndarray | None, kind=_f32p):
    if array is None:
        return None
    return array.ctypes.data_as(kind)


class _Lib:
    """ctypes signatures shared by the restatement (orc_*) and the reference build (ref_*)."""

    def __init__(self, path: str, prefix: str):
        self.path = path
        self.prefix = prefix
        self.lib = ctypes.CDLL(path)
        self._declare()

    def fn(self, name):
        return getattr(self.lib, self.prefix + name)

    def _declare(self):
        p = self.prefix
        L = self.lib
        getattr(L, p + "philox4x32_10").argtypes = [_u32p, _u32p, _u32p]
        getattr(L, p + "uniform_f32").argtypes = [_f32p, _i64, ctypes.c_float, ctypes.c_float,
                                                 _u64, _u64]
        getattr(L, p + "normal_f32").argtypes = [_f32p, _i64, ctypes.c_float, ctypes.c_float,
                                                _u64, _u64]
        getattr(L, p + "matvec_f32").argtypes = [_f32p, _f32p, _f32p, _i64, _i64]
        getattr(L, p + "gemv_f32").argtypes = [_f32p, _f32p, _f32p, _i64, _i64, ctypes.c_float,
                                              ctypes.c_float, _f32p, ctypes.c_int]
        getattr(L, p + "bias_add_f32").argtypes = [_f32p, _f32p, _f32p, _i64, _i64]
        getattr(L, p + "gelu_f32").argtypes = [_f32p, _f32p, _i64, ctypes.c_int]
        getattr(L, p + "where_f32").argtypes = [_u8p, _f32p, _f32p, _f32p, _i64]
        getattr(L, p + "softmax_f32").argtypes = [_f32p, _f32p, _i64, _i64, _i64]
        getattr(L, p + "argmax_f32").argtypes = [_f32p, _i64p, _i64, _i64]
        getattr(L, p + "sub_f32").argtypes = [_f32p, _f32p, _f32p, _i64]
        getattr(L, p + "dot_f32").argtypes = [_f32p, _f32p, _i64]
        getattr(L, p + "dot_f32").restype = ctypes.c_float
        for name in ("philox4x32_10", "uniform_f32", "normal_f32", "matvec_f32", "gemv_f32",
                     "bias_add_f32", "gelu_f32", "where_f32", "softmax_f32", "argmax_f32",
                     "sub_f32"):
            getattr(L, p + name).restype = None

    # -- shared wrappers ------------------------------------------------------------------------
    def philox(self, counter, key):
        c = np.asarray(counter, dtype=np.uint32)
        k = np.asarray(key, dtype=np.uint32)
        out = np.zeros(4, dtype=np.uint32)
        self.fn("philox4x32_10")(_ptr(c, _u32p), _ptr(k, _u32p), _ptr(out, _u32p))
        return out

    def uniform(self, n, low=0.0, high=1.0, seed=0, offset=0):
        out = np.empty(int(n), dtype=np.float32)
        self.fn("uniform_f32")(_ptr(out), n, low, high, seed, offset)
        return out

    def normal(self, n, mean=0.0, stddev=1.0, seed=0, offset=0):
        out = np.empty(int(n), dtype=np.float32)
        self.fn("normal_f32")(_ptr(out), n, mean, stddev, seed, offset)
        return out

    def matvec(self, a, x):
        a = np.ascontiguousarray(a, dtype=np.float32)
        x = np.ascontiguousarray(x, dtype=np.float32)
        y = np.empty(a.shape[0], dtype=np.float32)
        self.fn("matvec_f32")(_ptr(a), _ptr(x), _ptr(y), a.shape[0], a.shape[1])
        return y

    def gemv(self, a, x, alpha=1.0, y0=None, beta=0.0, trans=False):
        a = np.ascontiguousarray(a, dtype=np.float32)
        x = np.ascontiguousarray(x, dtype=np.float32)
        rows, cols = a.shape
        y = np.empty(cols if trans else rows, dtype=np.float32)
        y0c = None if y0 is None else np.ascontiguousarray(y0, dtype=np.float32)
        self.fn("gemv_f32")(_ptr(a), _ptr(x), _ptr(y), rows, cols, alpha, beta, _ptr(y0c),
                            1 if trans else 0)
        return y

    def dot(self, x, y):
        x = np.ascontiguousarray(x, dtype=np.float32)
        y = np.ascontiguousarray(y, dtype=np.float32)
        return np.float32(self.fn("dot_f32")(_ptr(x), _ptr(y), x.size))

    def sub(self, a, b):
        a = np.ascontiguousarray(a, dtype=np.float32)
        b = np.ascontiguousarray(b, dtype=np.float32)
        out = np.empty_like(a)
        self.fn("sub_f32")(_ptr(a), _ptr(b), _ptr(out), a.size)
        return out

    def bias_add(self, x, bias):
        x = np.ascontiguousarray(x, dtype=np.float32)
        bias = np.ascontiguousarray(bias, dtype=np.float32)
        out = np.empty_like(x)
        self.fn("bias_add_f32")(_ptr(x), _ptr(bias), _ptr(out), x.size, bias.size)
        return out

    def gelu(self, x, approximate=True):
        x = np.ascontiguousarray(x, dtype=np.float32)
        out = np.empty_like(x)
        self.fn("gelu_f32")(_ptr(x), _ptr(out), x.size, 1 if approximate else 0)
        return out

    def where(self, cond, x, y):
        cond = np.ascontiguousarray(cond, dtype=np.uint8)
        x = np.ascontiguousarray(x, dtype=np.float32)
        y = np.ascontiguousarray(y, dtype=np.float32)
        out = np.empty_like(x)
        self.fn("where_f32")(_ptr(cond, _u8p), _ptr(x), _ptr(y), _ptr(out), x.size)
        return out

    def softmax(self, x, axis=-1):
        x = np.ascontiguousarray(x, dtype=np.float32)
        axis = axis % x.ndim if x.ndim else 0
        shape = x.shape if x.ndim else (1,)
        outer = int(np.prod(shape[:axis], dtype=np.int64))
        length = int(shape[axis])
        inner = int(np.prod(shape[axis + 1:], dtype=np.int64))
        out = np.empty_like(x)
        self.fn("softmax_f32")(_ptr(x), _ptr(out), outer, length, inner)
        return out

    def argmax(self, x):
        x = np.ascontiguousarray(x, dtype=np.float32)
        width = x.shape[-1]
        rows = x.size // width if width else 0
        out = np.empty(x.shape[:-1], dtype=np.int64)
        self.fn("argmax_f32")(_ptr(x), _ptr(out, _i64p), rows, width)
        return out


class Oracle(_Lib):
    """The C restatement (oracle.c)."""

    def __init__(self):
        if not os.path.exists(ORACLE_SO):
            build()
        super().__init__(ORACLE_SO, "orc_")
        L = self.lib
        L.orc_sgemm_packed.argtypes = [_i64, _i64, _i64, _vp, _i64, _i64, _vp, _i64, _i64, _vp,
                                       _i64, _i64]
        L.orc_sgemm_packed.restype = None
        L.orc_axpby_f32.argtypes = [_f32p, _f32p, ctypes.c_float, _f32p, ctypes.c_float, _i64]
        L.orc_axpby_f32.restype = None
        L.orc_matmul_f64.argtypes = [_i64, _i64, _i64, _vp, _i64, _i64, _vp, _i64, _i64, _f64p,
                                     _f64p]
        L.orc_matmul_f64.restype = None
        L.orc_set_threads.argtypes = [ctypes.c_int]
        L.orc_set_threads.restype = ctypes.c_int

    def set_threads(self, threads: int) -> int:
        return self.lib.orc_set_threads(threads)

    def matmul(self, a, b, kc=768):
        """The packed CPU GEMM's arithmetic on numpy views (any strides, float32)."""
        a = np.asarray(a, dtype=np.float32)
        b = np.asarray(b, dtype=np.float32)
        m, k = a.shape
        k2, n = b.shape
        assert k == k2
        c = np.empty((m, n), dtype=np.float32)
        isz = a.itemsize
        self.lib.orc_sgemm_packed(m, n, k, a.ctypes.data, a.strides[0] // isz,
                                  a.strides[1] // isz, b.ctypes.data, b.strides[0] // isz,
                                  b.strides[1] // isz, c.ctypes.data, n, kc)
        return c

    def axpby(self, x, alpha, y0, beta):
        x = np.ascontiguousarray(x, dtype=np.float32)
        out = np.empty_like(x)
        y0c = None if y0 is None else np.ascontiguousarray(y0, dtype=np.float32)
        self.lib.orc_axpby_f32(_ptr(out), _ptr(x), alpha, _ptr(y0c), beta, x.size)
        return out

    def gemm(self, a, b, alpha=1.0, c0=None, beta=0.0, trans_a=False, trans_b=False, kc=768):
        """mensurflow::gemm's composition: matmul, then alpha, then + beta*c (blas.cpp:234-262)."""
        left = a.T if trans_a else a
        right = b.T if trans_b else b
        return self.axpby(self.matmul(left, right, kc), alpha, c0, beta)

    def matmul_f64(self, a, b):
        """Double-precision product and per-entry magnitude sum_p |a*b|."""
        a = np.asarray(a, dtype=np.float32)
        b = np.asarray(b, dtype=np.float32)
        m, k = a.shape
        n = b.shape[1]
        value = np.empty((m, n), dtype=np.float64)
        magnitude = np.empty((m, n), dtype=np.float64)
        isz = a.itemsize
        self.lib.orc_matmul_f64(m, n, k, a.ctypes.data, a.strides[0] // isz, a.strides[1] // isz,
                                b.ctypes.data, b.strides[0] // isz, b.strides[1] // isz,
                                _ptr(value, _f64p), _ptr(magnitude, _f64p))
        return value, magnitude


class Reference(_Lib):
    """The reference's own CPU kernels (oracle/_ref/libmfref.so)."""

    def __init__(self):
        if not os.path.exists(REF_SO):
            raise FileNotFoundError(f"{REF_SO} is not built (needs the reference sources)")
        super().__init__(REF_SO, "ref_")
        L = self.lib
        L.ref_matmul_packed.argtypes = [_vp, _i64, _i64, _vp, _i64, _i64, _vp, _i64, _i64, _i64,
                                        _i64, ctypes.c_int]
        L.ref_matmul_packed.restype = None
        L.ref_get_kc.restype = _i64
        L.ref_set_kc.argtypes = [_i64]
        L.ref_set_kc.restype = None
        L.ref_set_threads.argtypes = [ctypes.c_int]
        L.ref_set_threads.restype = None
        L.ref_max_threads.restype = ctypes.c_int
        L.ref_packed_supported.restype = ctypes.c_int
        for name in ("ref_mul_f32", "ref_add_f32"):
            getattr(L, name).argtypes = [_f32p, _f32p, _f32p, _i64]
            getattr(L, name).restype = None
        L.ref_scal_f32.argtypes = [ctypes.c_float, _f32p, _f32p, _i64]
        L.ref_scal_f32.restype = None
        L.ref_gemm_batched_f32.argtypes = [_vp, _i64p, _i64, _i64, _vp, _i64p, _i64, _i64, _vp,
                                           _vp, _i64, _i64, _i64, _i64, ctypes.c_float,
                                           ctypes.c_float]
        L.ref_gemm_batched_f32.restype = None

    def packed_supported(self) -> bool:
        return bool(self.lib.ref_packed_supported())

    def get_kc(self) -> int:
        return int(self.lib.ref_get_kc())

    def set_kc(self, kc: int) -> None:
        self.lib.ref_set_kc(kc)

    def set_threads(self, threads: int) -> None:
        self.lib.ref_set_threads(threads)

    def max_threads(self) -> int:
        return int(self.lib.ref_max_threads())

    def matmul(self, a, b, parallel=True, out=None):
        a = np.asarray(a, dtype=np.float32)
        b = np.asarray(b, dtype=np.float32)
        m, k = a.shape
        n = b.shape[1]
        c = np.empty((m, n), dtype=np.float32) if out is None else out
        isz = 4
        self.lib.ref_matmul_packed(a.ctypes.data, a.strides[0] // isz, a.strides[1] // isz,
                                   b.ctypes.data, b.strides[0] // isz, b.strides[1] // isz,
                                   c.ctypes.data, n, m, n, k, 1 if parallel else 0)
        return c


    def _binary(self, name, a, b):
        a = np.ascontiguousarray(a, dtype=np.float32)
        b = np.ascontiguousarray(b, dtype=np.float32)
        out = np.empty_like(a)
        getattr(self.lib, name)(_ptr(a), _ptr(b), _ptr(out), a.size)
        return out

    def gemm_composition(self, product, alpha, c0=None, beta=0.0):
        """mensurflow::gemm after its matmul (src/ops/blas.cpp:246-257), with the reference's
        own kernels: mul by alpha when alpha != 1, then add(result, scal(beta, c0)) when c0 is
        given and beta != 0."""
        result = np.ascontiguousarray(product, dtype=np.float32).copy()
        if alpha != 1.0:
            result = self._binary("ref_mul_f32", result, np.full_like(result, np.float32(alpha)))
        if c0 is not None and beta != 0.0:
            c0 = np.ascontiguousarray(c0, dtype=np.float32)
            scaled = np.empty_like(c0)
            self.lib.ref_scal_f32(beta, _ptr(c0), _ptr(scaled), c0.size)
            result = self._binary("ref_add_f32", result, scaled)
        return result

    def gemm_batched(self, a, b, a_offsets, b_offsets, m, n, k, rsa, csa, rsb, csb, alpha=1.0,
                     c0=None, beta=0.0):
        """gemm_batched_f32_parallel (gemm_batched.cpp:58-70) with its finish pass: one packed
        GEMM per matrix i of A (a.ravel() from a_offsets[i], strides rsa/csa) and B, then
        alpha * C + beta * C0. Returns C [batch, m, n]."""
        a = np.ascontiguousarray(a, dtype=np.float32).ravel()
        b = np.ascontiguousarray(b, dtype=np.float32).ravel()
        ao = np.ascontiguousarray(a_offsets, dtype=np.int64)
        bo = np.ascontiguousarray(b_offsets, dtype=np.int64)
        batch = ao.size
        c = np.empty((batch, m, n), np.float32)
        c0c = None if c0 is None else np.ascontiguousarray(c0, dtype=np.float32)
        self.lib.ref_gemm_batched_f32(a.ctypes.data, _ptr(ao, _i64p), rsa, csa, b.ctypes.data,
                                      _ptr(bo, _i64p), rsb, csb, c.ctypes.data,
                                      None if c0c is None else c0c.ctypes.data, batch, m, n, k,
                                      alpha, beta)
        return c


def has_reference() -> bool:
    return os.path.exists(REF_SO)
