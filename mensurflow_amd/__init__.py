"""mensurflow_amd -- an MI355X (gfx950) backend for mensurflow's fp32 BLAS hot path.

The product is two native libraries built in-tree (``mensurflow_amd/build.py``):

* ``_lib/libmfr_rocm.so``: hand-written HIP kernels behind the C ABI of
  ``include/mfr_rocm.h`` (fp32-MFMA GEMM with a fused epilogue, HBM-bound gemv, softmax,
  where, bias+gelu, argmax, strided copy);
* ``_lib/libmensurflow.so``: the C++17 host layer that plugs those kernels into mensurflow's
  ``Backend``/``Dispatcher`` API as the ``rocm`` device.

This Python module is a thin driver over the C ABI (device buffers, streams, events and the
compute entry points), used by the tests and ``bench.py``. It has no CPU fallback: without the
library, or without a gfx950 device, every call raises.
"""
from __future__ import annotations

import ctypes
import threading
from dataclasses import dataclass

import numpy as np

from . import abi
from .abi import ACT_GELU_ERF, ACT_GELU_TANH, ACT_NONE, GemmDesc  # noqa: F401

__all__ = [
    "ACT_NONE", "ACT_GELU_TANH", "ACT_GELU_ERF", "GemmDesc", "device_count", "device_info",
    "Stream", "DeviceArray", "Event", "sgemm", "gemm", "gemm_batched", "sgemv", "matvec", "dot",
    "bias_act", "where", "where_nd", "elementwise", "softmax", "argmax", "strided_copy", "fill", "attention",
    "attention_fused", "attention_composed", "gemm_plan",
]


def device_count() -> int:
    """Usable gfx950 devices (0 without a driver or device)."""
    lib = abi.load()
    n = ctypes.c_int(0)
    abi.check(lib.mfr_get_device_count(ctypes.byref(n)), "mfr_get_device_count")
    return n.value


@dataclass
class DeviceInfo:
    name: str
    memory_bytes: int
    compute_units: int
    clock_khz: int


def device_info(device: int = 0) -> DeviceInfo:
    lib = abi.load()
    name = ctypes.create_string_buffer(256)
    mem = ctypes.c_size_t(0)
    cus = ctypes.c_int(0)
    clk = ctypes.c_int(0)
    abi.check(lib.mfr_get_device_info(device, name, 256, ctypes.byref(mem), ctypes.byref(cus),
                                      ctypes.byref(clk)), "mfr_get_device_info")
    return DeviceInfo(name.value.decode(), mem.value, cus.value, clk.value)


class Stream:
    """An mfr_stream_t: one HIP stream on one device with its kernel workspace.

    The stream keeps the device memory of arrays released on it for its later allocations.
    Kernels and copies on one stream run in order, so work on a new array that takes a released
    block is queued after every use of the old array, and neither the release nor the allocation
    waits for the device (hipFree waits for the whole device; hipMalloc of a large block costs
    tens of microseconds). Blocks come in size classes (powers of two below 1 MiB, at least
    512 B; multiples of 2 MiB above); idle blocks are kept up to 1/8 of the device's memory
    (at least 1 GiB), past that a released block is freed. An array used by work queued on
    another stream must be released only after that work is done, as before."""

    _SMALL = 1 << 20
    _LARGE_STEP = 2 << 20

    def __init__(self, device: int = 0):
        lib = abi.load()
        self.device = device
        handle = ctypes.c_void_p()
        abi.check(lib.mfr_stream_create(device, ctypes.byref(handle)), "mfr_stream_create")
        self.handle = handle
        self._scratch: dict = {}
        self._idle: dict = {}
        self._idle_bytes = 0
        self._pool_lock = threading.Lock()   # host threads may share a stream
        mem = ctypes.c_size_t(0)
        lib.mfr_get_device_info(device, None, 0, ctypes.byref(mem), None, None)
        self._idle_limit = max(mem.value // 8, 1 << 30)

    @classmethod
    def size_class(cls, nbytes: int) -> int:
        if nbytes >= cls._SMALL:
            return (nbytes + cls._LARGE_STEP - 1) // cls._LARGE_STEP * cls._LARGE_STEP
        size = 512
        while size < nbytes:
            size *= 2
        return size

    def _take(self, size: int) -> int:
        """A device block of `size` bytes (a size class): an idle one, else a new allocation."""
        with self._pool_lock:
            blocks = self._idle.get(size)
            if blocks:
                self._idle_bytes -= size
                return blocks.pop()
        lib = abi.load()
        ptr = ctypes.c_void_p()
        if lib.mfr_malloc(self.device, size, ctypes.byref(ptr)) != abi.MFR_OK:
            self.release_idle()
            abi.check(lib.mfr_malloc(self.device, size, ctypes.byref(ptr)), "mfr_malloc")
        return ptr.value or 0

    def _give(self, size: int, ptr: int) -> None:
        with self._pool_lock:
            if self.handle is not None and self._idle_bytes + size <= self._idle_limit:
                self._idle.setdefault(size, []).append(ptr)
                self._idle_bytes += size
                return
        if self.handle is not None:
            self.synchronize()
        abi.check(abi.load().mfr_free(self.device, ptr), "mfr_free")

    def release_idle(self) -> None:
        """Free the idle blocks (after the work queued on the stream is done)."""
        if not self._idle:
            return
        if self.handle is not None:
            self.synchronize()
        lib = abi.load()
        with self._pool_lock:
            idle, self._idle, self._idle_bytes = self._idle, {}, 0
        for blocks in idle.values():
            for ptr in blocks:
                abi.check(lib.mfr_free(self.device, ptr), "mfr_free")

    def scratch(self, tag, shape, dtype=np.float32) -> "DeviceArray":
        """A device array of `shape` for temporaries of work queued on this stream. Each tag
        keeps one allocation between calls, replaced by a larger one when a call needs more.
        Work on one stream runs in order, so the temporaries of an earlier call are no longer
        read when later work on this stream writes them. The contents are whatever the last
        user of the tag left there."""
        dtype = np.dtype(dtype)
        nbytes = int(np.prod(shape, dtype=np.int64)) * dtype.itemsize
        held = self._scratch.get(tag)
        if held is None or held.nbytes_alloc < nbytes:
            if held is not None:
                held.close()
            held = DeviceArray((max(nbytes, 1),), np.uint8, self)
            self._scratch[tag] = held
        return DeviceArray(shape, dtype, self, _base=held, _ptr=held._ptr)

    def synchronize(self) -> None:
        abi.check(abi.load().mfr_stream_sync(self.handle), "mfr_stream_sync")

    def hip_stream(self) -> int:
        return abi.load().mfr_stream_handle(self.handle) or 0

    def close(self) -> None:
        for held in self._scratch.values():
            held.close()
        self._scratch.clear()
        self.release_idle()
        if self.handle is not None and self.handle.value:
            abi.check(abi.load().mfr_stream_destroy(self.handle), "mfr_stream_destroy")
        self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Event:
    def __init__(self):
        handle = ctypes.c_void_p()
        abi.check(abi.load().mfr_event_create(ctypes.byref(handle)), "mfr_event_create")
        self.handle = handle

    def record(self, stream: Stream) -> None:
        abi.check(abi.load().mfr_event_record(self.handle, stream.handle), "mfr_event_record")

    def elapsed_ms(self, end: "Event") -> float:
        ms = ctypes.c_float(0.0)
        abi.check(abi.load().mfr_event_elapsed_ms(self.handle, end.handle, ctypes.byref(ms)),
                  "mfr_event_elapsed_ms")
        return ms.value

    def __del__(self):
        try:
            if self.handle is not None and self.handle.value:
                abi.load().mfr_event_destroy(self.handle)
            self.handle = None
        except Exception:
            pass


class DeviceArray:
    """A contiguous device allocation viewed with numpy-style shape and element strides.

    Views (``transpose``, ``T``, ``view``, ``slice_rows``) share the allocation; the owner frees
    it when it is garbage collected or closed.
    """

    def __init__(self, shape, dtype=np.float32, stream: Stream | None = None, *, _base=None,
                 _offset=0, _strides=None, _ptr=None):
        self.shape = tuple(int(s) for s in shape)
        self.dtype = np.dtype(dtype)
        self.stream = stream
        self._base = _base
        self.offset = int(_offset)  # elements from the allocation start
        if _strides is None:
            strides, step = [], 1
            for s in reversed(self.shape):
                strides.append(step)
                step *= s
            _strides = tuple(reversed(strides))
        self.strides = tuple(int(s) for s in _strides)
        if _base is None:
            nbytes = int(np.prod(self.shape, dtype=np.int64)) * self.dtype.itemsize
            if stream is not None and stream.handle is not None and nbytes > 0:
                # A block of the stream's pool, returned to it by close().
                self.nbytes_alloc = Stream.size_class(nbytes)
                self._ptr = stream._take(self.nbytes_alloc)
                self._device = stream.device
            else:
                self.nbytes_alloc = nbytes
                ptr = ctypes.c_void_p()
                dev = stream.device if stream is not None else 0
                abi.check(abi.load().mfr_malloc(dev, nbytes, ctypes.byref(ptr)), "mfr_malloc")
                self._ptr = ptr.value or 0
                self._device = dev
            self._pooled = self._ptr != 0 and stream is not None and stream.handle is not None
        else:
            self._ptr = _ptr
            self._device = _base._device

    # -- construction --------------------------------------------------------------------------
    @classmethod
    def from_numpy(cls, array: np.ndarray, stream: Stream) -> "DeviceArray":
        host = np.ascontiguousarray(array)
        out = cls(host.shape, host.dtype, stream)
        out.upload(host)
        return out

    @classmethod
    def empty(cls, shape, stream: Stream, dtype=np.float32) -> "DeviceArray":
        return cls(shape, dtype, stream)

    # -- data movement ---------------------------------------------------------------------------
    @property
    def ptr(self) -> int:
        """Device address of the first element of this view."""
        return self._ptr + self.offset * self.dtype.itemsize

    @property
    def size(self) -> int:
        return int(np.prod(self.shape, dtype=np.int64))

    def is_contiguous(self) -> bool:
        step = 1
        for s, st in zip(reversed(self.shape), reversed(self.strides)):
            if s != 1 and st != step:
                return False
            step *= s
        return True

    def upload(self, host: np.ndarray) -> None:
        if not self.is_contiguous():
            raise ValueError("upload needs a contiguous view")
        host = np.ascontiguousarray(host, dtype=self.dtype)
        if host.shape != self.shape:
            raise ValueError(f"upload: host shape {host.shape} differs from {self.shape}")
        abi.check(abi.load().mfr_memcpy_h2d(self.stream.handle, self.ptr, host.ctypes.data,
                                            host.nbytes), "mfr_memcpy_h2d")

    def numpy(self) -> np.ndarray:
        """Copy to the host (waits for queued work), following strides for views."""
        if self.is_contiguous():
            out = np.empty(self.shape, dtype=self.dtype)
            abi.check(abi.load().mfr_memcpy_d2h(self.stream.handle, out.ctypes.data, self.ptr,
                                                out.nbytes), "mfr_memcpy_d2h")
            return out
        packed = strided_copy(self)
        return packed.numpy()

    # -- views -------------------------------------------------------------------------------------
    def _view(self, shape, strides, offset) -> "DeviceArray":
        base = self._base if self._base is not None else self
        v = DeviceArray(shape, self.dtype, self.stream, _base=base, _offset=offset,
                        _strides=strides, _ptr=self._ptr)
        return v

    def transpose(self, d0=-2, d1=-1) -> "DeviceArray":
        nd = len(self.shape)
        d0 %= nd
        d1 %= nd
        shape = list(self.shape)
        strides = list(self.strides)
        shape[d0], shape[d1] = shape[d1], shape[d0]
        strides[d0], strides[d1] = strides[d1], strides[d0]
        return self._view(shape, strides, self.offset)

    @property
    def T(self) -> "DeviceArray":
        return self.transpose(-2, -1)

    def view(self, shape) -> "DeviceArray":
        if not self.is_contiguous():
            raise ValueError("view: the array is not contiguous")
        shape = list(shape)
        if -1 in shape:
            i = shape.index(-1)
            rest = int(np.prod([s for j, s in enumerate(shape) if j != i], dtype=np.int64))
            shape[i] = self.size // rest
        if int(np.prod(shape, dtype=np.int64)) != self.size:
            raise ValueError(f"view: cannot view {self.shape} as {tuple(shape)}")
        strides, step = [], 1
        for s in reversed(shape):
            strides.append(step)
            step *= s
        return self._view(shape, tuple(reversed(strides)), self.offset)

    def expand(self, shape) -> "DeviceArray":
        shape = tuple(int(s) for s in shape)
        lead = len(shape) - len(self.shape)
        strides = [0] * lead
        for i, (s, st) in enumerate(zip(self.shape, self.strides)):
            want = shape[lead + i]
            if s == want:
                strides.append(st)
            elif s == 1:
                strides.append(0)
            else:
                raise ValueError(f"cannot expand {self.shape} to {shape}")
        return self._view(shape, strides, self.offset)

    def slice(self, dim, start, end) -> "DeviceArray":
        shape = list(self.shape)
        shape[dim] = end - start
        return self._view(shape, self.strides, self.offset + start * self.strides[dim])

    def close(self) -> None:
        if self._base is None and self._ptr:
            ptr, self._ptr = self._ptr, 0
            if self._pooled and self.stream.handle is not None:
                # Later users of the block are queued after the work still using this array.
                self.stream._give(self.nbytes_alloc, ptr)
                return
            # Kernels queued on the stream may still read or write this memory.
            if self.stream is not None and self.stream.handle is not None:
                self.stream.synchronize()
            abi.check(abi.load().mfr_free(self._device, ptr), "mfr_free")

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# ---- compute entry points -------------------------------------------------------------------------


def _ptr_or_none(arr):
    return None if arr is None else arr.ptr


def sgemm(stream: Stream, desc: GemmDesc) -> None:
    """mfr_sgemm on a filled descriptor."""
    abi.check(abi.load().mfr_sgemm(stream.handle, ctypes.byref(desc)), "mfr_sgemm")


def _fill_batch(field, values, dims):
    for i in range(dims):
        field[i] = int(values[i])


def gemm_batched(a: DeviceArray, b: DeviceArray, c: DeviceArray, *, alpha=1.0,
                 c0: DeviceArray | None = None, beta=0.0, bias: DeviceArray | None = None,
                 act=ACT_NONE, tile=0, stage=0, splits=0, causal=False) -> None:
    """c[...] = act(alpha*a@b + beta*c0 + bias) over the leading (batch) dimensions.

    a is [..., m, k], b is [..., k, n] (any strides with a unit stride in one matrix dimension;
    batch strides may be 0), c and c0 are [..., m, n] with unit column stride. The batch shapes
    must already agree (expand them first). tile is an abi.TILE_* value, stage an abi.STAGE_*
    value (copy operands that 16-byte loads cannot read into an aligned workspace first), splits
    the number of depth ranges (0 = automatic, 1 = none; split-K, abi.MAX_SPLITS at most).
    causal: c[..., i, j] = -inf wherever j > i (abi.GEMM_CAUSAL, attention's scores); only the
    panel path takes it, NotImplementedError elsewhere.
    """
    sgemm(c.stream, _gemm_desc(a, b, c, alpha, c0, beta, bias, act, tile, stage, splits,
                               causal))


def gemm_plan(a: DeviceArray, b: DeviceArray, c: DeviceArray, *, tile=0, stage=0, splits=0,
              c0: DeviceArray | None = None, beta=0.0,
              causal=False) -> tuple[int, int, int, int]:
    """(tile, stage, splits, regions) that gemm_batched(a, b, c, ...) would run with
    (mfr_sgemm_plan): AUTO resolved to a fixed tile, stage reported as STAGE_ALWAYS (operands
    copied first) or STAGE_NEVER, splits the depth ranges (1 = no split) -- both of the main
    region -- and regions the output rectangles launched separately (more than 1 when AUTO peels
    edge strips). Raises as gemm_batched would for a point that cannot run."""
    d = _gemm_desc(a, b, c, 1.0, c0, beta, None, ACT_NONE, tile, stage, splits, causal)
    t, st, sp, rg = ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int32()
    abi.check(abi.load().mfr_sgemm_plan(c.stream.device, ctypes.byref(d), ctypes.byref(t),
                                        ctypes.byref(st), ctypes.byref(sp), ctypes.byref(rg)),
              "mfr_sgemm_plan")
    return t.value, st.value, sp.value, rg.value


def _gemm_desc(a, b, c, alpha, c0, beta, bias, act, tile, stage, splits=0,
               causal=False) -> GemmDesc:
    m, k = a.shape[-2:]
    k2, n = b.shape[-2:]
    if k != k2:
        raise ValueError(f"inner dimensions differ: {a.shape} x {b.shape}")
    batch = c.shape[:-2]
    dims = len(batch)
    if dims > abi.MAX_BATCH_DIMS:
        raise ValueError("too many batch dimensions")
    for t in (a, b) + ((c0,) if c0 is not None else ()):
        if t.shape[:-2] != batch:
            raise ValueError(f"batch shapes differ: {t.shape} vs {c.shape}")
    if c.strides[-1] != 1 or (c0 is not None and c0.strides[-1] != 1):
        raise ValueError("c and c0 need a unit column stride")
    d = GemmDesc()
    d.m, d.n, d.k = m, n, k
    d.batch_dims = dims
    d.act = act
    _fill_batch(d.batch, batch, dims)
    d.a = a.ptr
    d.a_rs, d.a_cs = a.strides[-2], a.strides[-1]
    _fill_batch(d.a_bs, a.strides[:-2], dims)
    d.b = b.ptr
    d.b_rs, d.b_cs = b.strides[-2], b.strides[-1]
    _fill_batch(d.b_bs, b.strides[:-2], dims)
    d.c = c.ptr
    d.c_rs = c.strides[-2]
    _fill_batch(d.c_bs, c.strides[:-2], dims)
    if c0 is not None:
        d.c0 = c0.ptr
        d.c0_rs = c0.strides[-2]
        _fill_batch(d.c0_bs, c0.strides[:-2], dims)
    d.bias = _ptr_or_none(bias)
    d.alpha = alpha
    d.beta = beta
    d.tile = tile
    d.stage = stage
    d.splits = splits
    d.flags = abi.GEMM_CAUSAL if causal else 0
    return d


def gemm(a: DeviceArray, b: DeviceArray, *, alpha=1.0, c0: DeviceArray | None = None, beta=0.0,
         trans_a=False, trans_b=False, bias: DeviceArray | None = None, act=ACT_NONE,
         out: DeviceArray | None = None, tile=0, stage=0, splits=0) -> DeviceArray:
    """mensurflow::gemm's semantics (plus the fused bias/activation): a new [m, n] result."""
    left = a.T if trans_a else a
    right = b.T if trans_b else b
    m, n = left.shape[-2], right.shape[-1]
    if out is None:
        out = DeviceArray.empty((m, n), a.stream)
    gemm_batched(left, right, out, alpha=alpha, c0=c0, beta=beta, bias=bias, act=act, tile=tile,
                 stage=stage, splits=splits)
    return out


def sgemv(a: DeviceArray, x: DeviceArray, *, alpha=1.0, y0: DeviceArray | None = None, beta=0.0,
          trans=False, out: DeviceArray | None = None) -> DeviceArray:
    rows, cols = a.shape
    if a.strides[1] != 1:
        raise ValueError("gemv needs a row-major matrix (unit column stride)")
    n_out = cols if trans else rows
    if out is None:
        out = DeviceArray.empty((n_out,), a.stream)
    abi.check(abi.load().mfr_sgemv(a.stream.handle, 1 if trans else 0, rows, cols, alpha, a.ptr,
                                   a.strides[0], x.ptr, beta, _ptr_or_none(y0), out.ptr),
              "mfr_sgemv")
    return out


def matvec(a: DeviceArray, x: DeviceArray, out: DeviceArray | None = None) -> DeviceArray:
    m, k = a.shape
    if out is None:
        out = DeviceArray.empty((m,), a.stream)
    abi.check(abi.load().mfr_smatvec(a.stream.handle, m, k, a.ptr, a.strides[0], x.ptr, out.ptr),
              "mfr_smatvec")
    return out


def dot(x: DeviceArray, y: DeviceArray, out: DeviceArray | None = None) -> DeviceArray:
    """mensurflow::dot (src/ops/blas.cpp:41-68) through mfr_sdot: sum of x[i] * y[i] over two
    contiguous vectors of equal length, the products and their sum in double, rounded once; a
    0-d array."""
    if x.size != y.size:
        raise ValueError(f"dot: lengths differ ({x.size} and {y.size})")
    if out is None:
        out = DeviceArray.empty((), x.stream)
    abi.check(abi.load().mfr_sdot(x.stream.handle, x.size, x.ptr, y.ptr, out.ptr), "mfr_sdot")
    return out


def bias_act(x: DeviceArray, bias: DeviceArray | None, act=ACT_NONE,
             out: DeviceArray | None = None) -> DeviceArray:
    rows, cols = (x.shape if len(x.shape) == 2 else (1, x.size))
    if out is None:
        out = DeviceArray.empty(x.shape, x.stream)
    abi.check(abi.load().mfr_bias_act(x.stream.handle, x.ptr, _ptr_or_none(bias), out.ptr, rows,
                                      cols, act), "mfr_bias_act")
    return out


def where(cond: DeviceArray, x: DeviceArray, y: DeviceArray,
          out: DeviceArray | None = None) -> DeviceArray:
    if out is None:
        out = DeviceArray.empty(x.shape, x.stream)
    abi.check(abi.load().mfr_where(x.stream.handle, cond.ptr, x.ptr, y.ptr, out.ptr, x.size),
              "mfr_where")
    return out


def where_nd(cond: DeviceArray, x: DeviceArray, y: DeviceArray,
             out: DeviceArray | None = None) -> DeviceArray:
    """out = cond ? x : y with each operand read through its own strides (mfr_where_nd): cond,
    x and y are views of out's shape, expanded (stride 0) where they broadcast."""
    shape = out.shape if out is not None else x.shape
    for t in (cond, x, y):
        if t.shape != shape:
            raise ValueError(f"where_nd: operand shape {t.shape} differs from {shape}")
    if out is None:
        out = DeviceArray.empty(shape, x.stream)
    nd = len(shape)
    arr = ctypes.c_int64 * max(nd, 1)
    abi.check(abi.load().mfr_where_nd(x.stream.handle, nd, arr(*shape), cond.ptr,
                                      arr(*cond.strides), x.ptr, arr(*x.strides), y.ptr,
                                      arr(*y.strides), out.ptr), "mfr_where_nd")
    return out


def elementwise(op: int, a: DeviceArray, b: DeviceArray | None = None, alpha=1.0,
                out: DeviceArray | None = None) -> DeviceArray:
    """out = a + b (abi.EW_ADD), a - b (abi.EW_SUB), a * b (abi.EW_MUL) or alpha * a
    (abi.EW_SCAL, b unused) over contiguous arrays of a's size (mfr_elementwise)."""
    if out is None:
        out = DeviceArray.empty(a.shape, a.stream)
    b_ptr = None if b is None else b.ptr
    abi.check(abi.load().mfr_elementwise(a.stream.handle, op, a.ptr, b_ptr, alpha, out.ptr,
                                         a.size), "mfr_elementwise")
    return out


def softmax(x: DeviceArray, axis=-1, out: DeviceArray | None = None) -> DeviceArray:
    shape = x.shape if x.shape else (1,)
    axis %= len(shape)
    outer = int(np.prod(shape[:axis], dtype=np.int64))
    length = int(shape[axis])
    inner = int(np.prod(shape[axis + 1:], dtype=np.int64))
    if out is None:
        out = DeviceArray.empty(x.shape, x.stream)
    abi.check(abi.load().mfr_softmax(x.stream.handle, x.ptr, out.ptr, outer, length, inner),
              "mfr_softmax")
    return out


def argmax(x: DeviceArray, out: DeviceArray | None = None) -> DeviceArray:
    width = x.shape[-1]
    rows = x.size // width if width else int(np.prod(x.shape[:-1], dtype=np.int64))
    if out is None:
        out = DeviceArray.empty(x.shape[:-1], x.stream, np.int64)
    abi.check(abi.load().mfr_argmax(x.stream.handle, x.ptr, out.ptr, rows, width), "mfr_argmax")
    return out


def strided_copy(x: DeviceArray, out: DeviceArray | None = None) -> DeviceArray:
    if out is None:
        out = DeviceArray.empty(x.shape, x.stream, x.dtype)
    nd = len(x.shape)
    shape = (ctypes.c_int64 * max(nd, 1))(*x.shape)
    strides = (ctypes.c_int64 * max(nd, 1))(*x.strides)
    abi.check(abi.load().mfr_strided_copy(x.stream.handle, x.ptr, out.ptr, x.dtype.itemsize, nd,
                                          shape, strides), "mfr_strided_copy")
    return out


def fill(x: DeviceArray, value) -> None:
    bits = np.array([value], dtype=x.dtype).view(
        {1: np.uint8, 2: np.uint16, 4: np.uint32, 8: np.uint64}[x.dtype.itemsize])[0]
    abi.check(abi.load().mfr_fill(x.stream.handle, x.ptr, x.dtype.itemsize, x.size, int(bits)),
              "mfr_fill")


def attention_fused(q: DeviceArray, k: DeviceArray, v: DeviceArray,
                    mask: DeviceArray | None = None, causal: bool = False, scale: float = 0.0,
                    out: DeviceArray | None = None) -> DeviceArray:
    """mfr_attention: the whole op in one kernel (online softmax, no score matrix). q [..., Lq, D],
    k and v [..., Lk, D] with equal batch shapes (stride 0 for broadcast), D a multiple of 16 up to
    128;
    mask a uint8 array broadcastable to [..., Lq, Lk]. Raises NotImplementedError for layouts
    the kernel does not take."""
    lq, depth = q.shape[-2:]
    lk = k.shape[-2]
    batch = q.shape[:-2]
    dims = len(batch)
    if dims > abi.MAX_BATCH_DIMS:
        raise ValueError("too many batch dimensions")
    if k.shape != batch + (lk, depth) or v.shape != batch + (lk, depth):
        raise ValueError(f"attention: q {q.shape}, k {k.shape}, v {v.shape} do not agree")
    for t in (q, k, v):
        if t.strides[-1] != 1:
            raise NotImplementedError("attention: fused kernel needs unit stride along d")
    if out is None:
        out = DeviceArray.empty(batch + (lq, depth), q.stream)
    d = abi.AttentionDesc()
    d.lq, d.lk, d.d = lq, lk, depth
    d.batch_dims = dims
    d.causal = 1 if causal else 0
    _fill_batch(d.batch, batch, dims)
    for name, t in (("q", q), ("k", k), ("v", v), ("out", out)):
        setattr(d, name, t.ptr)
        setattr(d, name + "_rs", t.strides[-2])
        _fill_batch(getattr(d, name + "_bs"), t.strides[:-2], dims)
    if mask is not None:
        full = mask.expand(batch + (lq, lk))
        d.mask = full.ptr
        d.mask_rs, d.mask_cs = full.strides[-2], full.strides[-1]
        _fill_batch(d.mask_bs, full.strides[:-2], dims)
    d.scale = scale
    abi.check(abi.load().mfr_attention(q.stream.handle, ctypes.byref(d)), "mfr_attention")
    return out


def attention(q: DeviceArray, k: DeviceArray, v: DeviceArray, mask: DeviceArray | None = None,
              causal: bool = False, scale: float = 0.0, fused: bool | None = None) -> DeviceArray:
    """mensurflow::attention (src/ops/attention.cpp:48-98). fused=None runs the fused kernel
    (attention_fused) when it takes the layout and the composition otherwise; True only the
    fused kernel; False only the composition."""
    if fused is not False:
        try:
            return attention_fused(q, k, v, mask=mask, causal=causal, scale=scale)
        except NotImplementedError:
            if fused:
                raise
    return attention_composed(q, k, v, mask=mask, causal=causal, scale=scale)


def attention_composed(q: DeviceArray, k: DeviceArray, v: DeviceArray,
                       mask: DeviceArray | None = None, causal: bool = False,
                       scale: float = 0.0) -> DeviceArray:
    """mensurflow::attention's composition on the device (src/ops/attention.cpp:48-98): scores =
    gemm_batched(q, k^T, alpha=scale), where(mask, scores, -inf) with the mask and the -inf
    scalar read through broadcast views (mfr_where_nd; mensurflow::where packs them to the
    scores' shape), the causal mask the same way, softmax over the keys, gemm_batched(weights,
    v). The causal mask is the scores GEMM's own (causal=True: the same bits as the where over
    the lower triangle, without the pass over the scores) where the GEMM takes it, the where
    otherwise. q [..., Lq, D], k [..., Lk, D], v [..., Lk, Dv] with equal batch shapes; mask a
    Bool (uint8) array broadcastable to [..., Lq, Lk]. Every array is on q's stream; the scores
    are that stream's scratch array, reused by later calls."""
    stream = q.stream
    lq, depth = q.shape[-2:]
    lk = k.shape[-2]
    batch = q.shape[:-2]
    if scale == 0.0:
        scale = float(np.float32(1.0 / np.sqrt(depth))) if depth > 0 else 1.0
    scores = stream.scratch("attention.scores", batch + (lq, lk))
    causal_done = False
    if causal:
        try:
            gemm_batched(q, k.transpose(-2, -1), scores, alpha=scale, causal=True)
            causal_done = True
        except NotImplementedError:
            pass
    if not causal_done:
        gemm_batched(q, k.transpose(-2, -1), scores, alpha=scale)
    minus_inf = None

    def masked(keep: DeviceArray) -> DeviceArray:
        nonlocal minus_inf
        if minus_inf is None:
            minus_inf = stream.scratch("attention.scalar", (1,))
            fill(minus_inf, -np.inf)
        return where_nd(keep.expand(scores.shape), scores, minus_inf.expand(scores.shape),
                        out=scores)

    if mask is not None:
        masked(mask)
    if causal and not causal_done:
        # The [Lq, Lk] lower triangle, kept on the stream until a call needs another shape.
        lower = stream._scratch.get("attention.causal")
        if lower is None or lower.shape != (lq, lk):
            if lower is not None:
                lower.close()
            lower = DeviceArray.from_numpy(np.tril(np.ones((lq, lk), dtype=np.uint8)), stream)
            stream._scratch["attention.causal"] = lower
        masked(lower)
    weights = softmax(scores, axis=-1, out=scores)
    out = DeviceArray.empty(batch + (lq, v.shape[-1]), stream)
    gemm_batched(weights, v, out)
    return out
