"""Device tensors: a pooled device allocation plus a numpy-style view.

A :class:`DeviceTensor` is (storage, element offset, shape, element strides,
dtype).  Views (reshape of a contiguous tensor, transpose, slice, squeeze,
unsqueeze, broadcast) share storage exactly as the numpy views returned by
the reference's Reshape/Transpose/Squeeze/Unsqueeze/Slice/Split branches do
(tools/ref_runtime.py:511-549).  Storage comes from libkk's bucketed pool
(kk_alloc/kk_free) and goes back to it when the last view is dropped.
"""
import ctypes
import functools
import math

import numpy as np

from . import _lib

NP_TO_CODE = {
    np.dtype(np.float32): _lib.F32, np.dtype(np.int8): _lib.I8,
    np.dtype(np.uint8): _lib.U8, np.dtype(np.int32): _lib.I32,
    np.dtype(np.int64): _lib.I64, np.dtype(np.bool_): _lib.BOOL,
    np.dtype(np.float16): _lib.F16,
}
CODE_TO_NP = {v: k for k, v in NP_TO_CODE.items()}

_state = {"device": None, "downloads": 0}  # downloads: DeviceTensor.numpy calls so far


def init(device=0):
    """Initialise libkk on `device` (idempotent)."""
    if _state["device"] is None:
        _lib.call("kk_init", int(device))
        _state["device"] = int(device)
    return _state["device"]


def device_count():
    n = ctypes.c_int(0)
    _lib.call("kk_device_count", ctypes.byref(n))
    return n.value


def sync():
    init()
    _lib.call("kk_sync")


def pool_stats():
    """(live_bytes, pooled_bytes, peak_live_bytes) of the device pool."""
    vals = [ctypes.c_size_t(0) for _ in range(3)]
    _lib.call("kk_pool_stats", *[ctypes.byref(v) for v in vals])
    return tuple(v.value for v in vals)


def dispatch_count():
    """Kernels launched by libkk since init, outside graph recording."""
    n = ctypes.c_uint64(0)
    _lib.call("kk_dispatch_count", ctypes.byref(n))
    return n.value


def pool_trim(budget_bytes=0):
    init()
    _lib.call("kk_pool_trim", int(budget_bytes))


_alloc_out = ctypes.c_void_p()  # out-parameter of kk_alloc (the walk is single-threaded)
_alloc_ref = ctypes.byref(_alloc_out)
_fast = {}  # bound entry points of the allocation path


class Storage:
    """One pooled device buffer."""

    __slots__ = ("ptr", "nbytes", "__weakref__")

    def __init__(self, nbytes):
        if _state["device"] is None:
            init()
        alloc = _fast.get("kk_alloc")
        if alloc is None:
            alloc = _fast["kk_alloc"] = _lib.load().kk_alloc
        nbytes = int(nbytes)
        rc = alloc(nbytes if nbytes > 0 else 1, _alloc_ref)
        if rc:
            _lib.raise_error("kk_alloc", rc)
        self.ptr = _alloc_out.value
        self.nbytes = nbytes

    def __del__(self):
        ptr, self.ptr = getattr(self, "ptr", None), None
        if ptr and _lib._lib is not None:
            try:
                _lib._lib.kk_free(ptr)
            except Exception:  # interpreter shutdown: the process frees it
                pass


_PROTOS = {}  # (shape, strides, dtype) -> KKTensor with data unset


@functools.lru_cache(maxsize=4096)
def _contig_strides(shape):
    st, acc = [], 1
    for d in reversed(shape):
        st.append(acc)
        acc *= int(d)
    return tuple(reversed(st))


class DeviceTensor:
    """A strided view of device memory (element strides, numpy semantics)."""

    __slots__ = ("storage", "offset", "shape", "strides", "dtype", "_desc", "host")

    def __init__(self, storage, shape, dtype, strides=None, offset=0):
        self.storage = storage
        self.shape = tuple(map(int, shape))
        self.dtype = dtype if isinstance(dtype, np.dtype) else np.dtype(dtype)
        if self.dtype not in NP_TO_CODE:
            raise TypeError(f"unsupported device dtype {self.dtype}")
        self.strides = tuple(map(int, strides)) if strides is not None \
            else _contig_strides(self.shape)
        self.offset = int(offset)
        self.host = None  # cached host value of a constant uploaded once
        if len(self.shape) > _lib.KK_MAX_RANK:
            raise ValueError(f"rank {len(self.shape)} exceeds {_lib.KK_MAX_RANK}")
        self._desc = None

    # ----------------------------------------------------------- creation
    @classmethod
    def empty(cls, shape, dtype=np.float32):
        shape = tuple(map(int, shape))
        dtype = dtype if isinstance(dtype, np.dtype) else np.dtype(dtype)
        if dtype not in NP_TO_CODE:
            raise TypeError(f"unsupported device dtype {dtype}")
        if len(shape) > _lib.KK_MAX_RANK:
            raise ValueError(f"rank {len(shape)} exceeds {_lib.KK_MAX_RANK}")
        t = object.__new__(cls)  # a fresh contiguous tensor: no view checks
        t.storage = Storage(math.prod(shape) * dtype.itemsize)
        t.shape = shape
        t.dtype = dtype
        t.strides = _contig_strides(shape)
        t.offset = 0
        t.host = None
        t._desc = None
        return t

    @classmethod
    def from_numpy(cls, arr):
        arr = np.asarray(arr)
        if not arr.flags.c_contiguous:  # (np.ascontiguousarray would make 0-d arrays 1-d)
            arr = arr.copy(order="C")
        if arr.dtype not in NP_TO_CODE:
            raise TypeError(f"unsupported dtype {arr.dtype}")
        t = cls.empty(arr.shape, arr.dtype)
        if arr.nbytes:
            _lib.call("kk_upload", ctypes.c_void_p(t.ptr),
                      arr.ctypes.data_as(ctypes.c_void_p), arr.nbytes)
        return t

    # ------------------------------------------------------------ queries
    @property
    def ptr(self):
        return self.storage.ptr + self.offset * self.dtype.itemsize

    @property
    def ndim(self):
        return len(self.shape)

    @property
    def size(self):
        return math.prod(self.shape)

    @property
    def code(self):
        return NP_TO_CODE[self.dtype]

    def is_contiguous(self):
        if self.size == 0:
            return True
        acc = 1
        for d, s in zip(reversed(self.shape), reversed(self.strides)):
            if d != 1 and s != acc:
                return False
            acc *= d
        return True

    def desc(self):
        """The kk_tensor descriptor (cached; views are immutable).  Descriptors
        of one (shape, strides, dtype) differ only in the data pointer: each
        is copied from a cached prototype."""
        if self._desc is None:
            key = (self.shape, self.strides, self.dtype)
            proto = _PROTOS.get(key)
            if proto is None:
                proto = _lib.KKTensor()
                proto.dtype = NP_TO_CODE[self.dtype]
                proto.rank = len(self.shape)
                for i, (n, s) in enumerate(zip(self.shape, self.strides)):
                    proto.shape[i] = n
                    proto.strides[i] = s
                if len(_PROTOS) < 4096:
                    _PROTOS[key] = proto
            d = _lib.KKTensor.from_buffer_copy(proto)
            d.data = self.storage.ptr + self.offset * self.dtype.itemsize
            self._desc = d
        return ctypes.byref(self._desc)

    def __repr__(self):
        return f"DeviceTensor(shape={self.shape}, dtype={self.dtype}, strides={self.strides})"

    # ------------------------------------------------------------- copies
    def contiguous(self):
        if self.is_contiguous():
            return self
        out = DeviceTensor.empty(self.shape, self.dtype)
        _lib.call("kk_copy", out.desc(), self.desc())
        return out

    def astype(self, dtype):
        dtype = np.dtype(dtype)
        out = DeviceTensor.empty(self.shape, dtype)
        _lib.call("kk_copy", out.desc(), self.desc())
        return out

    def numpy(self):
        """Download (waits for all enqueued work)."""
        _state["downloads"] += 1
        src = self.contiguous()
        host = np.empty(self.shape, dtype=self.dtype)
        if host.nbytes:
            _lib.call("kk_download", host.ctypes.data_as(ctypes.c_void_p),
                      ctypes.c_void_p(src.ptr), host.nbytes)
        return host

    # -------------------------------------------------------------- views
    def _view(self, shape, strides, offset=None):
        return DeviceTensor(self.storage, shape, self.dtype, strides,
                            self.offset if offset is None else offset)

    def reshape(self, shape):
        shape = list(int(d) for d in shape)
        if -1 in shape:
            known = math.prod(d for d in shape if d != -1)
            shape[shape.index(-1)] = self.size // known if known else 0
        if math.prod(shape) != self.size:
            raise ValueError(f"cannot reshape {self.shape} into {tuple(shape)}")
        src = self if self.is_contiguous() else self.contiguous()
        return src._view(shape, _contig_strides(tuple(shape)))

    def transpose(self, perm=None):
        if perm is None:
            perm = list(range(self.ndim))[::-1]
        perm = [int(p) % self.ndim for p in perm]
        return self._view([self.shape[p] for p in perm], [self.strides[p] for p in perm])

    def expand_dims(self, axis):
        r = self.ndim + 1
        axis = int(axis) % r if axis < 0 else int(axis)
        shape = list(self.shape)
        strides = list(self.strides)
        # A unit axis is never stepped along; give it the stride a contiguous
        # layout would have.
        inner = self.strides[axis] * self.shape[axis] if axis < self.ndim else 1
        shape.insert(axis, 1)
        strides.insert(axis, inner)
        return self._view(shape, strides)

    def squeeze(self, axes=None):
        if axes is None:
            keep = [i for i, d in enumerate(self.shape) if d != 1]
        else:
            ax = {int(a) % self.ndim for a in axes}
            for a in ax:
                if self.shape[a] != 1:
                    raise ValueError(f"cannot squeeze axis {a} of extent {self.shape[a]}")
            keep = [i for i in range(self.ndim) if i not in ax]
        return self._view([self.shape[i] for i in keep], [self.strides[i] for i in keep])

    def slice_axis(self, axis, start, stop, step=1):
        """View of range(start, stop, step) along `axis` (already clamped)."""
        n = len(range(start, stop, step))
        shape = list(self.shape)
        strides = list(self.strides)
        off = self.offset + (start * self.strides[axis] if n else 0)
        shape[axis] = n
        strides[axis] = self.strides[axis] * step
        return self._view(shape, strides, off)

    def broadcast_to(self, shape):
        shape = tuple(int(d) for d in shape)
        pad = len(shape) - self.ndim
        if pad < 0:
            raise ValueError("cannot broadcast to a lower rank")
        strides = []
        for i, d in enumerate(shape):
            if i < pad:
                strides.append(0)
                continue
            sd = self.shape[i - pad]
            if sd == d:
                strides.append(self.strides[i - pad])
            elif sd == 1:
                strides.append(0)
            else:
                raise ValueError(f"cannot broadcast {self.shape} to {shape}")
        return self._view(shape, strides)
