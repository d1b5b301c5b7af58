"""Device memory, streams and events over libc3hip.so.

`DeviceArray` is the array type the registry kernels and the executor pass
around in place of the reference's CuPy arrays (c32/kernel_registry.py:8-16):
a pointer, a shape and a NumPy dtype, always C-contiguous.  Views share the
owner's memory, exactly like the arena views the reference builds with
`byte_view.view(cp.float32)` (c35/executor.py:569-573).

Kernels launch on the *current stream* (`using_stream`), the counterpart of
CuPy's `with stream:` blocks (c35/executor.py:843-846).
"""

from __future__ import annotations

import contextlib
import ctypes as C
import math
from typing import Iterator, Optional, Sequence, Tuple

import numpy as np

from . import _lib

_DTYPE_CODES = {
    np.dtype(np.float32): _lib.F32,
    np.dtype(np.float16): _lib.F16,
    np.dtype(np.int8): _lib.I8,
    np.dtype(np.int32): _lib.I32,
    np.dtype(np.int64): _lib.I64,
    np.dtype(np.uint8): _lib.U8,
    np.dtype(np.bool_): _lib.BOOL,
    np.dtype(np.float64): _lib.F64,
}

# bfloat16 has no NumPy dtype: it is carried as uint16 storage with this tag.
BF16 = np.dtype([("bf16", np.uint16)])


def dtype_code(dtype: np.dtype) -> int:
    dtype = np.dtype(dtype)
    if dtype == BF16:
        return _lib.BF16
    try:
        return _DTYPE_CODES[dtype]
    except KeyError:
        raise TypeError(f"dtype {dtype} has no libc3hip code") from None


_initialized = False


def init(device: int = 0) -> None:
    """Bind the calling process to `device` (one process per GPU)."""
    global _initialized
    if not _initialized:
        _lib.check(_lib.lib().c3h_init(device), "c3h_init")
        _initialized = True


def device_count() -> int:
    n = C.c_int(0)
    rc = _lib.lib().c3h_device_count(C.byref(n))
    return n.value if rc == 0 else 0


def device_props(device: int = 0) -> _lib.Props:
    props = _lib.Props()
    _lib.check(_lib.lib().c3h_device_props(device, C.byref(props)), "c3h_device_props")
    return props


def synchronize() -> None:
    _lib.check(_lib.lib().c3h_device_synchronize(), "c3h_device_synchronize")


class Buffer:
    """One hipMalloc allocation (the plan slab, or a standalone array)."""

    __slots__ = ("ptr", "nbytes", "__weakref__")

    def __init__(self, nbytes: int) -> None:
        init()
        ptr = C.c_void_p()
        _lib.check(_lib.lib().c3h_malloc(C.byref(ptr), max(int(nbytes), 1)), "c3h_malloc")
        self.ptr = int(ptr.value or 0)
        self.nbytes = int(nbytes)

    def __del__(self) -> None:
        if getattr(self, "ptr", 0) and _lib._LIB is not None:
            _lib._LIB.c3h_free(self.ptr)
            self.ptr = 0


class DeviceArray:
    """A C-contiguous device tensor: pointer + shape + dtype (+ owner)."""

    __slots__ = ("ptr", "shape", "dtype", "owner")

    def __init__(self, ptr: int, shape: Sequence[int], dtype, owner=None) -> None:
        self.ptr = int(ptr)
        self.shape = tuple(int(d) for d in shape)
        self.dtype = np.dtype(dtype)
        self.owner = owner

    # -- construction ---------------------------------------------------
    @classmethod
    def empty(cls, shape: Sequence[int], dtype=np.float32) -> "DeviceArray":
        shape = tuple(int(d) for d in shape)
        nbytes = math.prod(shape) * np.dtype(dtype).itemsize
        buf = Buffer(nbytes)
        return cls(buf.ptr, shape, dtype, buf)

    @classmethod
    def from_host(cls, host: np.ndarray, dtype=None, stream: Optional[int] = None) -> "DeviceArray":
        host = np.ascontiguousarray(host if dtype is None else host.astype(dtype))
        out = cls.empty(host.shape, host.dtype)
        out.copy_from_host(host, stream)
        return out

    # -- metadata ---------------------------------------------------------
    @property
    def ndim(self) -> int:
        return len(self.shape)

    @property
    def size(self) -> int:
        return math.prod(self.shape)

    @property
    def itemsize(self) -> int:
        return self.dtype.itemsize

    @property
    def nbytes(self) -> int:
        return self.size * self.itemsize

    @property
    def code(self) -> int:
        return dtype_code(self.dtype)

    def __repr__(self) -> str:
        return f"DeviceArray(shape={self.shape}, dtype={self.dtype}, ptr=0x{self.ptr:x})"

    # -- views ------------------------------------------------------------
    def reshape(self, *shape) -> "DeviceArray":
        if len(shape) == 1 and isinstance(shape[0], (tuple, list)):
            shape = tuple(shape[0])
        shape = list(int(d) for d in shape)
        if shape.count(-1) > 1:
            raise ValueError("can only specify one unknown dimension")
        if -1 in shape:
            known = math.prod(d for d in shape if d != -1)
            if known == 0 or self.size % known:
                raise ValueError(f"cannot reshape array of size {self.size} into {tuple(shape)}")
            shape[shape.index(-1)] = self.size // known
        if math.prod(shape) != self.size:
            raise ValueError(f"cannot reshape array of size {self.size} into {tuple(shape)}")
        return DeviceArray(self.ptr, shape, self.dtype, self.owner)

    def ravel(self) -> "DeviceArray":
        return DeviceArray(self.ptr, (self.size,), self.dtype, self.owner)

    def view(self, dtype) -> "DeviceArray":
        dtype = np.dtype(dtype)
        total = self.nbytes
        if total % dtype.itemsize:
            raise ValueError("byte size is not a multiple of the new itemsize")
        return DeviceArray(self.ptr, (total // dtype.itemsize,), dtype, self.owner)

    def flat(self, start: int, stop: int) -> "DeviceArray":
        """1-D element range [start, stop) of the flattened array."""
        if not 0 <= start <= stop <= self.size:
            raise ValueError(f"flat range [{start}, {stop}) outside size {self.size}")
        return DeviceArray(self.ptr + start * self.itemsize, (stop - start,), self.dtype, self.owner)

    def byte_range(self, offset: int, nbytes: int) -> "DeviceArray":
        """uint8 view of bytes [offset, offset + nbytes)."""
        if offset < 0 or offset + nbytes > self.nbytes:
            raise ValueError("byte range outside the array")
        return DeviceArray(self.ptr + offset, (nbytes,), np.uint8, self.owner)

    def split_axis0(self, start: int, stop: int) -> "DeviceArray":
        """Rows [start, stop) along axis 0 (contiguous)."""
        row = math.prod(self.shape[1:]) if self.ndim > 1 else 1
        return DeviceArray(self.ptr + start * row * self.itemsize, (stop - start,) + self.shape[1:],
                           self.dtype, self.owner)

    # -- transfers --------------------------------------------------------
    def copy_from_host(self, host: np.ndarray, stream: Optional[int] = None) -> None:
        host = np.ascontiguousarray(host)
        if host.nbytes != self.nbytes:
            raise ValueError(f"H2D byte size mismatch: host={host.nbytes}, device={self.nbytes}")
        if stream is None:
            _lib.check(_lib.lib().c3h_memcpy_h2d(self.ptr, host.ctypes.data, host.nbytes), "h2d")
        else:
            _lib.check(_lib.lib().c3h_memcpy_h2d_async(self.ptr, host.ctypes.data, host.nbytes, stream), "h2d")

    def get(self) -> np.ndarray:
        """Synchronous copy to a new host array (device-wide sync first)."""
        synchronize()
        host = np.empty(self.shape, dtype=self.dtype)
        _lib.check(_lib.lib().c3h_memcpy_d2h(host.ctypes.data, self.ptr, self.nbytes), "d2h")
        return host

    def copy_from(self, other: "DeviceArray", stream: Optional[int] = None) -> None:
        if other.nbytes != self.nbytes:
            raise ValueError("D2D byte size mismatch")
        _lib.check(_lib.lib().c3h_memcpy_d2d_async(self.ptr, other.ptr, self.nbytes,
                                                  current_stream() if stream is None else stream), "d2d")


class PinnedArray:
    """Page-locked host memory (hipHostMalloc) viewed as a NumPy array.

    Async H2D/D2H copies from or into it do not stage through a bounce
    buffer, so they overlap with kernels and with host work."""

    __slots__ = ("ptr", "nbytes", "array", "__weakref__")

    def __init__(self, shape: Sequence[int], dtype=np.float32) -> None:
        init()
        shape = tuple(int(d) for d in shape)
        dtype = np.dtype(dtype)
        self.nbytes = math.prod(shape) * dtype.itemsize
        ptr = C.c_void_p()
        _lib.check(_lib.lib().c3h_host_alloc(C.byref(ptr), max(self.nbytes, 1)), "c3h_host_alloc")
        self.ptr = int(ptr.value or 0)
        raw = (C.c_uint8 * max(self.nbytes, 1)).from_address(self.ptr)
        self.array = np.frombuffer(raw, dtype=np.uint8, count=self.nbytes).view(dtype).reshape(shape)

    def __del__(self) -> None:
        if getattr(self, "ptr", 0) and _lib._LIB is not None:
            self.array = None
            _lib._LIB.c3h_host_free(self.ptr)
            self.ptr = 0


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    """Decode bfloat16 bit patterns (uint16 or BF16-tagged) to float32."""
    u = np.asarray(bits).view(np.uint16).astype(np.uint32) << 16
    return u.view(np.float32)


def f32_to_bf16(values: np.ndarray) -> np.ndarray:
    """Round float32 to bfloat16 bit patterns (round to nearest even)."""
    u = np.ascontiguousarray(values, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7F800000) == 0x7F800000
    nan &= (u & 0x007FFFFF) != 0
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r = np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), r)
    return r.view(BF16)


# ---------------------------------------------------------------- streams
class Stream:
    """A persistent non-blocking hipStream_t at the default priority."""

    __slots__ = ("handle",)

    def __init__(self) -> None:
        init()
        h = C.c_void_p()
        _lib.check(_lib.lib().c3h_stream_create(C.byref(h)), "c3h_stream_create")
        self.handle = int(h.value)

    def synchronize(self) -> None:
        _lib.check(_lib.lib().c3h_stream_synchronize(self.handle), "c3h_stream_synchronize")

    def wait_event(self, event: "Event") -> None:
        _lib.check(_lib.lib().c3h_stream_wait_event(self.handle, event.handle), "c3h_stream_wait_event")

    def __del__(self) -> None:
        if getattr(self, "handle", 0) and _lib._LIB is not None:
            _lib._LIB.c3h_stream_destroy(self.handle)
            self.handle = 0


class Event:
    __slots__ = ("handle",)

    def __init__(self, timing: bool = False) -> None:
        init()
        h = C.c_void_p()
        _lib.check(_lib.lib().c3h_event_create(C.byref(h), int(timing)), "c3h_event_create")
        self.handle = int(h.value)

    def record(self, stream: Optional[Stream] = None) -> None:
        _lib.check(_lib.lib().c3h_event_record(self.handle, stream.handle if stream else current_stream()),
                   "c3h_event_record")

    def synchronize(self) -> None:
        _lib.check(_lib.lib().c3h_event_synchronize(self.handle), "c3h_event_synchronize")

    def elapsed_ms(self, end: "Event") -> float:
        ms = C.c_float()
        _lib.check(_lib.lib().c3h_event_elapsed_ms(C.byref(ms), self.handle, end.handle), "elapsed")
        return float(ms.value)

    def __del__(self) -> None:
        if getattr(self, "handle", 0) and _lib._LIB is not None:
            _lib._LIB.c3h_event_destroy(self.handle)
            self.handle = 0


_CURRENT: list = [None]


def current_stream() -> Optional[int]:
    """Raw hipStream_t handle kernels launch on (None = null stream)."""
    s = _CURRENT[-1]
    return s.handle if isinstance(s, Stream) else s


@contextlib.contextmanager
def using_stream(stream: Optional[Stream]) -> Iterator[None]:
    _CURRENT.append(stream)
    try:
        yield
    finally:
        _CURRENT.pop()


def empty_like_shape(shape: Tuple[int, ...], dtype=np.float32) -> DeviceArray:
    return DeviceArray.empty(shape, dtype)
