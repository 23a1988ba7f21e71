"""A minimal device tensor handle over the library's own memory.

``DeviceTensor`` is a strided view (sizes, strides in elements, dtype code,
device index) of memory that the library's caching allocator owns; views
share the block of the tensor they come from.  It exists so the operator
mirror in ``ops`` can be driven from Python the way TensorPlay would drive
the registered kernels -- it is not a tensor library.

bfloat16 has no numpy dtype: on the host it travels as ``np.uint16`` bit
patterns.
"""

from __future__ import annotations

import ctypes as C

import numpy as np

from . import _abi
from . import _library

NP_TO_CODE = {
    np.dtype(np.float32): _abi.FLOAT32,
    np.dtype(np.float16): _abi.FLOAT16,
    np.dtype(np.float64): _abi.FLOAT64,
    np.dtype(np.int8): _abi.INT8,
    np.dtype(np.int16): _abi.INT16,
    np.dtype(np.int32): _abi.INT32,
    np.dtype(np.int64): _abi.INT64,
    np.dtype(np.uint8): _abi.UINT8,
    np.dtype(np.bool_): _abi.BOOL,
}
CODE_TO_NP = {v: k for k, v in NP_TO_CODE.items()}
CODE_TO_NP[_abi.BFLOAT16] = np.dtype(np.uint16)
NAMES = {
    _abi.FLOAT32: "float32", _abi.FLOAT16: "float16", _abi.BFLOAT16: "bfloat16",
    _abi.FLOAT64: "float64", _abi.INT8: "int8", _abi.INT16: "int16", _abi.INT32: "int32",
    _abi.INT64: "int64", _abi.UINT8: "uint8", _abi.BOOL: "bool",
}
BY_NAME = {v: k for k, v in NAMES.items()}


class DeclinedError(RuntimeError):
    """The device path declined (TP_AMD_DECLINED): TensorPlay would run the
    operator on the host; this mirror has no host path and raises."""


class DeviceError(RuntimeError):
    """A failure reported by the library (TP_AMD_ERROR)."""


def check(status: int) -> None:
    if status == _abi.OK:
        return
    message = _library().tp_mlu_last_error().decode()
    if status == _abi.DECLINED:
        raise DeclinedError(message)
    raise DeviceError(message)


def dtype_code(dtype) -> int:
    if isinstance(dtype, int):
        return dtype
    if isinstance(dtype, str):
        return BY_NAME[dtype]
    return NP_TO_CODE[np.dtype(dtype)]


class _Block:
    """Owns one allocator block; returns it to the pool when collected."""

    __slots__ = ("ctx", "lib")

    def __init__(self, ctx: int | None):
        self.ctx = ctx
        self.lib = _library()

    def __del__(self):
        if self.ctx:
            try:
                self.lib.tp_amd_free(self.ctx)
            except Exception:  # interpreter teardown
                pass
            self.ctx = None


def contiguous_strides(shape) -> tuple[int, ...]:
    strides, s = [], 1
    for d in reversed(shape):
        strides.append(s)
        s *= max(d, 1)
    return tuple(reversed(strides))


class DeviceTensor:
    """A strided view of library-owned device memory."""

    def __init__(self, ref: _abi.Tensor, owner=None):
        self._ref = ref
        if owner is None and ref.ctx:
            owner = _Block(ref.ctx)
        self._owner = owner
        self._ref.ctx = None  # ownership lives in _owner, never in views

    # -- construction ---------------------------------------------------
    @staticmethod
    def from_result(ref: _abi.Tensor, base: "DeviceTensor | None" = None) -> "DeviceTensor":
        """Wrap a result an entry point wrote; a NULL ctx means a view of ``base``."""
        if ref.ctx:
            return DeviceTensor(ref)
        return DeviceTensor(ref, base._owner if base is not None else None)

    @staticmethod
    def empty(shape, dtype="float32", device: int = 0) -> "DeviceTensor":
        shape = tuple(int(s) for s in shape)
        sizes = (C.c_int64 * max(len(shape), 1))(*shape)
        out = _abi.Tensor()
        check(_library().tp_amd_empty(sizes, len(shape), dtype_code(dtype), device, 0,
                                      C.byref(out)))
        return DeviceTensor(out)

    @staticmethod
    def from_numpy(array: np.ndarray, device: int = 0, dtype=None) -> "DeviceTensor":
        """Copy a host array to the device.  ``dtype="bfloat16"`` reads
        ``array`` as uint16 bit patterns."""
        array = np.asarray(array, order="C")
        code = dtype_code(dtype) if dtype is not None else NP_TO_CODE[array.dtype]
        if code == _abi.BFLOAT16:
            array = array.view(np.uint16) if array.dtype.itemsize == 2 else array
            assert array.dtype == np.uint16, "bfloat16 data travels as uint16 bit patterns"
        out = DeviceTensor.empty(array.shape, code, device)
        host = host_view(array, code)
        check(_library().tp_amd_copy_(C.byref(out._ref), C.byref(host), 0))
        return out

    # -- properties -----------------------------------------------------
    @property
    def ref(self) -> _abi.Tensor:
        return self._ref

    @property
    def shape(self) -> tuple[int, ...]:
        return tuple(self._ref.sizes[i] for i in range(self._ref.ndim))

    @property
    def strides(self) -> tuple[int, ...]:
        return tuple(self._ref.strides[i] for i in range(self._ref.ndim))

    @property
    def dtype(self) -> int:
        return self._ref.dtype

    @property
    def dtype_name(self) -> str:
        return NAMES[self._ref.dtype]

    @property
    def device(self) -> int:
        return self._ref.device

    @property
    def ndim(self) -> int:
        return self._ref.ndim

    @property
    def data_ptr(self) -> int:
        return self._ref.data or 0

    def numel(self) -> int:
        n = 1
        for s in self.shape:
            n *= s
        return n

    def is_contiguous(self) -> bool:
        expected = 1
        for size, stride in zip(reversed(self.shape), reversed(self.strides)):
            if size == 1:
                continue
            if stride != expected:
                return False
            expected *= size
        return True

    def __repr__(self) -> str:
        return (f"DeviceTensor(shape={self.shape}, strides={self.strides}, "
                f"dtype={self.dtype_name}, device={self.device})")

    # -- host round trip ------------------------------------------------
    def numpy(self) -> np.ndarray:
        """Copy to a new host array (bfloat16 as uint16 bit patterns)."""
        out = np.empty(self.shape, dtype=CODE_TO_NP[self.dtype])
        host = host_view(out, self.dtype)
        check(_library().tp_amd_copy_(C.byref(host), C.byref(self._ref), 0))
        return out

    # -- views ----------------------------------------------------------
    def _view(self, shape, strides, offset_elems: int = 0) -> "DeviceTensor":
        ref = _abi.Tensor()
        C.memmove(C.byref(ref), C.byref(self._ref), C.sizeof(_abi.Tensor))
        ref.ndim = len(shape)
        for i in range(_abi.MAX_DIMS):
            ref.sizes[i] = shape[i] if i < len(shape) else 0
            ref.strides[i] = strides[i] if i < len(shape) else 0
        esize = _library().tp_amd_element_size(self.dtype)
        ref.data = (self._ref.data or 0) + offset_elems * esize or None
        ref.ctx = None
        return DeviceTensor(ref, self._owner)

    def transpose(self, a: int, b: int) -> "DeviceTensor":
        shape, strides = list(self.shape), list(self.strides)
        shape[a], shape[b] = shape[b], shape[a]
        strides[a], strides[b] = strides[b], strides[a]
        return self._view(shape, strides)

    def t(self) -> "DeviceTensor":
        assert self.ndim == 2
        return self.transpose(0, 1)

    def permute(self, *order) -> "DeviceTensor":
        return self._view([self.shape[i] for i in order], [self.strides[i] for i in order])

    def expand(self, *shape) -> "DeviceTensor":
        shape = list(shape[0]) if len(shape) == 1 and isinstance(shape[0], (tuple, list)) else list(shape)
        pad = len(shape) - self.ndim
        strides = []
        for i, s in enumerate(shape):
            j = i - pad
            if j < 0:
                strides.append(0)
            elif self.shape[j] == s:
                strides.append(self.strides[j])
            else:
                assert self.shape[j] == 1, f"cannot expand {self.shape} to {shape}"
                strides.append(0)
        return self._view(shape, strides)

    def view(self, *shape) -> "DeviceTensor":
        shape = list(shape[0]) if len(shape) == 1 and isinstance(shape[0], (tuple, list)) else list(shape)
        if -1 in shape:
            known = 1
            for s in shape:
                if s != -1:
                    known *= s
            shape[shape.index(-1)] = self.numel() // known
        assert self.is_contiguous(), "view() needs a contiguous tensor"
        return self._view(shape, contiguous_strides(shape))

    reshape = view

    def unsqueeze(self, dim: int) -> "DeviceTensor":
        shape, strides = list(self.shape), list(self.strides)
        dim = dim if dim >= 0 else dim + self.ndim + 1
        inner = strides[dim] * shape[dim] if dim < self.ndim else 1
        shape.insert(dim, 1)
        strides.insert(dim, inner)
        return self._view(shape, strides)

    def __getitem__(self, index) -> "DeviceTensor":
        if not isinstance(index, tuple):
            index = (index,)
        shape, strides = [], []
        offset = 0
        dim = 0
        for item in index:
            if isinstance(item, slice):
                start, stop, step = item.indices(self.shape[dim])
                n = max(0, (stop - start + (step - (1 if step > 0 else -1))) // step)
                offset += start * self.strides[dim]
                shape.append(n)
                strides.append(self.strides[dim] * step)
            else:
                i = item if item >= 0 else item + self.shape[dim]
                offset += i * self.strides[dim]
            dim += 1
        shape += list(self.shape[dim:])
        strides += list(self.strides[dim:])
        return self._view(shape, strides, offset)


def host_view(array: np.ndarray, code: int | None = None) -> _abi.Tensor:
    """A tp_amd_tensor describing a host numpy array (device -1).  The array
    must outlive the call that uses the view."""
    ref = _abi.Tensor()
    ref.data = array.ctypes.data if array.size else None
    ref.ctx = None
    ref.ndim = array.ndim
    item = array.itemsize
    for i in range(array.ndim):
        ref.sizes[i] = array.shape[i]
        ref.strides[i] = array.strides[i] // item
    ref.dtype = code if code is not None else NP_TO_CODE[array.dtype]
    ref.device = -1
    return ref
