"""Device tensors.

``DeviceTensor`` keeps the reference's API (``SpikeTensor``,
spike/src/spike/spike_tensor.py:9-83, and ``DeviceTensor``,
nkipy/src/nkipy/runtime/device_tensor.py:48-103): ``from_numpy`` /
``numpy`` / ``write_from_numpy`` and the torch counterparts, a shape, a
dtype and a name.  Its ``tensor_ref`` is a :class:`DeviceBuffer`, the
analogue of ``NrtTensor`` (spike/src/tensor.cpp:9-115): an owned HIP
allocation that refuses use after free and frees itself when collected.

bf16 / fp8 arrays travel as their bit patterns; with no ``ml_dtypes`` the
NumPy side uses the stand-in dtypes of :mod:`nkipy_amd.core.dtypes`.
"""

from __future__ import annotations

import ctypes
import math
from typing import Tuple

import numpy as np

from nkipy_amd.core import dtypes as dt
from nkipy_amd.runtime.hip import SpikeError, get_runtime


class DeviceBuffer:
    """An owned device allocation (``NrtTensor`` analogue)."""

    __slots__ = ("rt", "ptr", "size", "name", "core_id", "_owner", "__weakref__")

    def __init__(self, size: int, name: str = None, core_id: int = 0):
        self.rt = get_runtime()
        self.size = int(size)
        self.ptr = self.rt.malloc(max(self.size, 1))
        self.name = name
        self.core_id = self.rt.device if core_id is None else core_id
        self._owner = True

    @property
    def is_freed(self) -> bool:
        return self.ptr is None or self.rt.is_closed

    @property
    def va(self) -> int:
        return self.ptr

    def _live(self):
        if self.is_freed:
            raise SpikeError(
                "Unable to access a freed tensor. Please check the lifetime of the tensor."
            )

    def write(self, host_addr: int, nbytes: int, offset: int = 0):
        self._live()
        if offset + nbytes > self.size:
            raise SpikeError(
                "The write operation exceeds the tensor bound. "
                f"Tensor size: {self.size} bytes; Input size: {nbytes} bytes; Offset: {offset} bytes."
            )
        self.rt.h2d(self.ptr + offset, host_addr, nbytes)

    def read(self, host_addr: int, nbytes: int, offset: int = 0):
        self._live()
        if offset + nbytes > self.size:
            raise SpikeError(
                "The read operation exceeds the tensor bound. "
                f"Tensor size: {self.size} bytes; Read size: {nbytes} bytes; Offset: {offset} bytes."
            )
        self.rt.d2h(host_addr, self.ptr + offset, nbytes)

    def free(self):
        if self.ptr is not None and self._owner and not self.rt.is_closed:
            self.rt.free(self.ptr)
        self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

    def __repr__(self):
        return f"DeviceBuffer(ptr={self.ptr and hex(self.ptr)}, name='{self.name}', size={self.size})"


def _host_bytes(array: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(dt.numpy_storage(np.ascontiguousarray(array)))


class DeviceTensor:
    """A tensor in device memory."""

    def __init__(self, tensor_ref: DeviceBuffer, shape: Tuple[int, ...], dtype, name: str = None):
        shape = (shape,) if isinstance(shape, int) else tuple(int(s) for s in shape)
        self.tensor_ref = tensor_ref
        self.shape = shape
        self.dtype = dt.canonical(dtype)
        self.name = name
        self._size = math.prod(shape) if shape else 1

    # -- properties ------------------------------------------------------
    @property
    def ptr(self) -> int:
        self.tensor_ref._live()
        return self.tensor_ref.ptr

    @property
    def size(self) -> int:
        return self._size

    @property
    def nbytes(self) -> int:
        return self.size * self.dtype.itemsize

    @property
    def ndim(self) -> int:
        return len(self.shape)

    # -- construction ----------------------------------------------------
    @classmethod
    def empty(cls, shape, dtype, name: str = None, core_id: int = 0) -> "DeviceTensor":
        shape = (shape,) if isinstance(shape, int) else tuple(shape)
        d = dt.canonical(dtype)
        n = int(np.prod(shape)) * d.itemsize if shape else d.itemsize
        return cls(DeviceBuffer(n, name=name, core_id=core_id), shape, d, name)

    @classmethod
    def from_numpy(cls, array: np.ndarray, name: str = None, core_id: int = 0) -> "DeviceTensor":
        array = np.ascontiguousarray(array)
        t = cls.empty(array.shape, array.dtype, name=name, core_id=core_id)
        if array.nbytes:
            raw = _host_bytes(array)
            t.tensor_ref.write(raw.ctypes.data, raw.nbytes)
        return t

    @classmethod
    def from_torch(cls, tensor, name: str = None, core_id: int = 0) -> "DeviceTensor":
        import torch

        t = tensor.detach().to("cpu").contiguous()
        d = dt.from_torch_dtype(t.dtype)
        out = cls.empty(tuple(t.shape), d, name=name, core_id=core_id)
        if t.numel():
            out.tensor_ref.write(t.data_ptr(), t.numel() * t.element_size())
        return out

    # -- I/O ---------------------------------------------------------------
    def numpy(self) -> np.ndarray:
        out = np.empty(self.shape, dtype=self.dtype)
        if out.nbytes:
            raw = dt.numpy_storage(out)
            self.tensor_ref.read(raw.ctypes.data, raw.nbytes)
        return out

    def write_from_numpy(self, array: np.ndarray):
        array = np.ascontiguousarray(array)
        if array.nbytes != self.nbytes:
            raise ValueError(
                f"Size mismatch: source {array.nbytes} bytes, target {self.nbytes} bytes"
            )
        raw = _host_bytes(array)
        self.tensor_ref.write(raw.ctypes.data, raw.nbytes)

    def torch(self):
        import torch

        td = dt.torch_dtype(self.dtype)
        out = torch.empty(self.shape, dtype=td)
        if out.numel():
            self.tensor_ref.read(out.data_ptr(), self.nbytes)
        return out

    def write_from_torch(self, tensor):
        t = tensor.detach().to("cpu").contiguous()
        nbytes = t.numel() * t.element_size()
        if nbytes != self.nbytes:
            raise ValueError(f"Size mismatch: source {nbytes} bytes, target {self.nbytes} bytes")
        self.tensor_ref.write(t.data_ptr(), nbytes)

    def free(self):
        self.tensor_ref.free()

    def __repr__(self):
        return f"{type(self).__name__}(shape={self.shape}, dtype={dt.name(self.dtype)}, name={self.name})"
