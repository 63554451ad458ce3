"""A `.data_ptr()` object over a library-owned HBM buffer.

Counterpart of the reference's MetalBuffer (python/triton_metal/buffer.py:35-114):
same constructor arguments, dtype names, `data_ptr`, `copy_from`/`copy_to`,
`numpy`, `from_numpy`, `tolist`, `free`.  On MI355X the buffer lives in device
memory.  `data_ptr()` is `tm_buffer_contents`: a host address that behaves like
the reference's unified memory (the library keeps a pinned host mirror of a
buffer once it has been asked for one, and copies it around each launch that
binds the buffer, and waits), so code that reads or writes through it works
unchanged; `unmap()` drops the mirror.
The copies `copy_from`/`copy_to`/`numpy`/`write` are `tm_buffer_write`/
`tm_buffer_read` and never create a mirror.

numpy has no bfloat16: bf16 buffers exchange raw 16-bit words (np.uint16), and
`bf16_bits` / `bf16_values` convert (round-to-nearest-even).
"""

import numpy as np

from . import _core

#: Element sizes for the dtype names the reference accepts.
_ITEMSIZE = {
    "float16": 2, "bfloat16": 2, "float32": 4, "int8": 1, "int16": 2, "int32": 4,
    "int64": 8, "uint8": 1, "uint16": 2, "uint32": 4, "uint64": 8,
}

#: The numpy dtype a buffer of each element type reads back as.
_NUMPY = {name: (np.uint16 if name == "bfloat16" else np.dtype(name)) for name in _ITEMSIZE}


def bf16_bits(values) -> np.ndarray:
    """float32 -> bfloat16 bit patterns (uint16), round to nearest even; NaN kept."""
    x = np.ascontiguousarray(values, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(x)
    if nan.any():
        rounded[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return rounded


def bf16_values(bits) -> np.ndarray:
    """bfloat16 bit patterns (uint16) -> float32 (exact)."""
    b = np.ascontiguousarray(bits, dtype=np.uint16)
    return (b.astype(np.uint32) << 16).view(np.float32)


def round_to(values, dtype: str) -> np.ndarray:
    """float32 values rounded to `dtype` and back: what a kernel of that element
    type sees."""
    x = np.asarray(values, dtype=np.float32)
    if dtype in ("bfloat16", "bf16"):
        return bf16_values(bf16_bits(x)).reshape(x.shape)
    if dtype in ("float16", "f16"):
        return x.astype(np.float16).astype(np.float32)
    return x.copy()


def _element_name(dtype) -> str:
    """'float32', np.float32, torch.bfloat16, 'bfloat16' ... -> the bare element
    name the size table uses."""
    name = str(dtype).rsplit(".", 1)[-1]
    if name not in _ITEMSIZE:
        raise TypeError(f"unsupported dtype {dtype!r}; expected one of {sorted(_ITEMSIZE)}")
    return name


class DeviceBuffer:
    """HBM the GPU reads and writes; the host moves bytes in and out."""

    def __init__(self, shape, dtype="float32"):
        self.shape = (shape,) if isinstance(shape, int) else tuple(int(d) for d in shape)
        self.dtype = _element_name(dtype)
        self.itemsize = _ITEMSIZE[self.dtype]
        self.numel = int(np.prod(self.shape, dtype=np.int64))
        self.nbytes = self.numel * self.itemsize
        self.tm_handle = _core.alloc_buffer(self.nbytes)

    def data_ptr(self):
        """Host address of the contents (the buffer's host mirror).

        The first call makes a pinned host copy of the whole buffer.  From
        then on every launch that binds the buffer copies it host -> HBM
        before the dispatch and back after it, and waits for it (launch_async
        included): a caller that only wants a pointer pays two full-buffer
        copies and a synchronisation per launch.  `unmap()` ends that."""
        return _core.buffer_contents(self.tm_handle)

    def unmap(self):
        """Drop the host mirror made by `data_ptr()` (writes through it reach
        HBM first); the address it returned is invalid afterwards."""
        _core.buffer_unmap(self.tm_handle)

    def __len__(self):
        return self.shape[0] if self.shape else 0

    def copy_from(self, address, nbytes=None):
        """Copy `nbytes` from a host address (e.g. `numpy_array.ctypes.data`)."""
        _core.buffer_write(self.tm_handle, 0, address, self.nbytes if nbytes is None else nbytes)

    def copy_to(self, address, nbytes=None):
        _core.buffer_read(self.tm_handle, 0, address, self.nbytes if nbytes is None else nbytes)

    def numpy(self) -> np.ndarray:
        out = np.empty(self.shape, dtype=_NUMPY[self.dtype])
        self.copy_to(out.ctypes.data, out.nbytes)
        return out

    def float32(self) -> np.ndarray:
        """Contents widened to float32 (bf16 words decoded)."""
        out = self.numpy()
        if self.dtype == "bfloat16":
            return bf16_values(out).reshape(self.shape)
        return out.astype(np.float32)

    def tolist(self):
        return self.numpy().reshape(-1).tolist()

    def write(self, array) -> "DeviceBuffer":
        """Upload a host array of exactly this buffer's size (float input is
        converted to the element type; bf16 with round-to-nearest-even)."""
        array = np.asarray(array)
        if self.dtype == "bfloat16" and array.dtype != np.uint16:
            array = bf16_bits(array)
        else:
            array = np.ascontiguousarray(array, dtype=_NUMPY[self.dtype])
        if array.nbytes != self.nbytes:
            raise ValueError(f"array of {array.nbytes} bytes for a {self.nbytes}-byte buffer")
        array = np.ascontiguousarray(array)
        self.copy_from(array.ctypes.data, array.nbytes)
        return self

    @classmethod
    def from_numpy(cls, array, dtype=None):
        array = np.ascontiguousarray(array)
        dtype = dtype or str(array.dtype)
        buf = cls(array.shape, dtype)
        buf.write(array)
        return buf

    def free(self):
        if self.tm_handle:
            _core.free_buffer(self.tm_handle)
            self.tm_handle = 0

    def __repr__(self):
        return f"DeviceBuffer(shape={self.shape}, dtype='{self.dtype}', handle={self.tm_handle})"


#: The reference's name for the same object.
MetalBuffer = DeviceBuffer
