"""ctypes binding to libtritonmetal.so (the gfx950 C ABI).  No logic here.

One-to-one bindings for the `tm_*` exports, with the reference's rule that the
documented failure sentinel (NULL / 0 / -1) becomes a RuntimeError carrying
`tm_last_error` (reference python/triton_metal/_core.py:65-132).  The library
is searched at TRITON_METAL_CORE_LIB, then next to this package
(../lib/libtritonmetal.so, where triton-metal_amd/build.py puts it).
"""

import ctypes
import os
import struct
from pathlib import Path

_LIBRARY = "libtritonmetal.so"

_SEARCH = [
    os.environ.get("TRITON_METAL_CORE_LIB"),
    str(Path(__file__).resolve().parent / _LIBRARY),
    str(Path(__file__).resolve().parents[1] / "lib" / _LIBRARY),
]


def _load() -> ctypes.CDLL:
    for path in _SEARCH:
        if path and os.path.exists(path):
            return ctypes.CDLL(path)
    raise OSError(
        f"{_LIBRARY} not found; run `python triton-metal_amd/build.py` (or "
        "`python -c 'import __graft_entry__ as g; g.build()'`) or set TRITON_METAL_CORE_LIB. "
        "Searched:\n  " + "\n  ".join(p for p in _SEARCH if p)
    )


_lib = _load()
#: Absolute path of the loaded library (tests check which .so is in use).
LIBRARY_PATH = _lib._name

_i64 = ctypes.c_int64
_i32 = ctypes.c_int32
_ptr = ctypes.c_void_p
_str = ctypes.c_char_p

_SIGNATURES = {
    # name: (restype, argtypes) — the reference's 23 exports
    "tm_version": (_ptr, []),
    "tm_last_error": (_ptr, []),
    "tm_free": (None, [_ptr]),
    "tm_is_active": (_i32, []),
    "tm_is_usable": (_i32, []),
    "tm_unusable_reason": (_ptr, []),
    "tm_device_name": (_ptr, []),
    "tm_emit_msl": (_ptr, [_str, _i32]),
    "tm_kernel_info": (_ptr, [_str, _i32]),
    "tm_compile_msl": (_i64, [_str]),
    "tm_load_metallib": (_i64, [_ptr, _i64]),
    "tm_release_library": (_i32, [_i64]),
    "tm_load_kernel": (_i64, [_i64, _str]),
    "tm_kernel_max_threads": (_i64, [_i64]),
    "tm_release_kernel": (_i32, [_i64]),
    "tm_alloc_buffer": (_i64, [_i64]),
    "tm_buffer_contents": (_ptr, [_i64]),
    "tm_buffer_length": (_i64, [_i64]),
    "tm_buffer_write": (_i32, [_i64, _i64, _ptr, _i64]),
    "tm_buffer_read": (_i32, [_i64, _i64, _ptr, _i64]),
    "tm_free_buffer": (_i32, [_i64]),
    "tm_launch": (
        _i32,
        [_i64, _i64, _i64, _i64, _i64, ctypes.POINTER(_i32), ctypes.POINTER(_i64), _i32],
    ),
    "tm_live_handle_count": (_i64, []),
    # extensions (no reference counterpart)
    "tm_launch_async": (
        _i32,
        [_i64, _i64, _i64, _i64, _i64, ctypes.POINTER(_i32), ctypes.POINTER(_i64), _i32],
    ),
    "tm_synchronize": (_i32, []),
    "tm_launch_timed": (
        _i32,
        [_i64, _i64, _i64, _i64, _i64, ctypes.POINTER(_i32), ctypes.POINTER(_i64), _i32,
         _i32, ctypes.POINTER(ctypes.c_float)],
    ),
    "tm_kernel_variant": (_ptr, [_i64]),
    "tm_launch_noalloc": (
        _i32,
        [_i64, _i64, _i64, _i64, _i64, ctypes.POINTER(_i32), ctypes.POINTER(_i64), _i32],
    ),
    "tm_buffer_unmap": (_i32, [_i64]),
}

#: The exports the reference's C ABI has (reference _core.py:70-100).
REFERENCE_EXPORTS = tuple(list(_SIGNATURES)[:23])

for _name, (_restype, _argtypes) in _SIGNATURES.items():
    _fn = getattr(_lib, _name)
    _fn.restype = _restype
    _fn.argtypes = _argtypes


def _take_string(ptr):
    if not ptr:
        return None
    try:
        return ctypes.cast(ptr, ctypes.c_char_p).value.decode()
    finally:
        _lib.tm_free(ptr)


def last_error() -> str:
    return _take_string(_lib.tm_last_error())


def _check(value, sentinel):
    if value == sentinel:
        raise RuntimeError(last_error())
    return value


def _check_string(ptr):
    text = _take_string(ptr)
    if text is None:
        raise RuntimeError(last_error())
    return text


# --- Device -----------------------------------------------------------------


def version() -> str:
    return _take_string(_lib.tm_version())


def is_active() -> bool:
    return bool(_lib.tm_is_active())


def is_usable() -> bool:
    """Whether the device ran the library's MFMA probe kernel correctly."""
    return bool(_lib.tm_is_usable())


def unusable_reason():
    """Why `is_usable()` is False, or None when the device is usable."""
    return _take_string(_lib.tm_unusable_reason())


def device_name():
    return _take_string(_lib.tm_device_name())


# --- Libraries --------------------------------------------------------------


def emit_msl(module: str, num_simdgroups: int = 4) -> str:
    return _check_string(_lib.tm_emit_msl(module.encode(), num_simdgroups))


def kernel_info(module: str, num_simdgroups: int = 4) -> str:
    """Launch metadata as a JSON document, computed in the native library."""
    return _check_string(_lib.tm_kernel_info(module.encode(), num_simdgroups))


def compile_msl(source: str) -> int:
    """A built-in spec ("builtin element=bf16 head_dim=128 causal=1") or HIP
    source compiled for gfx950 by hiprtc -> library handle."""
    return _check(_lib.tm_compile_msl(source.encode()), 0)


def load_metallib(image: bytes) -> int:
    """A gfx950 code object image -> library handle."""
    return _check(_lib.tm_load_metallib(image, len(image)), 0)


def release_library(handle: int) -> None:
    _check(_lib.tm_release_library(handle), -1)


# --- Runtime ----------------------------------------------------------------


def load_kernel(library: int, name: str) -> int:
    return _check(_lib.tm_load_kernel(library, name.encode()), 0)


def kernel_max_threads(kernel: int) -> int:
    return _check(_lib.tm_kernel_max_threads(kernel), -1)


def release_kernel(handle: int) -> None:
    _check(_lib.tm_release_kernel(handle), -1)


def alloc_buffer(nbytes: int) -> int:
    return _check(_lib.tm_alloc_buffer(nbytes), 0)


def buffer_contents(handle: int) -> int:
    """Host address of the buffer's contents: its pinned host mirror, made on
    the first call.  While the mirror exists every launch that binds the
    buffer copies it to HBM and back and waits; buffer_unmap drops it."""
    return _check(_lib.tm_buffer_contents(handle), None)


def buffer_unmap(handle: int) -> None:
    """Drop the host mirror (host writes through it reach HBM first); the
    address buffer_contents gave is invalid afterwards."""
    _check(_lib.tm_buffer_unmap(handle), -1)


def buffer_length(handle: int) -> int:
    return _check(_lib.tm_buffer_length(handle), -1)


def buffer_write(handle: int, offset: int, address: int, nbytes: int) -> None:
    _check(_lib.tm_buffer_write(handle, offset, ctypes.c_void_p(address), nbytes), -1)


def buffer_read(handle: int, offset: int, address: int, nbytes: int) -> None:
    _check(_lib.tm_buffer_read(handle, offset, ctypes.c_void_p(address), nbytes), -1)


def free_buffer(handle: int) -> None:
    _check(_lib.tm_free_buffer(handle), -1)


#: `tm_launch` argument kinds (reference _core.py:233-240).
ARG_BUFFER = 0
ARG_I32 = 1
ARG_F32 = 2
ARG_I64 = 3


def float_bits(value: float) -> int:
    """`f32` scalars travel in the low 32 bits of a `values[i]` slot."""
    return struct.unpack("<I", struct.pack("<f", value))[0]


def _arrays(kinds, values):
    count = len(kinds)
    return (_i32 * count)(*kinds), (_i64 * count)(*values), count


def launch(kernel, grid, threads_per_threadgroup, kinds, values) -> None:
    """Dispatch `kernel` over `grid` (3 workgroup counts) and wait."""
    kind_array, value_array, count = _arrays(kinds, values)
    _check(
        _lib.tm_launch(kernel, grid[0], grid[1], grid[2], threads_per_threadgroup, kind_array,
                       value_array, count),
        -1,
    )


def launch_async(kernel, grid, threads_per_threadgroup, kinds, values) -> None:
    """Queue a dispatch on the library stream without waiting."""
    kind_array, value_array, count = _arrays(kinds, values)
    _check(
        _lib.tm_launch_async(kernel, grid[0], grid[1], grid[2], threads_per_threadgroup,
                             kind_array, value_array, count),
        -1,
    )


def launch_noalloc(kernel, grid, threads_per_threadgroup, kinds, values) -> None:
    """launch() that allocates no device memory: a work buffer comes from the
    library's static device scratch (64 MiB); larger requests raise."""
    kind_array, value_array, count = _arrays(kinds, values)
    _check(
        _lib.tm_launch_noalloc(kernel, grid[0], grid[1], grid[2], threads_per_threadgroup,
                               kind_array, value_array, count),
        -1,
    )


def synchronize() -> None:
    _check(_lib.tm_synchronize(), -1)


def launch_timed(kernel, grid, threads_per_threadgroup, kinds, values, repeats) -> float:
    """Milliseconds for `repeats` back-to-back dispatches, between HIP events."""
    kind_array, value_array, count = _arrays(kinds, values)
    elapsed = ctypes.c_float(0.0)
    _check(
        _lib.tm_launch_timed(kernel, grid[0], grid[1], grid[2], threads_per_threadgroup,
                             kind_array, value_array, count, repeats, ctypes.byref(elapsed)),
        -1,
    )
    return float(elapsed.value)


def kernel_variant(kernel: int) -> str:
    """Device function the kernel's last dispatch ran (the rocprof name)."""
    return _check_string(_lib.tm_kernel_variant(kernel))


def live_handle_count() -> int:
    return _lib.tm_live_handle_count()
