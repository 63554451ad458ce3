"""The tm_* C ABI end to end on the device (reference CABITests.swift:93-318,
python/tests/test_plugin_shape.py:183-300).  The reference compiles its test
kernels from ttir; here they are HIP source compiled for gfx950 by the
library's hiprtc path, or a code object built by hipcc."""

import array
import ctypes
import os
import shutil
import subprocess

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

VECTOR_ADD = r"""
extern "C" __global__ void add_kernel(const float *a, const float *b, float *out, int n) {
  const int start = blockIdx.x * 1024, end = min(n, start + 1024);
  for (int i = start + threadIdx.x; i < end; i += blockDim.x) out[i] = a[i] + b[i];
}
"""

SCALE_BIAS = r"""
extern "C" __global__ void scale_bias_kernel(const float *x, float *y, float scale, float bias,
                                             int n) {
  for (int i = threadIdx.x; i < n; i += blockDim.x) y[i] = x[i] * scale + bias;
}
"""

I64_KERNEL = r"""
extern "C" __global__ void i64_kernel(long long *out, long long base, int n) {
  const int i = blockIdx.x * 8 + threadIdx.x;
  if (threadIdx.x < 8 && i < n) out[i] = base + i;
}
"""

COPY = r"""
extern "C" __global__ void copy_kernel(const float *x, float *y) { y[threadIdx.x] = x[threadIdx.x]; }
"""


def _upload(core, values):
    data = array.array("f", values)
    handle = core.alloc_buffer(4 * len(data))
    core.buffer_write(handle, 0, data.buffer_info()[0], 4 * len(data))
    return handle


def _download(core, handle, n, code="f"):
    out = array.array(code, [0] * n)
    core.buffer_read(handle, 0, out.buffer_info()[0], out.itemsize * n)
    return out


def test_probe_passed(core, device):
    assert core.is_usable()
    assert core.unusable_reason() is None
    assert "gfx950" in device


def test_vector_add_round_trips_through_the_c_abi(core, device):
    n = 5000
    a = [i * 0.5 for i in range(n)]
    b = [float(i % 13) for i in range(n)]
    live = core.live_handle_count()
    library = core.compile_msl(VECTOR_ADD)
    kernel = core.load_kernel(library, "add_kernel")
    assert core.kernel_max_threads(kernel) >= 128
    ba, bb = _upload(core, a), _upload(core, b)
    out = core.alloc_buffer(4 * n)
    assert core.buffer_length(out) == 4 * n
    core.launch(kernel, ((n + 1023) // 1024, 1, 1), 128,
                [core.ARG_BUFFER] * 3 + [core.ARG_I32], [ba, bb, out, n])
    assert list(_download(core, out, n)) == [x + y for x, y in zip(a, b)]
    # Reading past the end is refused rather than corrupting the host.
    host = (ctypes.c_float * n)()
    assert core._lib.tm_buffer_read(out, 4, host, 4 * n) == -1
    assert "exceeds the" in core.last_error()
    for h in (ba, bb, out):
        core.free_buffer(h)
    core.release_kernel(kernel)
    core.release_library(library)
    assert core.live_handle_count() == live


def test_float_scalar_launch_arguments(core, device):
    n = 64
    library = core.compile_msl(SCALE_BIAS)
    kernel = core.load_kernel(library, "scale_bias_kernel")
    bin_, bout = _upload(core, [float(i) for i in range(n)]), core.alloc_buffer(4 * n)
    try:
        core.launch(kernel, (1, 1, 1), 128,
                    [core.ARG_BUFFER, core.ARG_BUFFER, core.ARG_F32, core.ARG_F32, core.ARG_I32],
                    [bin_, bout, core.float_bits(2.5), core.float_bits(-1.75), n])
        assert list(_download(core, bout, n)) == [i * 2.5 - 1.75 for i in range(n)]
        assert core._lib.tm_launch(kernel, 1, 1, 1, 128, None, None, 5) == -1
        assert "NULL argument arrays" in core.last_error()
    finally:
        core.free_buffer(bin_)
        core.free_buffer(bout)
        core.release_kernel(kernel)
        core.release_library(library)


def test_i64_scalar_arguments_survive_the_launch_abi(core, device):
    base, n = 1 << 40, 24
    library = core.compile_msl(I64_KERNEL)
    kernel = core.load_kernel(library, "i64_kernel")
    out = core.alloc_buffer(8 * n)
    try:
        core.launch(kernel, (3, 1, 1), 64, [core.ARG_BUFFER, core.ARG_I64, core.ARG_I32],
                    [out, base, n])
        assert list(_download(core, out, n, "q")) == [base + i for i in range(n)]
    finally:
        core.free_buffer(out)
        core.release_kernel(kernel)
        core.release_library(library)


def test_compile_errors_surface_as_zero_handle(core, device):
    assert core._lib.tm_compile_msl(b"not hip at all") == 0
    assert "HIP compilation failed" in core.last_error()


def _host_view(core, handle, n):
    """What the reference's MetalBuffer._view() builds (python/triton_metal/
    buffer.py:62-63): a ctypes array over tm_buffer_contents."""
    return (ctypes.c_float * n).from_address(core.buffer_contents(handle))


def test_buffer_contents_is_a_host_view(core, device):
    """tm_buffer_contents is host-addressable, as the reference's unified
    memory is: values written with tm_buffer_write are visible through it,
    values written through it reach tm_buffer_read and the next launch, and a
    launch's results are in it when the launch returns."""
    src = _upload(core, [float(i) for i in range(64)])
    dst = core.alloc_buffer(256)
    library = core.compile_msl(COPY)
    kernel = core.load_kernel(library, "copy_kernel")
    try:
        view = _host_view(core, src, 64)
        assert core.buffer_contents(src) % 16 == 0
        assert list(view) == [float(i) for i in range(64)]
        for i in range(64):
            view[i] = 100.0 + i                  # host writes through the pointer
        assert list(_download(core, src, 64)) == [100.0 + i for i in range(64)]
        out = _host_view(core, dst, 64)          # mapped before the launch
        core.launch(kernel, (1, 1, 1), 64, [core.ARG_BUFFER] * 2, [src, dst])
        assert list(out) == [100.0 + i for i in range(64)]
        assert list(_download(core, dst, 64)) == [100.0 + i for i in range(64)]
        value = ctypes.c_float(-2.5)
        core.buffer_write(src, 8, ctypes.addressof(value), 4)
        assert view[2] == -2.5
        # the reference's tolist(): list(self._view())
        assert list(_host_view(core, src, 4)) == [100.0, 101.0, -2.5, 103.0]
    finally:
        core.free_buffer(src)
        core.free_buffer(dst)
        core.release_kernel(kernel)
        core.release_library(library)


def test_unmap_drops_the_host_mirror(core, device):
    """tm_buffer_unmap copies host writes made through the mirror down to HBM,
    frees it, and later launches work on HBM alone; a second
    tm_buffer_contents makes a fresh mirror of the current contents."""
    src = _upload(core, [float(i) for i in range(64)])
    dst = core.alloc_buffer(256)
    library = core.compile_msl(COPY)
    kernel = core.load_kernel(library, "copy_kernel")
    try:
        view = _host_view(core, src, 64)
        view[5] = -7.0                           # written through the mirror only
        assert core._lib.tm_buffer_unmap(src) == 0
        assert core._lib.tm_buffer_unmap(src) == 0   # no mirror: no-op
        core.launch(kernel, (1, 1, 1), 64, [core.ARG_BUFFER] * 2, [src, dst])
        want = [float(i) for i in range(64)]
        want[5] = -7.0
        assert list(_download(core, dst, 64)) == want
        assert list(_host_view(core, src, 64)) == want
        assert core._lib.tm_buffer_unmap(src) == 0
        assert core._lib.tm_buffer_unmap(0) == -1
        assert "is not live" in core.last_error()
    finally:
        core.free_buffer(src)
        core.free_buffer(dst)
        core.release_kernel(kernel)
        core.release_library(library)


def test_host_view_of_a_kernel_output_mapped_after_the_launch(core, device):
    src = _upload(core, [float(i) for i in range(64)])
    dst = core.alloc_buffer(256)
    library = core.compile_msl(COPY)
    kernel = core.load_kernel(library, "copy_kernel")
    try:
        core.launch(kernel, (1, 1, 1), 64, [core.ARG_BUFFER] * 2, [src, dst])
        assert list(_host_view(core, dst, 64)) == [float(i) for i in range(64)]
    finally:
        core.free_buffer(src)
        core.free_buffer(dst)
        core.release_kernel(kernel)
        core.release_library(library)


def test_copy_bounds_do_not_wrap(core, device):
    handle = core.alloc_buffer(16)
    byte = ctypes.c_uint8(0)
    try:
        assert core._lib.tm_buffer_write(handle, 2**63 - 1, ctypes.addressof(byte), 1) == -1
        assert "exceeds the" in core.last_error()
        assert core._lib.tm_buffer_read(handle, 15, ctypes.addressof(byte), 2**63 - 1) == -1
        assert "exceeds the" in core.last_error()
        assert core._lib.tm_buffer_read(handle, 15, ctypes.addressof(byte), 1) == 0
    finally:
        core.free_buffer(handle)


def test_async_launch_survives_releasing_its_handles(core, device):
    """A dispatch still queued when its kernel and library are released runs to
    completion: the library drains its stream before unloading the code object."""
    n = 1 << 20
    a = _upload(core, [1.0] * n)
    b = _upload(core, [2.0] * n)
    out = core.alloc_buffer(4 * n)
    library = core.compile_msl(VECTOR_ADD)
    kernel = core.load_kernel(library, "add_kernel")
    try:
        B, I = core.ARG_BUFFER, core.ARG_I32
        for _ in range(4):
            assert core._lib.tm_launch_async(kernel, n // 1024, 1, 1, 256,
                                             (ctypes.c_int32 * 4)(B, B, B, I),
                                             (ctypes.c_int64 * 4)(a, b, out, n), 4) == 0
        core.release_kernel(kernel)
        core.release_library(library)
        assert core._lib.tm_synchronize() == 0
        got = _download(core, out, n)
        assert got[0] == 3.0 and got[n - 1] == 3.0
    finally:
        for h in (a, b, out):
            core.free_buffer(h)


def test_code_object_loading_through_the_abi(core, device, tmp_path):
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(hipcc):
        pytest.fail("hipcc is missing on a GPU box")
    src = tmp_path / "copy.hip"
    src.write_text("#include <hip/hip_runtime.h>\n" + COPY)
    image_path = tmp_path / "copy.hsaco"
    subprocess.run([hipcc, "--offload-arch=gfx950", "--genco", "-O2", str(src), "-o",
                    str(image_path)], check=True, timeout=120)
    image = image_path.read_bytes()
    library = core.load_metallib(image)
    kernel = core.load_kernel(library, "copy_kernel")
    src_buf = _upload(core, [float(i) for i in range(64)])
    dst_buf = core.alloc_buffer(256)
    try:
        core.launch(kernel, (1, 1, 1), 64, [core.ARG_BUFFER] * 2, [src_buf, dst_buf])
        assert list(_download(core, dst_buf, 64)) == [float(i) for i in range(64)]
    finally:
        core.free_buffer(src_buf)
        core.free_buffer(dst_buf)
        core.release_kernel(kernel)
        core.release_library(library)
    garbage = bytes([0xAB] * 64)
    assert core._lib.tm_load_metallib(garbage, 64) == 0
    assert "could not load metallib" in core.last_error()


def test_device_buffer_exposes_data_ptr(core, device):
    from triton_metal.buffer import MetalBuffer
    live = core.live_handle_count()
    buffer = MetalBuffer((4, 8), "float32")
    try:
        assert buffer.nbytes == 128
        assert buffer.data_ptr() % 16 == 0
        source = array.array("f", [1.5] * 32)
        buffer.copy_from(source.buffer_info()[0])
        assert buffer.tolist()[:3] == [1.5, 1.5, 1.5]
        bf = MetalBuffer(8, "bfloat16")
        assert bf.itemsize == 2 and bf.nbytes == 16
        bf.write(np.arange(8, dtype=np.float32))
        assert list(bf.float32()) == list(range(8))
        bf.free()
    finally:
        buffer.free()
    assert core.live_handle_count() == live


def test_builtin_launch_checks_buffer_extents(core, device):
    lib = core.compile_msl("builtin element=f32")
    kernel = core.load_kernel(lib, "matmul_kernel")
    small = core.alloc_buffer(64)
    try:
        with pytest.raises(RuntimeError, match="needs 4096 bytes but its buffer holds 64"):
            core.launch(kernel, (1, 1, 1), 128, [0, 0, 0] + [1] * 9,
                        [small, small, small, 32, 32, 32, 32, 1, 32, 1, 32, 1])
    finally:
        core.free_buffer(small)
        core.release_kernel(kernel)
        core.release_library(lib)


@pytest.mark.parametrize("builtin,args", [
    # M = 2^31 - 1 rows at a stride of 2^31 - 1: the extent in bytes exceeds 2^63
    ("matmul_kernel", [2**31 - 1, 1, 1, 2**31 - 1, 1, 1, 1, 1, 1]),
    # 65535 heads of 2^31 - 1 rows at stride 2^31 - 1
    ("attn_bwd_preprocess", [2**31 - 1, 2**31 - 1, 2**31 - 1, 2**31 - 1]),
])
def test_extent_checks_do_not_wrap(core, device, builtin, args):
    """Sizes whose byte extent overflows 64 bits are refused on the host, not
    wrapped into a small number that passes the check."""
    lib = core.compile_msl("builtin element=f32")
    kernel = core.load_kernel(lib, builtin)
    small = core.alloc_buffer(64)
    try:
        nbuf = 3
        grid = (1, 1, 1) if builtin == "matmul_kernel" else (1, 65535, 1)
        with pytest.raises(RuntimeError, match="needs 9223372036854775807 bytes but its buffer holds 64"):
            core.launch(kernel, grid, 128, [0] * nbuf + [1] * len(args), [small] * nbuf + args)
    finally:
        core.free_buffer(small)
        core.release_kernel(kernel)
        core.release_library(lib)


def test_concurrent_launches_from_several_threads(core, device):
    """Threads sharing one library and kernel handle launch GEMMs on their own
    buffers at once (tm_launch holds no caller state between calls): every
    result is right and no handle leaks."""
    import threading

    from triton_metal import ops
    from triton_metal.buffer import DeviceBuffer
    kernel = ops.library("bf16").kernels["matmul_kernel"]
    live = core.live_handle_count()
    errors = []

    def worker(seed):
        try:
            rng = np.random.default_rng(seed)
            m, n, k = 256 + 64 * seed, 512, 128 + 32 * seed
            a = rng.standard_normal((m, k), dtype=np.float32)
            b = rng.standard_normal((k, n), dtype=np.float32)
            A = DeviceBuffer.from_numpy(a, "bfloat16")
            B = DeviceBuffer.from_numpy(b, "bfloat16")
            C = DeviceBuffer((m, n), "bfloat16")
            try:
                a, b = A.float32(), B.float32()
                for _ in range(5):
                    grid, kinds, values = ops.matmul_args(A, B, C, m, n, k)
                    core.launch(kernel, grid, 128, kinds, values)
                    got = C.float32()
                    want = a.astype(np.float64) @ b.astype(np.float64)
                    err = np.max(np.abs(got - want) / np.maximum(1.0, np.abs(want)))
                    if err > 2e-2:
                        errors.append((seed, float(err)))
            finally:
                for x in (A, B, C):
                    x.free()
        except Exception as e:  # noqa: BLE001 - reported below
            errors.append((seed, repr(e)))

    threads = [threading.Thread(target=worker, args=(t,)) for t in range(6)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert errors == []
    assert core.live_handle_count() == live


def test_concurrent_workspace_launches_from_several_threads(core, device):
    """Threads sharing one library launch GEMMs that take the K-split path
    (fp32 partials in the library workspace, then a reduce dispatch) with
    sizes that grow the workspace while other threads' sequences are queued
    (tm_launch_async, one wait at the end).  Each launch plans and queues its
    whole sequence under the library's launch lock, so no sequence binds a
    freed workspace or sums another thread's partials."""
    import threading

    from triton_metal import ops
    from triton_metal.buffer import DeviceBuffer
    kernel = ops.library("bf16").kernels["matmul_kernel"]
    errors = []
    barrier = threading.Barrier(4)

    def worker(seed):
        try:
            rng = np.random.default_rng(100 + seed)
            # a few rows against a long K: the planner splits K across workgroups
            m, n, k = 64, 1024 + 256 * seed, 4096 + 2048 * seed
            a = rng.standard_normal((m, k), dtype=np.float32)
            b = rng.standard_normal((k, n), dtype=np.float32)
            A = DeviceBuffer.from_numpy(a, "bfloat16")
            B = DeviceBuffer.from_numpy(b, "bfloat16")
            outs = [DeviceBuffer((m, n), "bfloat16") for _ in range(4)]
            try:
                a, b = A.float32(), B.float32()
                want = a.astype(np.float64) @ b.astype(np.float64)
                barrier.wait()
                for C in outs:
                    grid, kinds, values = ops.matmul_args(A, B, C, m, n, k)
                    core.launch_async(kernel, grid, 128, kinds, values)
                core.synchronize()
                for C in outs:
                    got = C.float32()
                    err = np.max(np.abs(got - want) / np.maximum(1.0, np.abs(want)))
                    if err > 2e-2:
                        errors.append((seed, float(err)))
            finally:
                for x in (A, B, *outs):
                    x.free()
        except Exception as e:  # noqa: BLE001 - reported below
            errors.append((seed, repr(e)))

    threads = [threading.Thread(target=worker, args=(t,)) for t in range(4)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert errors == []
    assert "K ranges" in core.kernel_variant(kernel)


BLOCK_KERNEL = r"""
#include <hip/hip_runtime.h>
struct Block { const void *a, *b; void *c; int m, n, k, s0, s1, s2, s3, s4, s5; const void *bias; };
extern "C" __global__ void block_kernel(Block p) { if (threadIdx.x == 0) ((int *)p.c)[0] = p.m; }
/* 28 bytes of fields, 4 bytes of tail padding */
struct Tail { const void *a; void *b; int m, n, k; };
extern "C" __global__ void tail_kernel(Tail p) { if (threadIdx.x == 0) ((int *)p.b)[0] = p.m + p.n + p.k; }
"""


def test_user_launches_must_bind_the_declared_arguments(core, device, tmp_path):
    """The library reads each user kernel's parameter layout from its code
    object and refuses a launch that packs another one: the kernel would read
    its grid size and the rest of its implicit values from the wrong bytes."""
    library = core.compile_msl(SCALE_BIAS)
    kernel = core.load_kernel(library, "scale_bias_kernel")
    bin_, bout = core.alloc_buffer(256), core.alloc_buffer(256)
    try:
        with pytest.raises(RuntimeError, match=r"declares 5 arguments \(28 bytes\) but the launch "
                                               r"binds 3 \(20 bytes\)"):
            core.launch(kernel, (1, 1, 1), 64, [core.ARG_BUFFER, core.ARG_BUFFER, core.ARG_I32],
                        [bin_, bout, 4])
        with pytest.raises(RuntimeError, match=r"argument 2 is 4 bytes at offset 16 \(by_value\) "
                                               r"but the launch binds 8 bytes at offset 16"):
            core.launch(kernel, (1, 1, 1), 64,
                        [core.ARG_BUFFER, core.ARG_BUFFER, core.ARG_I64, core.ARG_F32, core.ARG_I32],
                        [bin_, bout, 1, core.float_bits(1.0), 4])
    finally:
        core.free_buffer(bin_)
        core.free_buffer(bout)
        core.release_kernel(kernel)
        core.release_library(library)

    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    src = tmp_path / "block.hip"
    src.write_text(BLOCK_KERNEL)
    image_path = tmp_path / "block.hsaco"
    subprocess.run([hipcc, "--offload-arch=gfx950", "--genco", "-O2", str(src), "-o",
                    str(image_path)], check=True, timeout=120)
    library = core.load_metallib(image_path.read_bytes())
    kernel = core.load_kernel(library, "block_kernel")
    out = core.alloc_buffer(64)
    try:
        # the reference's 12 matmul arguments against one 72-byte by-value block
        with pytest.raises(RuntimeError, match=r"declares 1 argument \(72 bytes\) but the launch "
                                               r"binds 12 \(60 bytes\)"):
            core.launch(kernel, (1, 1, 1), 64, [core.ARG_BUFFER] * 3 + [core.ARG_I32] * 9,
                        [out, out, out] + [7] * 9)
        # a by-value struct may be bound field by field, in order (13 fields, 72 bytes)
        core.launch(kernel, (1, 1, 1), 64, [core.ARG_BUFFER] * 3 + [core.ARG_I32] * 9 + [core.ARG_I64],
                    [out, out, out] + [7] * 9 + [0])
        assert _download(core, out, 1, "i")[0] == 7
        # one argument that covers only the start of the block
        with pytest.raises(RuntimeError, match=r"argument 0 is 72 bytes at offset 0 \(by_value\) "
                                               r"but the launch binds 8 bytes at offset 0"):
            core.launch(kernel, (1, 1, 1), 64, [core.ARG_I64], [0])
        # a struct whose fields stop short of its size by tail padding only
        tail = core.load_kernel(library, "tail_kernel")
        try:
            core.launch(tail, (1, 1, 1), 64, [core.ARG_BUFFER] * 2 + [core.ARG_I32] * 3,
                        [out, out, 1, 20, 300])
            assert _download(core, out, 1, "i")[0] == 321
            with pytest.raises(RuntimeError, match=r"declares 1 argument \(32 bytes\) but the launch "
                                                   r"binds 4 \(24 bytes\)"):
                core.launch(tail, (1, 1, 1), 64, [core.ARG_BUFFER] * 2 + [core.ARG_I32] * 2,
                            [out, out, 1, 20])
        finally:
            core.release_kernel(tail)
    finally:
        core.free_buffer(out)
        core.release_kernel(kernel)
        core.release_library(library)


@pytest.mark.parametrize("element", ["bf16", "f32"])
def test_batch_in_z_grid_matches_flattened_heads(core, device, element):
    """The reference's callers put B*H in program_id(1) (attention_training.py:
    223-246); a caller that carries the batch in z, grid (cdiv(S, BLOCK_M), H, B),
    gets the same results as the flattened (cdiv(S, BLOCK_M), B*H, 1): the
    built-ins take heads = gy * gz."""
    from triton_metal import ops
    batch, heads, seq, dim = 2, 3, 96, 64
    rng = np.random.default_rng(5)
    layer = ops.AttentionLayer(batch * heads, seq, dim, element, causal=True)
    try:
        for name in ("q", "k", "v", "do"):
            layer.upload(name, rng.standard_normal((batch * heads, seq, dim), dtype=np.float32))
        kern = layer.lib.kernels
        results = []
        for split in (False, True):
            for name, (grid, kinds, values) in (("attn_fwd", layer.fwd_args()),
                                                ("attn_bwd_preprocess", layer.pre_args()),
                                                ("attn_bwd_dq", layer.dq_args()),
                                                ("attn_bwd_dkdv", layer.dkdv_args())):
                if split:
                    grid = (grid[0], heads, batch)
                core.launch(kern[name], grid, 128, kinds, values)
            results.append({n: layer.read(n) for n in ("o", "lse", "dq", "dk", "dv")})
        for n in results[0]:
            assert np.array_equal(results[0][n], results[1][n]), n
    finally:
        layer.free()
