"""The tm_* C ABI contract, on any machine (no GPU needed).

Mirrors the reference's Tests/TritonMetalCoreTests/CABITests.swift:19-318 and
python/tests/test_plugin_shape.py:112-355 for everything that does not need a
kernel to run: exports, sentinels, tm_last_error text, NULL arguments, handle
validity, launch-argument validation and the built-in library's metadata.
"""

import ctypes
import json
import re
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]


def declared_exports():
    text = (ROOT / "include" / "tritonmetal.h").read_text()
    return sorted(set(re.findall(r"^[a-z][\w \*]*?\b(tm_\w+)\(", text, re.M)))


def test_library_is_the_in_tree_build(core):
    assert Path(core.LIBRARY_PATH).resolve() == (
        ROOT / "triton-metal_amd" / "lib" / "libtritonmetal.so").resolve()


def test_every_declared_export_is_present(core):
    names = declared_exports()
    assert len(names) == 29
    for name in names:
        assert hasattr(core._lib, name), name
    # The reference's 23 exports are all declared.
    assert set(core.REFERENCE_EXPORTS) <= set(names)


def test_version_round_trip(core):
    assert core.version() == "0.0.1"


def test_is_usable_agrees_with_its_reason(core):
    usable = core.is_usable()
    reason = core.unusable_reason()
    assert (reason is None) == usable
    if usable:
        assert core.is_active()
        assert "gfx950" in core.device_name()
    if not core.is_active():
        assert core.device_name() is None


def test_last_error_is_cleared_by_reading(core):
    assert core._lib.tm_alloc_buffer(0) == 0
    assert "buffer length must be positive" in core.last_error()
    assert core.last_error() == "no error"


def test_invalid_handles_are_rejected(core):
    lib = core._lib
    assert lib.tm_load_kernel(999_999, b"k") == 0
    assert "library handle 999999 is not live" in core.last_error()
    assert lib.tm_buffer_length(999_999) == -1
    assert "is not live" in core.last_error()
    assert lib.tm_free_buffer(999_999) == -1
    assert lib.tm_launch(999_999, 1, 1, 1, 32, None, None, 0) == -1
    assert "kernel handle" in core.last_error()
    assert lib.tm_kernel_max_threads(999_999) == -1
    assert "kernel handle 999999 is not live" in core.last_error()
    assert lib.tm_buffer_contents(999_999) is None
    assert "is not live" in core.last_error()
    assert lib.tm_release_kernel(999_999) == -1
    assert lib.tm_release_library(999_999) == -1
    with pytest.raises(RuntimeError, match="is not live"):
        core.load_kernel(999_999, "matmul_kernel")
    with pytest.raises(RuntimeError, match="is not live"):
        core.buffer_length(999_999)


def test_null_string_arguments_are_rejected(core):
    lib = core._lib
    assert lib.tm_emit_msl(None, 4) is None
    assert "tm_emit_msl received a NULL module" in core.last_error()
    assert lib.tm_kernel_info(None, 4) is None
    assert "tm_kernel_info received a NULL module" in core.last_error()
    assert lib.tm_compile_msl(None) == 0
    assert "tm_compile_msl received NULL source" in core.last_error()
    assert lib.tm_load_kernel(1, None) == 0
    assert "NULL kernel name" in core.last_error()


def test_empty_code_object_is_rejected(core):
    assert core._lib.tm_load_metallib(None, 0) == 0
    assert "empty image" in core.last_error()


def test_bad_copies_are_refused_before_the_handle_is_looked_up(core):
    value = ctypes.c_float(0)
    lib = core._lib
    assert lib.tm_buffer_write(1, 0, None, 4) == -1
    assert "invalid bounds" in core.last_error()
    assert lib.tm_buffer_write(1, 0, ctypes.byref(value), -1) == -1
    assert "invalid bounds" in core.last_error()
    assert lib.tm_buffer_read(1, -4, ctypes.byref(value), 4) == -1
    assert "invalid bounds" in core.last_error()


def test_ttir_is_not_lowered(core):
    with pytest.raises(RuntimeError, match="ttir lowering is not part of this library"):
        core.emit_msl("module {}")
    with pytest.raises(RuntimeError, match="ttir lowering is not part of this library"):
        core.kernel_info("module {}")


# --- the built-in library ----------------------------------------------------


def test_builtin_spec_round_trips_through_emit(core):
    assert core.emit_msl("builtin element=bf16 head_dim=128 causal=1") == \
        "builtin element=bf16 head_dim=128 causal=1"
    assert core.emit_msl("builtin") == "builtin element=f32 head_dim=64 causal=0"
    assert core.emit_msl("builtin element=bf16 bwd=split") == \
        "builtin element=bf16 head_dim=64 causal=0"
    assert core.emit_msl("builtin element=bf16 head_dim=128 bwd=atomic") == \
        "builtin element=bf16 head_dim=128 causal=0 bwd=atomic"


@pytest.mark.parametrize("spec,message", [
    ("builtin element=f64", "unsupported element 'f64'"),
    ("builtin head_dim=0", "head_dim must be an integer in 1..128"),
    ("builtin head_dim=129", "head_dim must be an integer in 1..128"),
    ("builtin causal=2", "causal must be 0 or 1"),
    ("builtin bwd=fast", "bwd must be split or atomic"),
    ("builtin bwd=stash", "bwd must be split or atomic"),
    ("builtin colour=red", "unknown key 'colour'"),
    ("builtin element", "expected key=value"),
])
def test_builtin_spec_errors(core, spec, message):
    with pytest.raises(RuntimeError, match=re.escape(message)):
        core.compile_msl(spec)


def test_kernel_info_publishes_every_builtin(core):
    info = json.loads(core.kernel_info("builtin element=bf16 head_dim=128 causal=1"))
    kernels = {k["name"]: k for k in info["kernels"]}
    assert set(kernels) == {"matmul_kernel", "attn_fwd", "attn_bwd_preprocess", "attn_bwd_dq",
                            "attn_bwd_dkdv", "sae_encode_kernel", "tm_probe"}
    mm = kernels["matmul_kernel"]
    assert [a["dtype"] for a in mm["args"]] == ["bf16"] * 3 + ["i32"] * 9
    assert [a["kind"] for a in mm["args"]] == [0, 0, 0] + [1] * 9
    fwd = kernels["attn_fwd"]
    # Q, K, V, O, sm_scale, stride_head, stride_seq, n_ctx, L, stride_lse
    # (AttentionKernel.swift:75-78 with emitStats).
    assert [a["kind"] for a in fwd["args"]] == [0, 0, 0, 0, 2, 1, 1, 1, 0, 1]
    assert fwd["args"][8]["dtype"] == "f32"
    assert fwd["head_dim"] == 128 and fwd["causal"] is True
    dkdv = kernels["attn_bwd_dkdv"]
    assert len(dkdv["args"]) == 13
    for k in kernels.values():
        assert k["threads_per_threadgroup"] > 0 and k["block_size"] > 0


def test_fused_backward_is_offered_only_with_bwd_atomic(core):
    split = json.loads(core.kernel_info("builtin element=bf16 head_dim=128 causal=1"))
    assert "attn_bwd_fused" not in {k["name"] for k in split["kernels"]}
    info = json.loads(core.kernel_info("builtin element=bf16 head_dim=128 causal=1 bwd=atomic"))
    fused = {k["name"]: k for k in info["kernels"]}["attn_bwd_fused"]
    # Q, K, V, dO, dQ, dK, dV, L, Delta, sm_scale, stride_head, stride_seq,
    # stride_lse, n_ctx: the dK/dV list with dQ inserted before dK
    assert [a["kind"] for a in fused["args"]] == [0] * 9 + [2, 1, 1, 1, 1]
    assert [a["dtype"] for a in fused["args"]] == ["bf16"] * 7 + ["f32"] * 3 + ["i32"] * 4
    lib = core.compile_msl("builtin element=bf16 head_dim=128 causal=1")
    try:
        with pytest.raises(RuntimeError, match="bwd=atomic"):
            core.load_kernel(lib, "attn_bwd_fused")
    finally:
        core.release_library(lib)


def test_sae_encoder_declares_the_arguments_its_wrapper_binds(core):
    # SAEEncoderTests.swift:138-145: four f32 pointers (x, w, b, out), three
    # i32 scalars (M, D, F), block shape [64, 64].
    info = json.loads(core.kernel_info("builtin element=f32"))
    sae = {k["name"]: k for k in info["kernels"]}["sae_encode_kernel"]
    assert [a["dtype"] for a in sae["args"]] == ["f32"] * 4 + ["i32"] * 3
    assert [a["kind"] for a in sae["args"]] == [0] * 4 + [1] * 3
    assert [a["index"] for a in sae["args"]] == list(range(7))
    assert sae["block_shape"] == [64, 64]


@pytest.mark.parametrize("shapes,message", [
    # SAEEncoderTests.swift:118-135, same inputs and messages.
    (((8, 64), (32, 128), (128,)), "contraction dimensions differ"),
    (((8, 64), (64, 128), (64,)), "128 features but b_enc has 64"),
    (((8,), (64, 128), (128,)), "expects x [M, D]"),
    (((8, 64), (64, 128), (1, 128)), "expects x [M, D]"),
])
def test_sae_encoder_refuses_mismatched_shapes(shapes, message):
    from triton_metal.ops import SAEEncoder
    with pytest.raises(ValueError, match=re.escape(message)):
        SAEEncoder.check_shapes(*shapes)
    assert SAEEncoder.check_shapes((8, 64), (64, 128), (128,)) == (8, 64, 128)


def test_builtin_kernels_load_by_reference_name(core):
    live = core.live_handle_count()
    lib = core.compile_msl("builtin element=f16 head_dim=80")
    handles = [core.load_kernel(lib, n) for n in
               ("matmul_kernel", "attn_fwd", "attn_bwd_preprocess", "attn_bwd_dq", "attn_bwd_dkdv",
                "sae_encode_kernel")]
    assert all(h > 0 for h in handles)
    assert core.kernel_max_threads(handles[0]) >= 128
    with pytest.raises(RuntimeError, match=r"kernel 'add_kernel' not found in library \(available: "):
        core.load_kernel(lib, "add_kernel")
    for h in handles:
        core.release_kernel(h)
    core.release_library(lib)
    assert core.live_handle_count() == live


@pytest.fixture
def matmul_kernel(core):
    lib = core.compile_msl("builtin element=f32")
    kernel = core.load_kernel(lib, "matmul_kernel")
    yield kernel
    core.release_kernel(kernel)
    core.release_library(lib)


def test_unknown_launch_argument_kind_is_rejected(core, matmul_kernel):
    with pytest.raises(RuntimeError, match="unknown launch argument kind 7"):
        core.launch(matmul_kernel, (1, 1, 1), 32, [7], [0])


def test_null_argument_arrays_are_rejected(core, matmul_kernel):
    assert core._lib.tm_launch(matmul_kernel, 1, 1, 1, 128, None, None, 5) == -1
    assert "NULL argument arrays" in core.last_error()


def test_launch_geometry_is_validated(core, matmul_kernel):
    kinds = [core.ARG_I32] * 12
    with pytest.raises(RuntimeError, match="grid must be positive"):
        core.launch(matmul_kernel, (0, 1, 1), 128, kinds, [1] * 12)
    with pytest.raises(RuntimeError, match="exceeds the pipeline maximum"):
        core.launch(matmul_kernel, (1, 1, 1), 2048, kinds, [1] * 12)


def test_builtin_signatures_are_enforced(core, matmul_kernel):
    with pytest.raises(RuntimeError, match="matmul_kernel expects 12 arguments, got 3"):
        core.launch(matmul_kernel, (1, 1, 1), 128, [1, 1, 1], [1, 2, 3])
    with pytest.raises(RuntimeError, match=r"argument 0 must be a buffer \(kind 0\), got kind 1"):
        core.launch(matmul_kernel, (1, 1, 1), 128, [1] * 12, [1] * 12)
    lib = core.compile_msl("builtin element=bf16 head_dim=64")
    fwd = core.load_kernel(lib, "attn_fwd")
    try:
        with pytest.raises(RuntimeError, match="attn_fwd expects 8 or 10 arguments, got 9"):
            core.launch(fwd, (1, 1, 1), 128, [1] * 9, [0] * 9)
    finally:
        core.release_kernel(fwd)
        core.release_library(lib)


# --- the Python buffer object --------------------------------------------------


def test_buffer_rejects_a_dtype_with_no_element_type():
    from triton_metal.buffer import MetalBuffer
    with pytest.raises(TypeError, match="unsupported dtype"):
        MetalBuffer(4, "float64")


def test_bf16_conversion_rounds_to_nearest_even():
    from triton_metal.buffer import bf16_bits, bf16_values
    x = np.array([1.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -2.5, 3.0e38, np.inf, 1e-40],
                 dtype=np.float32)
    bits = bf16_bits(x)
    # 1 + 2^-8 is a tie between 1 and 1 + 2^-7: even mantissa (1.0) wins;
    # 1 + 3*2^-8 ties between 1+2^-7 and 1+2^-6: 1+2^-6 is even.
    assert list(bf16_values(bits)[:4]) == [1.0, 1.0, 1.0 + 2 ** -6, -2.5]
    assert bits[0] == 0x3F80
    assert np.isinf(bf16_values(bits)[5])
    assert np.isnan(bf16_values(bf16_bits(np.array([np.nan], np.float32))))[0]
    assert np.array_equal(bf16_values(bf16_bits(bf16_values(bits))), bf16_values(bits))


def test_handle_table_is_safe_under_concurrent_use(core):
    """The handle table is one locked table shared by every thread (the
    reference's Runtime.swift:250-290): concurrent create/load/release from
    several threads yields unique handles, every release succeeds, and the live
    count returns to where it started."""
    import threading

    names = ("matmul_kernel", "attn_fwd", "attn_bwd_preprocess", "attn_bwd_dq", "attn_bwd_dkdv",
             "sae_encode_kernel")
    live = core.live_handle_count()
    seen, errors, lock = [], [], threading.Lock()

    def worker(seed):
        try:
            for i in range(60):
                spec = f"builtin element={('f32', 'f16', 'bf16')[(seed + i) % 3]} head_dim=64"
                lib = core.compile_msl(spec)
                kernels = [core.load_kernel(lib, n) for n in names]
                with lock:
                    seen.extend([lib] + kernels)
                for k in kernels:
                    core.release_kernel(k)
                core.release_library(lib)
        except Exception as exc:  # surfaced below
            errors.append(repr(exc))

    threads = [threading.Thread(target=worker, args=(t,)) for t in range(8)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors[:3]
    assert len(seen) == len(set(seen)) == 8 * 60 * 7
    assert core.live_handle_count() == live
