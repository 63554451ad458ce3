"""sae_encode_kernel, the fused encoder relu(x @ W_enc + b_enc), on the device
against the fp64 oracle.

Cases follow Tests/TritonMetalMLXTests/SAEEncoderTests.swift:28-180 with its
inputs (MLXTestSupport.swift:82-90) and its metric: max |got - want| divided by
max(max |want|, 1), below 2e-6 for f32 (:28-41).  The 16-bit element types
are this build's extension, checked with the GEMM's hybrid metric
|a - b| / max(1, |b|) against the oracle on inputs rounded to the element type
(DotTests.swift:533-553), at 2e-2."""

import numpy as np
import pytest

from oracle import generators as G
from oracle import reference as R
from oracle import tolerance as T
from triton_metal import _core, ops
from triton_metal.buffer import DeviceBuffer, round_to

pytestmark = pytest.mark.gpu

DT = {"f32": "float32", "f16": "float16", "bf16": "bfloat16"}


def inputs(rows, model, features):
    return (G.synthetic([rows, model], offset=1, modulus=71),
            G.synthetic([model, features], offset=7, modulus=53),
            G.synthetic([features], offset=3, modulus=29))


def scaled_error(got, want):
    return float(np.max(np.abs(got - want)) / max(float(np.max(np.abs(want))), 1.0))


def encode(x, w, b, element="f32"):
    return ops.SAEEncoder(element).numpy(x, w, b)


@pytest.mark.parametrize("rows,model,features", [
    (64, 32, 64), (128, 128, 256), (64, 512, 2048),          # whole blocks (:44-50)
    (100, 300, 700), (1, 1, 1), (7, 13, 5), (65, 33, 65),     # ragged (:52-60)
    (1, 512, 4096),                                           # one token, wide dictionary (:62-68)
    (2048, 256, 1024),                                        # 128 tiles: the fp32 MFMA kernel
])
def test_f32_matches_the_oracle(device, rows, model, features):
    x, w, b = inputs(rows, model, features)
    got = encode(x, w, b)
    assert got.shape == (rows, features)
    err = scaled_error(got, R.sae_encode(x, w, b))
    print(f"[{rows},{model}]@[{model},{features}] scaled error {err:.3g}")
    assert err < 2e-6


def test_relu_zeroes_the_negative_half(device):
    # SAEEncoderTests.swift:70-83: a -5 bias drives most units to exactly zero.
    x = G.synthetic([32, 64], offset=1)
    w = G.synthetic([64, 128], offset=7, modulus=53)
    b = np.full(128, -5.0, np.float32)
    got = encode(x, w, b)
    assert np.max(np.abs(got - R.sae_encode(x, w, b))) < 1e-6
    assert np.count_nonzero(got == 0) > 128
    assert got.min() == 0.0


def test_the_result_is_the_kernels_own_output_buffer(device):
    # SAEEncoderTests.swift:86-99: the kernel writes `out` in place; a grid of
    # (1, 1) is a request the library covers with its own tiles.
    x, w, b = (G.synthetic([64, 64], offset=1), G.synthetic([64, 64], offset=7, modulus=53),
               G.synthetic([64], offset=3, modulus=29))
    bufs = [DeviceBuffer.from_numpy(a, "float32") for a in (x, w, b)]
    out = DeviceBuffer((64, 64), "float32").write(np.full((64, 64), 7.0, np.float32))
    enc = ops.SAEEncoder("f32")
    _, kinds, values = enc.args(*bufs, out, 64, 64, 64)
    _core.launch(enc.kernel, (1, 1, 1), 128, kinds, values)
    assert np.max(np.abs(out.float32() - R.sae_encode(x, w, b))) < 1e-6
    for a in (*bufs, out):
        a.free()


def test_repeated_launches_agree(device):
    # SAEEncoderTests.swift:102-111.
    x, w, b = inputs(70, 130, 90)
    first = encode(x, w, b)
    for _ in range(4):
        assert np.array_equal(encode(x, w, b), first)


def test_zero_width_contraction_gives_relu_of_the_bias(device):
    b = G.synthetic([70], offset=3, modulus=29)
    enc = ops.SAEEncoder("f32")
    xb, wb = DeviceBuffer((3, 1), "float32"), DeviceBuffer((1, 70), "float32")
    bb = DeviceBuffer.from_numpy(b, "float32")
    out = DeviceBuffer((3, 70), "float32")
    _, kinds, values = enc.args(xb, wb, bb, out, 3, 0, 70)
    _core.launch(enc.kernel, (1, 2, 1), 128, kinds, values)
    assert np.array_equal(out.float32(), np.tile(np.maximum(b, 0), (3, 1)))
    for a in (xb, wb, bb, out):
        a.free()


def test_short_buffers_are_refused(device):
    enc = ops.SAEEncoder("f32")
    x, w, b = (DeviceBuffer(s, "float32") for s in ((8, 64), (64, 128), (64,)))
    out = DeviceBuffer((8, 128), "float32")
    _, kinds, values = enc.args(x, w, b, out, 8, 64, 128)
    with pytest.raises(RuntimeError, match="sae_encode_kernel argument 2 .b. needs 512 bytes"):
        _core.launch(enc.kernel, (1, 2, 1), 128, kinds, values)
    for a in (x, w, b, out):
        a.free()


@pytest.mark.parametrize("element", ["bf16", "f16"])
@pytest.mark.parametrize("rows,model,features,variant", [
    (512, 1024, 2048, "fast_t64"),   # whole 64 x 64 x 64 tiles
    (2048, 1024, 2048, "fast_t128"), # whole 128 x 128 x 64 tiles
    (100, 300, 700, "generic"),      # rows not 16-byte aligned
    (100, 512, 1000, "ragged_t64"),  # M and N short of whole tiles
    (333, 136, 264, "ragged_t64"),   # ragged K
    (4096, 256, 4096, "w4"),         # 256 tiles of 256 x 256: one per compute unit (4-wave kernel)
    (4000, 264, 4104, "ragged"),
])
def test_16bit_matches_the_oracle(device, element, rows, model, features, variant):
    rng = np.random.default_rng(5)
    x = round_to(rng.standard_normal((rows, model), dtype=np.float32), element)
    w = round_to(rng.standard_normal((model, features), dtype=np.float32) / np.sqrt(model), element)
    b = round_to(rng.standard_normal(features, dtype=np.float32), element)
    enc = ops.SAEEncoder(element)
    got = enc.numpy(x, w, b)
    assert _core.kernel_variant(enc.kernel) == f"tm_sae_{variant}_{element}"
    want = R.sae_encode(x, w, b)
    err = T.hybrid_error(got, want)
    print(f"{element} [{rows},{model}]@[{model},{features}] hybrid {err:.3g}")
    assert err <= 2e-2
    # the ReLU is exact: every unit whose pre-activation is clearly negative is 0
    assert np.all(got[want == 0] == 0) or np.all(np.abs(got[want == 0]) <= 2e-2)
    assert got.min() >= 0.0
