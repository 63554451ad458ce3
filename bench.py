"""Benchmark of the dense hot path on one MI355X, through the tm_* C ABI.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]

A step is one FlashAttention-2 forward + backward (attn_fwd, attn_bwd_preprocess,
attn_bwd_dq, attn_bwd_dkdv) at the benchmark's config 5: bf16, B4 H32 S4096 D128,
causal, Q/K/V/dO ~ N(0,1), inputs resident in HBM.  `value` is that step's
algorithmic TFLOP/s under the reference's FLOP convention (4*S^2*D forward,
10*S^2*D backward per batch*head, AttentionBenchmark.swift:64-68,
AttentionBackwardBenchmark.swift:45-49), halved for the causal mask.

Also measured in the same run and reported under "components":
  - bf16 GEMM 8192^3 (config 3), 2*M*N*K FLOPs;
  - bf16 FA2 forward at B8 H16 S1024 D64 non-causal (config 4);
  - the fused bf16 SAE encoder relu(x @ W_enc + b_enc) at 8192 x 2048 x 16384.
Per-kernel durations come from HIP events recorded on the library's stream
around back-to-back dispatches (tm_launch_timed).

The CPU baseline times the oracle's float32 BLAS restatement of the reference's
attention forward and backward (oracle/reference.py
attention_head_causal_blocked_f32, after attention_training.py:170-187, causal)
on a bounded sample of the workload on the host cores: one warm-up, median of 3.

After its timings every measured configuration is checked: sampled heads of O,
L, Delta, dQ, dK, dV and sampled rows of every GEMM and SAE output against fp64
from the same rounded inputs (the reference's verify-before-timing rule,
GEMMBenchmark.swift:320-375).  A miss prints the errors and exits 1 with no
JSON line; the line carries the errors under "verified".
Prints ONE JSON line.
"""

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "triton-metal_amd"))
sys.path.insert(0, str(ROOT))

import numpy as np  # noqa: E402

#: MI355X published dense peaks (TFLOP/s) and HBM bandwidth (GB/s).
PEAK_TFLOPS = {"bf16": 2500.0, "f16": 2500.0, "f32": 157.3}
PEAK_HBM_GBS = 8000.0

METRIC = "FA2 fwd/bwd TFLOP/s (b4 h32 s4096 d128 bf16) + GEMM TFLOP/s, % MFMA peak"


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--sample-ms", type=float, default=25.0,
                    help="GPU time per timing sample of one kernel (the reference packs "
                         "dispatches into ~25 ms samples and takes the median of 3)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=12.0,
                    help="target CPU time of the baseline sample")
    ap.add_argument("--only", choices=["all", "fa", "gemm", "reference"], default="all")
    ap.add_argument("--vendor", action="store_true",
                    help="time the vendor libraries on the same shapes (torch.matmul = hipBLASLt at "
                         "config 3; torch scaled_dot_product_attention, each ROCm backend, at "
                         "config 5) as one JSON line and exit; a comparison, not a baseline")
    ap.add_argument("--probes", action="store_true",
                    help="print the device probe rates (MFMA shapes, exp2, LDS reads, fp32 atomics) "
                         "as one JSON line and exit")
    ap.add_argument("--profile-pass", action="store_true",
                    help="for rocprofv3 --pmc runs: one copy kernel of known size (the "
                         "FETCH_SIZE / WRITE_SIZE calibration) and one dispatch of each hot kernel")
    ap.add_argument("--operand-data", choices=OPERAND_DATA, default="normal",
                    help="with --profile-pass: the operands' values (normal: N(0,1) as everywhere "
                         "else; trunc4: N(0,1) with the low 4 mantissa bits cleared; zeros)")
    ap.add_argument("--data-study", action="store_true",
                    help="time the config 5 attention kernels, the 8192^3 GEMM and the SAE encoder "
                         "on each kind of --operand-data (same shapes and instruction streams) as "
                         "one JSON line and exit")
    args = ap.parse_args()
    if args.operand_data != "normal" and not args.profile_pass:
        ap.error("--operand-data applies to --profile-pass only; the benchmark uses N(0,1)")
    return args


#: A plain device copy, the calibration kernel for rocprof's HBM byte counters.
COPY_SOURCE = r"""
extern "C" __global__ void tm_calibration_copy(const uint4 *src, uint4 *dst, long long n) {
  for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (long long)gridDim.x * blockDim.x)
    dst[i] = src[i];
}
"""
COPY_BYTES = 1 << 30


def profile_pass(core, ops):
    """One copy of COPY_BYTES (reads and writes that many bytes of HBM), then one
    dispatch each of attn_fwd, attn_bwd_preprocess, attn_bwd_dq, attn_bwd_dkdv at
    config 5, attn_fwd at config 4, the bwd=atomic backward (attn_bwd_fused: accumulator clear, fused
    kernel, dQ conversion) at config 5, matmul_kernel at config 3 and
    sae_encode_kernel at 8192 x 2048 x 16384."""
    from triton_metal.buffer import DeviceBuffer
    lib = core.compile_msl(COPY_SOURCE)
    kernel = core.load_kernel(lib, "tm_calibration_copy")
    src, dst = core.alloc_buffer(COPY_BYTES), core.alloc_buffer(COPY_BYTES)
    core.launch(kernel, (4096, 1, 1), 256, [0, 0, 3], [src, dst, COPY_BYTES // 16])
    core.free_buffer(src)
    core.free_buffer(dst)
    core.release_kernel(kernel)
    core.release_library(lib)
    B, H, S, D = 4, 32, 4096, 128
    layer = ops.AttentionLayer(B * H, S, D, "bf16", True)
    for i, name in enumerate(("q", "k", "v", "do")):
        layer.buffers[name].write(normal_bf16((B * H, S, D), 100 + i))
    layer.run_forward()
    layer.run_backward()
    layer.free()
    # config 4: the D = 64 forward
    c4 = ops.AttentionLayer(8 * 16, 1024, 64, "bf16", False)
    for i, name in enumerate(("q", "k", "v")):
        c4.buffers[name].write(normal_bf16((8 * 16, 1024, 64), 100 + i))
    c4.run_forward()
    c4.free()
    for mode in ("atomic",):
        fused = ops.AttentionLayer(B * H, S, D, "bf16", True, bwd=mode)
        for i, name in enumerate(("q", "k", "v", "do")):
            fused.buffers[name].write(normal_bf16((B * H, S, D), 100 + i))
        fused.run_forward()
        fused.run_backward()
        fused.free()
    n = 8192
    a = DeviceBuffer((n, n), "bfloat16").write(normal_bf16((n, n), 1))
    b = DeviceBuffer((n, n), "bfloat16").write(normal_bf16((n, n), 2))
    c = DeviceBuffer((n, n), "bfloat16")
    ops.matmul(a, b, c, n, n, n)
    for x in (a, b, c):
        x.free()
    rows, model, features = 8192, 2048, 16384
    x = DeviceBuffer((rows, model), "bfloat16").write(normal_bf16((rows, model), 3))
    w = DeviceBuffer((model, features), "bfloat16").write(normal_bf16((model, features), 4))
    bias = DeviceBuffer((features,), "bfloat16").write(normal_bf16((features,), 5))
    out = ops.SAEEncoder("bf16")(x, w, bias)
    for t in (x, w, bias, out):
        t.free()
    print(json.dumps({"profile_pass": "done", "copy_bytes": COPY_BYTES}), flush=True)


def vendor_reference():
    """torch's own kernels on this GPU at the headline shapes: hipBLASLt through
    torch.matmul (bf16 8192^3) and scaled_dot_product_attention (B4 H32 S4096
    D128 bf16 causal, forward and backward) under each backend torch offers on
    ROCm.  CUDA-event timing of back-to-back calls after a warm-up."""
    import torch
    import torch.nn.functional as F
    from torch.nn.attention import SDPBackend, sdpa_kernel

    def timed(fn, n, warm):
        for _ in range(warm):
            fn()
        torch.cuda.synchronize()
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(n):
            fn()
        stop.record()
        torch.cuda.synchronize()
        return start.elapsed_time(stop) / n

    out = {"torch": torch.__version__}
    n = 8192
    a = torch.randn(n, n, device="cuda", dtype=torch.bfloat16)
    b = torch.randn(n, n, device="cuda", dtype=torch.bfloat16)
    ms = timed(lambda: a @ b, 20, 5)
    out["matmul_bf16_8192"] = {"ms": round(ms, 4), "tflops": round(gemm_flops(n, n, n) / ms / 1e9, 1)}
    del a, b
    B, H, S, D = 4, 32, 4096, 128
    q, k, v = (torch.randn(B, H, S, D, device="cuda", dtype=torch.bfloat16, requires_grad=True)
               for _ in range(3))
    d_out = torch.randn(B, H, S, D, device="cuda", dtype=torch.bfloat16)
    f_fwd = attention_flops(B * H, S, D, True)
    f_bwd = attention_flops(B * H, S, D, True, backward=True)
    for name, backend in (("flash", SDPBackend.FLASH_ATTENTION),
                          ("efficient", SDPBackend.EFFICIENT_ATTENTION)):
        try:
            with sdpa_kernel(backend):
                fwd = lambda: F.scaled_dot_product_attention(q, k, v, is_causal=True)
                ms_f = timed(fwd, 10, 3)
                o = fwd()

                def bwd():
                    q.grad = k.grad = v.grad = None
                    o.backward(d_out, retain_graph=True)
                ms_b = timed(bwd, 10, 3)
            out[f"sdpa_{name}_config5"] = {
                "fwd_ms": round(ms_f, 4), "fwd_tflops": round(f_fwd / ms_f / 1e9, 1),
                "bwd_ms": round(ms_b, 4), "bwd_tflops": round(f_bwd / ms_b / 1e9, 1)}
        except RuntimeError as e:  # a backend this torch build lacks
            out[f"sdpa_{name}_config5"] = {"unavailable": str(e)[:200]}
    return out


#: Kinds of operand values for the data study: the MFMA-dense kernels run
#: slower on operands whose bits change more (the chip lowers its clock under
#: the power drawn), so the same kernel is timed on N(0,1), on N(0,1) with
#: fewer mantissa bits, and on zeros.
OPERAND_DATA = ("normal", "trunc4", "zeros")
_operand_data = "normal"


def normal_bf16(shape, seed):
    """N(0,1) from `seed` as bf16 bits; under the data study, transformed to
    the current kind of operand data."""
    from triton_metal.buffer import bf16_bits
    rng = np.random.default_rng(seed)
    x = bf16_bits(rng.standard_normal(shape, dtype=np.float32))
    if _operand_data == "trunc4":
        x &= np.uint16(0xFFF0)
    elif _operand_data == "zeros":
        x[...] = 0
    return x


def data_study(core, ops, sample_ms):
    """Kernel times on each kind of operand data, one process, same shapes."""
    global _operand_data
    out = {}
    try:
        for kind in OPERAND_DATA:
            _operand_data = kind
            _, per = bench_attention(core, ops, 4, 32, 4096, 128, True, 3, 3, sample_ms)
            rec = {name: round(v["ms"], 4) for name, v in per.items()}
            rec["gemm_bf16_8192"] = round(bench_gemm(core, ops, 8192, 3, sample_ms)[0], 4)
            rec["sae_encode_bf16_8192x2048x16384"] = round(
                bench_sae(core, ops, 8192, 2048, 16384, 3, sample_ms)[0], 4)
            out[kind] = rec
    finally:
        _operand_data = "normal"
    return out


def kernel_ms(core, kernel, grid, kinds, values, sample_ms):
    """Average duration of one dispatch, the reference's way
    (Sources/TritonMetalBench/GEMMBenchmark.swift:250-277): a calibration run
    sizes a sample of about `sample_ms` of back-to-back dispatches, a warm-up of
    four samples' worth settles the clocks, and the median of 3 samples timed
    with HIP events on the library stream is reported."""
    probe = core.launch_timed(kernel, grid, 128, kinds, values, 4) / 4
    repeats = max(4, int(sample_ms / max(probe, 1e-3)))
    core.launch_timed(kernel, grid, 128, kinds, values, 4 * repeats)
    samples = sorted(core.launch_timed(kernel, grid, 128, kinds, values, repeats) / repeats
                     for _ in range(3))
    return samples[1]


# --------------------------------------------------------------------------- #
# Verification of what was timed (the reference checks every benchmarked
# configuration against a CPU reference before believing its timings:
# GEMMBenchmark.swift:320-375, AttentionBackwardBenchmark.swift:263-414).
# fp64 numpy, outside every timed region; a miss ends the run without a line.
# --------------------------------------------------------------------------- #

#: bounds: O and the natural-log logsumexp within 2e-2 absolute, Delta, dQ,
#: dK, dV and GEMM rows within 2e-2 hybrid (|a - b| / max(1, |b|)) of fp64
#: computed from the same rounded inputs: north_star's 16-bit bar.  fp32
#: GEMMs: 1e-5 relative, max|a - b| / max|b| (its fp32 bar).
TOL_16 = 2e-2
TOL_F32 = 1e-5
#: fp32 attention: the reference's 2e-5 forward bound (AttentionTests.swift) with
#: room for the backward's longer sums
TOL_F32_ATTN = 1e-4


def _hybrid(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    if not np.all(np.isfinite(a)):
        return float("inf")
    return float(np.max(np.abs(a - b) / np.maximum(1.0, np.abs(b))))


def _relative(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    if not np.all(np.isfinite(a)):
        return float("inf")
    return float(np.max(np.abs(a - b)) / max(float(np.max(np.abs(b))), 1e-30))


def _abs(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    if not np.all(np.isfinite(a)):
        return float("inf")
    return float(np.max(np.abs(a - b)))


def _attention_head64(q, k, v, d_out, scale, causal):
    """One head in fp64: O, natural-log LSE, Delta, dQ, dK, dV (the
    definitions: softmax(Q K^T * scale) V and its gradients for upstream dO)."""
    q, k, v = (np.asarray(x, np.float64) for x in (q, k, v))
    s = (q @ k.T) * scale
    if causal:
        s[np.triu_indices(s.shape[0], 1)] = -np.inf
    peak = s.max(-1, keepdims=True)
    e = np.exp(s - peak)
    total = e.sum(-1, keepdims=True)
    p = e / total
    o = p @ v
    out = {"o": o, "lse": peak[:, 0] + np.log(total[:, 0])}
    if d_out is not None:
        d_out = np.asarray(d_out, np.float64)
        delta = np.sum(d_out * o, -1)
        ds = p * (d_out @ v.T - delta[:, None])
        out.update(delta=delta, dq=ds @ k * scale, dk=ds.T @ q * scale, dv=p.T @ d_out)
    return out


class Verifier:
    """Collects the worst error of every checked output; `failures` lists the
    outputs over their bound."""

    def __init__(self):
        self.record = {}
        self.failures = []

    def add(self, case, name, err, bound):
        rec = self.record.setdefault(case, {})
        rec[name] = max(rec.get(name, 0.0), round(err, 6))
        rec.setdefault("bound", {})[name] = bound
        if not err <= bound:
            self.failures.append(f"{case}.{name}: error {err:.3e} > {bound:g}")


def _read_rows(buf, first, count, row_elems):
    """Rows [first, first + count) of a buffer as float32 (bf16 decoded)."""
    from triton_metal import _core
    from triton_metal.buffer import _NUMPY, bf16_values
    out = np.empty(count * row_elems, dtype=_NUMPY[buf.dtype])
    _core.buffer_read(buf.tm_handle, first * row_elems * buf.itemsize, out.ctypes.data, out.nbytes)
    if buf.dtype == "bfloat16":
        return bf16_values(out).reshape(count, row_elems)
    return out.astype(np.float32).reshape(count, row_elems)


def _input_values(bits, element):
    """What a buffer of `element` holds after write() of bf16 words' values."""
    from triton_metal.buffer import bf16_values
    x = bf16_values(bits)
    return x.astype(np.float16).astype(np.float32) if element == "f16" else x


def verify_attention(layer, host, heads_to_check, verifier, case, backward):
    """The checked heads' outputs, read back after the timed runs, against fp64
    from the same rounded inputs."""
    seq, dim, el = layer.seq, layer.dim, layer.element
    tol = TOL_F32_ATTN if el == "f32" else TOL_16
    for h in heads_to_check:
        x = {n: _input_values(host[n][h], el) for n in host}
        want = _attention_head64(x["q"], x["k"], x["v"], x["do"] if backward else None,
                                 layer.scale, layer.causal)
        o = _read_rows(layer.buffers["o"], h * seq, seq, dim)
        lse = _read_rows(layer.buffers["lse"], h, 1, seq)[0]
        verifier.add(case, "o", _abs(o, want["o"]), tol)
        verifier.add(case, "lse", _abs(lse * math.log(2.0), want["lse"]), tol)
        if backward:
            # Delta is defined on the O the forward stored (element type), the
            # O attn_bwd_preprocess reads
            delta = _read_rows(layer.buffers["delta"], h, 1, seq)[0]
            want_delta = np.sum(o.astype(np.float64) * x["do"].astype(np.float64), -1)
            verifier.add(case, "delta", _hybrid(delta, want_delta), tol)
            for name in ("dq", "dk", "dv"):
                got = _read_rows(layer.buffers[name], h * seq, seq, dim)
                verifier.add(case, name, _hybrid(got, want[name]), tol)
    verifier.record[case]["heads"] = list(heads_to_check)


def bench_attention(core, ops, batch, heads, seq, dim, causal, steps, warmup, sample_ms,
                    backward=True, element="bf16", bwd="split", verifier=None, case=None,
                    check_heads=()):
    bh = batch * heads
    layer = ops.AttentionLayer(bh, seq, dim, element, causal, bwd=bwd)
    host = {}
    try:
        for i, name in enumerate(("q", "k", "v", "do")):
            x = normal_bf16((bh, seq, dim), 100 + i)
            if check_heads:
                host[name] = {h: x[h].copy() for h in check_heads}
            if element != "bf16":
                from triton_metal.buffer import bf16_values
                x = bf16_values(x)  # the same N(0,1) values, converted by write()
            layer.buffers[name].write(x)
        kern = layer.lib.kernels
        launches = [("attn_fwd", layer.fwd_args(True))]
        if backward and bwd != "split":
            launches += [("attn_bwd_preprocess", layer.pre_args()),
                         ("attn_bwd_fused", layer.fused_args())]
        elif backward:
            launches += [("attn_bwd_preprocess", layer.pre_args()),
                         ("attn_bwd_dq", layer.dq_args()),
                         ("attn_bwd_dkdv", layer.dkdv_args())]

        def step():
            for name, (grid, kinds, values) in launches:
                core.launch_async(kern[name], grid, 128, kinds, values)

        for _ in range(warmup):
            step()
        core.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            step()
        core.synchronize()
        wall_ms = (time.perf_counter() - t0) * 1e3 / max(steps, 1)

        per_kernel = {}
        for name, (grid, kinds, values) in launches:
            per_kernel[name] = {
                "ms": kernel_ms(core, kern[name], grid, kinds, values, sample_ms),
                "variant": core.kernel_variant(kern[name]),
            }
        core.synchronize()
        if verifier is not None and check_heads:
            verify_attention(layer, host, check_heads, verifier, case, backward)
    finally:
        layer.free()
    return wall_ms, per_kernel


def bench_gemm(core, ops, n, warmup, sample_ms, element="bf16", layout="nn", verifier=None,
               case=None, check_rows=64):
    """n^3 GEMM on N(0,1) operands.  layout "nt": B is passed transposed
    (stride_bk = 1, the x @ W^T layout); "tn": A transposed (stride_am = 1).
    After the timing, `check_rows` sampled rows of C against fp64."""
    from triton_metal.buffer import DeviceBuffer, bf16_values
    dtype = {"bf16": "bfloat16", "f16": "float16", "f32": "float32"}[element]
    strides = {"nn": (n, 1, n, 1, n, 1), "nt": (n, 1, 1, n, n, 1), "tn": (1, n, n, 1, n, 1)}[layout]
    host = {}

    def operand(seed):
        x = normal_bf16((n, n), seed)
        host[seed] = bf16_values(x) if element == "bf16" else bf16_values(x).astype(
            np.float16 if element == "f16" else np.float32).astype(np.float32)
        return DeviceBuffer((n, n), dtype).write(x if element == "bf16" else bf16_values(x))

    a, b = operand(1), operand(2)
    c = DeviceBuffer((n, n), dtype)
    try:
        kernel = ops.library(element).kernels["matmul_kernel"]
        grid, kinds, values = ops.matmul_args(a, b, c, n, n, n, strides)
        for _ in range(warmup):
            core.launch_async(kernel, grid, 128, kinds, values)
        core.synchronize()
        ms = kernel_ms(core, kernel, grid, kinds, values, sample_ms)
        variant = core.kernel_variant(kernel)
        core.synchronize()
        if verifier is not None:
            rows = np.sort(np.random.default_rng(n).choice(n, min(check_rows, n), replace=False))
            a_rows = host[1][:, rows].T if layout == "tn" else host[1][rows]
            b_full = host[2].T if layout == "nt" else host[2]
            want = a_rows.astype(np.float64) @ b_full.astype(np.float64)
            got = np.stack([_read_rows(c, int(r), 1, n)[0] for r in rows])
            if element == "f32":
                # north_star's fp32 bar: 1e-5 relative, max|a - b| / max|b| (the
                # reference's relative_error, attention_training.py:250-252)
                verifier.add(case, "c_rows_rel", _relative(got, want), TOL_F32)
            else:
                verifier.add(case, "c_rows", _hybrid(got, want), TOL_16)
            verifier.record[case]["rows"] = len(rows)
    finally:
        for x in (a, b, c):
            x.free()
    return ms, variant


def attention_flops(batch_heads, seq, dim, causal, backward=False) -> float:
    """The reference's FLOP convention: 4*S^2*D forward, 10*S^2*D backward per
    (batch*head) (AttentionBenchmark.swift:64-68, AttentionBackwardBenchmark.swift:45-49);
    causal counts half (this build's convention)."""
    per = (10.0 if backward else 4.0) * seq * seq * dim * batch_heads
    return per / 2 if causal else per


def gemm_flops(m, n, k) -> float:
    """2*M*N*K (GEMMBenchmark.swift:449-451)."""
    return 2.0 * m * n * k


def bench_sae(core, ops, rows, model, features, warmup, sample_ms, verifier=None, case=None):
    """The fused encoder relu(x @ W_enc + b_enc) in bf16 (sae_encode_kernel);
    afterwards 64 sampled rows against fp64."""
    from triton_metal.buffer import DeviceBuffer, bf16_values
    hx, hw, hb = (normal_bf16((rows, model), 3), normal_bf16((model, features), 4),
                  normal_bf16((features,), 5))
    x = DeviceBuffer((rows, model), "bfloat16").write(hx)
    w = DeviceBuffer((model, features), "bfloat16").write(hw)
    b = DeviceBuffer((features,), "bfloat16").write(hb)
    out = DeviceBuffer((rows, features), "bfloat16")
    try:
        enc = ops.SAEEncoder("bf16")
        grid, kinds, values = enc.args(x, w, b, out, rows, model, features)
        for _ in range(warmup):
            core.launch_async(enc.kernel, grid, 128, kinds, values)
        core.synchronize()
        ms = kernel_ms(core, enc.kernel, grid, kinds, values, sample_ms)
        variant = core.kernel_variant(enc.kernel)
        core.synchronize()
        if verifier is not None:
            sel = np.sort(np.random.default_rng(rows).choice(rows, 64, replace=False))
            want = np.maximum(bf16_values(hx[sel]).astype(np.float64)
                              @ bf16_values(hw).astype(np.float64)
                              + bf16_values(hb).astype(np.float64)[None, :], 0.0)
            got = np.stack([_read_rows(out, int(r), 1, features)[0] for r in sel])
            verifier.add(case, "out_rows", _hybrid(got, want), TOL_16)
            verifier.record[case]["rows"] = len(sel)
    finally:
        for a in (x, w, b, out):
            a.free()
    return ms, variant


def bench_latency_configs(core, ops, sample_ms):
    """Configs 1 and 2, the reference's latency-bound cases, timed as a caller
    sees them.  Config 1: fp32 GEMM 256^3 on U[-1, 1] inputs, one dispatch
    (device time from HIP events, and the wall time of one synchronous
    tm_launch).  Config 2: the training loop of attention_training.py:312-329
    at B1 H2 S96 D64 fp32, scale 1/8, lr 1e-3 on 0.5*||O - W||^2: per step,
    upload Q/K/V, forward, read O, upload dO = O - W, backward, read the
    gradients, SGD on the host -- wall time per step, and the device time of
    its four dispatches."""
    from triton_metal.buffer import DeviceBuffer
    rng = np.random.default_rng(0)
    a = DeviceBuffer.from_numpy(rng.uniform(-1, 1, (256, 256)).astype(np.float32), "float32")
    b = DeviceBuffer.from_numpy(rng.uniform(-1, 1, (256, 256)).astype(np.float32), "float32")
    c = DeviceBuffer((256, 256), "float32")
    try:
        kernel = ops.library("f32").kernels["matmul_kernel"]
        grid, kinds, values = ops.matmul_args(a, b, c, 256, 256, 256)
        device_ms = kernel_ms(core, kernel, grid, kinds, values, sample_ms)
        for _ in range(20):
            core.launch(kernel, grid, 128, kinds, values)
        t0 = time.perf_counter()
        for _ in range(200):
            core.launch(kernel, grid, 128, kinds, values)
        launch_us = (time.perf_counter() - t0) / 200 * 1e6
    finally:
        for x in (a, b, c):
            x.free()
    config1 = {"device_us": round(device_ms * 1e3, 2), "launch_us": round(launch_us, 2),
               "tflops": round(gemm_flops(256, 256, 256) / (device_ms * 1e-3) / 1e12, 3),
               "variant": core.kernel_variant(kernel)}

    q, k, v, w = (rng.standard_normal((2, 96, 64), dtype=np.float32) * np.float32(0.1)
                  for _ in range(4))
    layer = ops.AttentionLayer(2, 96, 64, "f32", scale=1 / 8)
    try:
        def train_step(q, k, v):
            o, _ = layer.forward(q, k, v)
            d_out = o - w
            dq, dk, dv = layer.backward(d_out)
            return q - 1e-3 * dq, k - 1e-3 * dk, v - 1e-3 * dv
        for _ in range(2):
            q, k, v = train_step(q, k, v)
        t0 = time.perf_counter()
        for _ in range(8):
            q, k, v = train_step(q, k, v)
        step_ms = (time.perf_counter() - t0) / 8 * 1e3
    finally:
        layer.free()
    _, kernels = bench_attention(core, ops, 1, 2, 96, 64, False, 0, 2, sample_ms, element="f32")
    config2 = {"step_ms": round(step_ms, 4),
               "device_us": round(sum(r["ms"] for r in kernels.values()) * 1e3, 2),
               "dispatches_per_step": 4}
    return config1, config2


def cpu_baseline(target_seconds):
    """The oracle's float32 BLAS restatement of the reference's attention forward
    and backward (oracle.reference.attention_head_causal_blocked_f32;
    attention_training.py:170-187 with the causal mask, by blocks of 512 query
    rows over the keys they can see), one (batch, head) of config 5 at a time
    (S=4096, D=128).  The reference's timing method (GEMMBenchmark.swift:
    250-277): one warm-up head, then 3 samples of about target_seconds / 3 each,
    the median sample's rate reported.  TFLOP/s credited with the causal half
    of the reference's FLOPs, as the GPU figure is; the blocked form executes
    36/64 of the full square, stated in `sample`."""
    from oracle import reference as R  # the CPU baseline is the oracle, timed

    seq, dim, block = 4096, 128, 512
    scale = np.float32(1 / math.sqrt(dim))
    rng = np.random.default_rng(0)
    q, k, v, d_out = (rng.standard_normal((seq, dim), dtype=np.float32) for _ in range(4))

    def one_head():
        return R.attention_head_causal_blocked_f32(q, k, v, d_out, scale, block=block)

    one_head()  # warm-up: BLAS thread pool, page faults of the work arrays
    samples = []
    for _ in range(3):
        heads = 0
        t0 = time.perf_counter()
        while True:
            one_head()
            heads += 1
            elapsed = time.perf_counter() - t0
            if elapsed >= target_seconds / 3 or heads >= 512:
                break
        flops = attention_flops(heads, seq, dim, True) + attention_flops(heads, seq, dim, True,
                                                                         backward=True)
        samples.append((flops / elapsed / 1e12, heads, elapsed))
    samples.sort()
    rate, heads, elapsed = samples[1]
    host_cpus = os.cpu_count()
    blas_threads, blas_library = None, None
    try:
        from threadpoolctl import threadpool_info
        info = [x for x in threadpool_info() if x.get("user_api") == "blas"]
        if info:
            blas_threads = int(info[0]["num_threads"])
            blas_library = info[0].get("internal_api")
    except Exception:
        pass
    nb = seq // block
    executed = nb * (nb + 1) // 2 / (nb * nb)
    return {
        "value": round(rate, 6),
        "unit": "TFLOP/s",
        # the threads the BLAS calls ran on (the whole of the work); the host's
        # logical CPUs beside it
        "cores": blas_threads if blas_threads else host_cpus,
        "host_cpus": host_cpus,
        "blas_threads": blas_threads,
        "blas_library": blas_library,
        "kind": "port",
        "samples_tflops": [round(x[0], 6) for x in sorted(samples, key=lambda x: x[0])],
        "sample": (f"(batch,head) slices of config 5 (S4096 D128 causal) forward+backward in numpy "
                   f"fp32 BLAS by {block}-row query blocks over visible keys only ({executed:.4f} "
                   f"of the full S^2 products executed; credited with the causal half, 0.5, as "
                   f"the GPU figure); 1 warm-up head, then the median of 3 samples (this one: "
                   f"{heads} heads in {elapsed:.1f} s)"),
    }


def measured_traffic(variant):
    """HBM bytes per dispatch of `variant` from the committed rocprofv3 --pmc
    FETCH_SIZE / WRITE_SIZE summary (profiles/hbm_traffic.json, scaled by the
    calibration copy), or None when that kernel has not been profiled."""
    path = ROOT / "profiles" / "hbm_traffic.json"
    try:
        rec = json.loads(path.read_text())["kernels"].get(variant)
    except (OSError, ValueError, KeyError):
        return None
    return None if rec is None else int(rec["traffic_bytes"])


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported in this build "
              "(every GPU box has one GPU, and the kernels need no cross-GPU step: the path "
              "shards over batch*heads with no communication).", file=sys.stderr)
        sys.exit(2)

    if args.vendor:
        # before this library touches the device: torch initialises HIP itself
        print(json.dumps({"vendor": vendor_reference()}))
        return
    from triton_metal import _core as core
    from triton_metal import ops

    if not core.is_usable():
        raise SystemExit("no usable gfx950 device: " + str(core.unusable_reason()))
    if args.probes:
        import bench_probes
        print(json.dumps({"probes": bench_probes.run(), "device": core.device_name()}))
        return
    if args.profile_pass:
        global _operand_data
        _operand_data = args.operand_data
        profile_pass(core, ops)
        return
    if args.data_study:
        print(json.dumps({"data_study_ms": data_study(core, ops, args.sample_ms),
                          "device": core.device_name()}))
        return

    components = {}
    result = {}
    verifier = Verifier()
    if args.only in ("all", "fa"):
        B, H, S, D = 4, 32, 4096, 128
        wall_ms, kernels = bench_attention(core, ops, B, H, S, D, True, args.steps, args.warmup,
                                           args.sample_ms, verifier=verifier,
                                           case="fa2_bf16_config5", check_heads=(0, 45, 90, 127))
        f_fwd = attention_flops(B * H, S, D, True)
        f_bwd = attention_flops(B * H, S, D, True, backward=True)
        fwd_ms = kernels["attn_fwd"]["ms"]
        bwd_ms = sum(kernels[k]["ms"] for k in ("attn_bwd_preprocess", "attn_bwd_dq",
                                                 "attn_bwd_dkdv"))
        # Algorithmic FLOPs credited per kernel: the 5 backward GEMMs are
        # dV = P^T dO, dP = dO V^T, dK = dS^T Q, S = Q K^T (all four in dkdv)
        # and dQ = dS K (the one unique GEMM of dq): 8 and 2 S^2 D per head.
        credit = {"attn_fwd": f_fwd, "attn_bwd_dkdv": f_bwd * 0.8, "attn_bwd_dq": f_bwd * 0.2,
                  "attn_bwd_preprocess": 0.0}
        for name, rec in kernels.items():
            rec["tflops"] = credit[name] / (rec["ms"] * 1e-3) / 1e12 if credit[name] else None
            rec["ms"] = round(rec["ms"], 4)
            if rec["tflops"]:
                rec["tflops"] = round(rec["tflops"], 2)
        pre_bytes = 2 * B * H * S * D * 2 + B * H * S * 4
        kernels["attn_bwd_preprocess"]["gbs"] = round(
            pre_bytes / (kernels["attn_bwd_preprocess"]["ms"] * 1e-3) / 1e9, 1)
        value = (f_fwd + f_bwd) / (wall_ms * 1e-3) / 1e12
        components["fa2_fwd"] = {"tflops": round(f_fwd / (fwd_ms * 1e-3) / 1e12, 2),
                                 "frac_of_peak": round(f_fwd / (fwd_ms * 1e-3) / 1e12 / 2500, 4),
                                 "ms": round(fwd_ms, 4)}
        components["fa2_bwd"] = {"tflops": round(f_bwd / (bwd_ms * 1e-3) / 1e12, 2),
                                 "frac_of_peak": round(f_bwd / (bwd_ms * 1e-3) / 1e12 / 2500, 4),
                                 "ms": round(bwd_ms, 4)}
        components["fa2_kernels"] = kernels
        dominant = max((k for k in kernels if credit[k]), key=lambda k: kernels[k]["ms"])
        achieved = credit[dominant] / (kernels[dominant]["ms"] * 1e-3) / 1e12
        result.update(
            value=round(value, 3), ms_per_step=round(wall_ms, 4),
            roofline={"bound": "mfma", "kernel": kernels[dominant]["variant"],
                      "achieved": round(achieved, 2), "peak": PEAK_TFLOPS["bf16"],
                      "unit": "TFLOP/s", "frac": round(achieved / PEAK_TFLOPS["bf16"], 4),
                      "traffic": measured_traffic(kernels[dominant]["variant"])})

        # config 4: forward only, B8 H16 S1024 D64 non-causal.
        _, k4 = bench_attention(core, ops, 8, 16, 1024, 64, False, 0, args.warmup,
                                args.sample_ms, backward=False, verifier=verifier,
                                case="fa2_fwd_bf16_config4", check_heads=(0, 77, 127))
        f4 = attention_flops(8 * 16, 1024, 64, False)
        ms4 = k4["attn_fwd"]["ms"]
        components["fa2_fwd_config4"] = {"tflops": round(f4 / (ms4 * 1e-3) / 1e12, 2),
                                         "frac_of_peak": round(f4 / (ms4 * 1e-3) / 1e12 / 2500, 4),
                                         "ms": round(ms4, 4), "variant": k4["attn_fwd"]["variant"]}
        # the opt-in single-pass backward (bwd=atomic) at config 5, beside the split one
        _, ka = bench_attention(core, ops, B, H, S, D, True, 0, args.warmup, args.sample_ms,
                                bwd="atomic", verifier=verifier, case="fa2_bf16_config5_atomic",
                                check_heads=(3, 126))
        ms_a = ka["attn_bwd_preprocess"]["ms"] + ka["attn_bwd_fused"]["ms"]
        components["fa2_bwd_atomic"] = {
            "tflops": round(f_bwd / (ms_a * 1e-3) / 1e12, 2),
            "frac_of_peak": round(f_bwd / (ms_a * 1e-3) / 1e12 / 2500, 4),
            "ms": round(ms_a, 4), "fused_ms": round(ka["attn_bwd_fused"]["ms"], 4),
            "vs_split": round(bwd_ms / ms_a, 3), "variant": ka["attn_bwd_fused"]["variant"]}
        # fp16 variant of config 5 (the reference's own attention element type)
        _, k16 = bench_attention(core, ops, B, H, S, D, True, 0, args.warmup, args.sample_ms,
                                 element="f16", verifier=verifier, case="fa2_f16_config5",
                                 check_heads=(1, 100))
        ms_f = k16["attn_fwd"]["ms"]
        ms_b = sum(k16[n]["ms"] for n in ("attn_bwd_preprocess", "attn_bwd_dq", "attn_bwd_dkdv"))
        components["fa2_f16_config5"] = {
            "fwd_tflops": round(f_fwd / (ms_f * 1e-3) / 1e12, 2),
            "bwd_tflops": round(f_bwd / (ms_b * 1e-3) / 1e12, 2),
            "fwd_ms": round(ms_f, 4), "bwd_ms": round(ms_b, 4),
            "variants": [k16[n]["variant"] for n in k16]}
    if args.only in ("all", "reference"):
        # The reference's own published shapes (fp32, non-causal, Apple M1 Max figures in
        # docs/ARCHITECTURE.md:910-912, :1184-1186, :1262-1264), run on the same kernels
        # any fp32 caller reaches.
        ref = {}
        for n in (1024, 2048, 4096):
            ms, variant = bench_gemm(core, ops, n, 2, args.sample_ms, element="f32",
                                     verifier=verifier, case=f"gemm_f32_{n}")
            ref[f"gemm_f32_{n}"] = {"tflops": round(gemm_flops(n, n, n) / (ms * 1e-3) / 1e12, 2),
                                    "ms": round(ms, 4), "variant": variant}
        # fp32 at three shapes, f16 at the two the reference also publishes in f16
        # (docs/ARCHITECTURE.md:1187-1188, :1265-1266)
        for element, heads, seq in (("f32", 8, 512), ("f32", 8, 1024), ("f32", 16, 2048),
                                    ("f16", 8, 512), ("f16", 8, 1024)):
            _, kr = bench_attention(core, ops, 1, heads, seq, 64, False, 0, 2, args.sample_ms,
                                    element=element, verifier=verifier,
                                    case=f"fa2_{element}_h{heads}_s{seq}_d64", check_heads=(0, heads - 1))
            ms_f = kr["attn_fwd"]["ms"]
            ms_b = sum(kr[k]["ms"] for k in ("attn_bwd_preprocess", "attn_bwd_dq", "attn_bwd_dkdv"))
            ref[f"fa2_{element}_h{heads}_s{seq}_d64"] = {
                "fwd_tflops": round(attention_flops(heads, seq, 64, False) / (ms_f * 1e-3) / 1e12, 3),
                "bwd_tflops": round(attention_flops(heads, seq, 64, False, backward=True)
                                    / (ms_b * 1e-3) / 1e12, 3),
                "fwd_ms": round(ms_f, 4), "bwd_ms": round(ms_b, 4)}
        config1, config2 = bench_latency_configs(core, ops, args.sample_ms)
        ref["config1_gemm_f32_256"] = config1
        ref["config2_training_step_f32"] = config2
        components["reference_shapes_f32"] = ref
    if args.only in ("all", "gemm"):
        n = 8192
        ms, variant = bench_gemm(core, ops, n, args.warmup, args.sample_ms, verifier=verifier,
                                 case="gemm_bf16_8192_config3")
        tf = gemm_flops(n, n, n) / (ms * 1e-3) / 1e12
        components["gemm_bf16_8192"] = {"tflops": round(tf, 2),
                                        "frac_of_peak": round(tf / 2500, 4),
                                        "ms": round(ms, 4), "variant": variant}
        ms16, variant16 = bench_gemm(core, ops, n, args.warmup, args.sample_ms, element="f16",
                                     verifier=verifier, case="gemm_f16_8192")
        tf16 = gemm_flops(n, n, n) / (ms16 * 1e-3) / 1e12
        components["gemm_f16_8192"] = {"tflops": round(tf16, 2),
                                       "frac_of_peak": round(tf16 / 2500, 4),
                                       "ms": round(ms16, 4), "variant": variant16}
        # Other sizes and operand layouts on the same kernels (tile choice by size;
        # B or A passed transposed).
        more = {}
        for n2, layout in ((1024, "nn"), (2048, "nn"), (4096, "nn"), (8192, "nt"), (8192, "tn")):
            ms2, variant2 = bench_gemm(core, ops, n2, 2, args.sample_ms, layout=layout,
                                       verifier=verifier, case=f"gemm_bf16_{layout}_{n2}")
            more[f"{layout}_{n2}"] = {"tflops": round(gemm_flops(n2, n2, n2) / (ms2 * 1e-3) / 1e12, 2),
                                      "ms": round(ms2, 4), "variant": variant2}
        components["gemm_bf16_sizes_and_layouts"] = more
        # The fused SAE encoder at an 8x dictionary over 8192 tokens of width 2048.
        rows, model, features = 8192, 2048, 16384
        ms_s, variant_s = bench_sae(core, ops, rows, model, features, args.warmup,
                                    args.sample_ms, verifier=verifier, case="sae_encode_bf16")
        tf_s = gemm_flops(rows, features, model) / (ms_s * 1e-3) / 1e12
        components["sae_encode_bf16_8192x2048x16384"] = {
            "tflops": round(tf_s, 2), "frac_of_peak": round(tf_s / 2500, 4),
            "ms": round(ms_s, 4), "variant": variant_s}
        if args.only == "gemm":
            result.update(value=round(tf, 3), ms_per_step=round(ms, 4),
                          roofline={"bound": "mfma", "kernel": variant, "achieved": round(tf, 2),
                                    "peak": 2500.0, "unit": "TFLOP/s",
                                    "frac": round(tf / 2500, 4),
                                    "traffic": measured_traffic(variant)})

    if verifier.failures:
        print("bench.py: results failed verification, no figure reported:\n  "
              + "\n  ".join(verifier.failures), file=sys.stderr, flush=True)
        print(json.dumps({"verified": {"ok": False, "failures": verifier.failures,
                                       "cases": verifier.record}}), file=sys.stderr, flush=True)
        sys.exit(1)
    line = {
        "metric": METRIC,
        "value": result.get("value"),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": result.get("ms_per_step"),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic N(0,1) bf16 inputs, resident in HBM",
        "config": {"workload": "fa2_fwd_bwd_bf16_causal (config 5)", "batch": 4,
                   "heads": 32, "seq_len": 4096, "head_dim": 128, "causal": True,
                   "parallelism": "none (1 GPU)"} if args.only != "gemm" else
                  {"workload": "gemm_bf16_8192 (config 3)", "m": 8192, "n": 8192,
                   "k": 8192, "parallelism": "none (1 GPU)"},
        "roofline": result.get("roofline"),
        "cpu_baseline": None if args.no_cpu_baseline else cpu_baseline(args.cpu_seconds),
        "verified": {"ok": not verifier.failures, "cases": verifier.record},
        "components": components,
        "device": core.device_name(),
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
