"""Device probes: the gfx950 rates the kernel designs are built on.

Each probe is a small HIP kernel compiled at run time (tm_compile_msl with HIP
source) and timed with tm_launch_timed.  Rates are reported per CU per clock at
the nominal 2.4 GHz and as totals, so they compare directly with the MI355X
published peaks (256 CUs; dense bf16 MFMA 2.5 PFLOP/s = 4096 FLOP/clk/CU).

  mfma_16x16x32 / mfma_32x32x16   back-to-back bf16 MFMAs, 4 independent chains
  gemm_wave_mfma_16x16x32 / _32x32x16
                                  the MFMA stream of the bf16 GEMM's wave (a
                                  128 x 64 sub-tile, 64 k per step, 8 waves =
                                  2 per SIMD) with operand bits changing every
                                  step, no memory: the issue ceiling a GEMM of
                                  that shape can reach
  exp2                            v_exp_f32 throughput
  lds_b128 / lds_tr_b64           ds_read_b128 and ds_read_b64_tr_b16 bytes, on
                                  conflict-free addresses
  atomic_add_f32 / rmw_f32        fp32 atomic adds vs plain read-add-write on
                                  coalesced [32 x 128] tiles (the dQ tile of a
                                  fused backward)
  atomic_dq_config5               the dQ atomic adds alone of a fused backward
                                  at config 5, in their real pattern

Run: python bench.py --probes
"""

import json

from triton_metal import _core

CUS = 256
CLOCK_HZ = 2.4e9

_SOURCE = r'''
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

__device__ unsigned lds_address(const void *p) {
  return (unsigned)(size_t)((__attribute__((address_space(3))) const char *)p);
}

extern "C" __global__ __launch_bounds__(256) void probe_mfma16(unsigned *out, int iters) {
  bf16x8 a, b;
  for (int i = 0; i < 8; ++i) { a[i] = (__bf16)(threadIdx.x * 0.001f); b[i] = (__bf16)(i * 0.01f); }
  f32x4 c0 = {0, 0, 0, 0}, c1 = c0, c2 = c0, c3 = c0;
  for (int it = 0; it < iters; ++it) {
    c0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c0, 0, 0, 0);
    c1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c1, 0, 0, 0);
    c2 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c2, 0, 0, 0);
    c3 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c3, 0, 0, 0);
  }
  f32x4 s = c0 + c1 + c2 + c3;
  if (s[0] == 1234.5f) out[0] = 1;
}

extern "C" __global__ __launch_bounds__(256) void probe_mfma32(unsigned *out, int iters) {
  bf16x8 a, b;
  for (int i = 0; i < 8; ++i) { a[i] = (__bf16)(threadIdx.x * 0.001f); b[i] = (__bf16)(i * 0.01f); }
  f32x16 c0 = {}, c1 = {}, c2 = {}, c3 = {};
  for (int it = 0; it < iters; it += 2) {
    c0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c0, 0, 0, 0);
    c1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c1, 0, 0, 0);
    c2 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c2, 0, 0, 0);
    c3 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c3, 0, 0, 0);
  }
  f32x16 s = c0 + c1 + c2 + c3;
  if (s[0] == 1234.5f) out[0] = 1;
}

extern "C" __global__ __launch_bounds__(256) void probe_exp2(unsigned *out, int iters) {
  float x0 = threadIdx.x * 1e-6f, x1 = x0 + 1e-7f, x2 = x0 + 2e-7f, x3 = x0 + 3e-7f;
  for (int it = 0; it < iters; ++it) {
    x0 = __builtin_amdgcn_exp2f(x0); x1 = __builtin_amdgcn_exp2f(x1);
    x2 = __builtin_amdgcn_exp2f(x2); x3 = __builtin_amdgcn_exp2f(x3);
  }
  if (x0 + x1 + x2 + x3 == 1234.5f) out[0] = 1;
}

extern "C" __global__ __launch_bounds__(256) void probe_lds_b128(unsigned *out, int iters) {
  __shared__ __attribute__((aligned(16))) char lds[65536];
  for (int i = threadIdx.x; i < 16384; i += 256) ((unsigned *)lds)[i] = i;
  __syncthreads();
  const unsigned base = lds_address(lds) + (threadIdx.x & 63) * 16 + (threadIdx.x >> 6) * 1024;
  u32x4 acc = {0, 0, 0, 0};
  for (int it = 0; it < iters; ++it) {
    u32x4 r0, r1, r2, r3, r4, r5, r6, r7;
    asm volatile(
        "ds_read_b128 %0, %8\n ds_read_b128 %1, %8 offset:4096\n"
        "ds_read_b128 %2, %8 offset:8192\n ds_read_b128 %3, %8 offset:12288\n"
        "ds_read_b128 %4, %8 offset:16384\n ds_read_b128 %5, %8 offset:20480\n"
        "ds_read_b128 %6, %8 offset:24576\n ds_read_b128 %7, %8 offset:28672\n"
        "s_waitcnt lgkmcnt(0)"
        : "=v"(r0), "=v"(r1), "=v"(r2), "=v"(r3), "=v"(r4), "=v"(r5), "=v"(r6), "=v"(r7)
        : "v"(base));
    acc ^= r0 ^ r1 ^ r2 ^ r3 ^ r4 ^ r5 ^ r6 ^ r7;
  }
  if (acc[0] == 0x12345678u) out[0] = acc[1];
}

extern "C" __global__ __launch_bounds__(256) void probe_lds_tr(unsigned *out, int iters) {
  __shared__ __attribute__((aligned(16))) char lds[65536];
  for (int i = threadIdx.x; i < 16384; i += 256) ((unsigned *)lds)[i] = i;
  __syncthreads();
  /* 16-lane groups read 4 rows x 32 bytes; rows and groups offset so that the
   * 64 lanes cover distinct banks */
  const int l = threadIdx.x & 63;
  const unsigned base = lds_address(lds) + ((l >> 2) & 3) * 544 + (l & 3) * 8 + (l >> 4) * 2176 +
                        (threadIdx.x >> 6) * 8192;
  u32x2 acc = {0, 0};
  for (int it = 0; it < iters; ++it) {
    u32x2 r0, r1, r2, r3, r4, r5, r6, r7;
    asm volatile(
        "ds_read_b64_tr_b16 %0, %8\n ds_read_b64_tr_b16 %1, %8 offset:32\n"
        "ds_read_b64_tr_b16 %2, %8 offset:64\n ds_read_b64_tr_b16 %3, %8 offset:96\n"
        "ds_read_b64_tr_b16 %4, %8 offset:128\n ds_read_b64_tr_b16 %5, %8 offset:160\n"
        "ds_read_b64_tr_b16 %6, %8 offset:192\n ds_read_b64_tr_b16 %7, %8 offset:224\n"
        "s_waitcnt lgkmcnt(0)"
        : "=v"(r0), "=v"(r1), "=v"(r2), "=v"(r3), "=v"(r4), "=v"(r5), "=v"(r6), "=v"(r7)
        : "v"(base));
    acc ^= r0 ^ r1 ^ r2 ^ r3 ^ r4 ^ r5 ^ r6 ^ r7;
  }
  if (acc[0] == 0x12345678u) out[0] = acc[1];
}

/* The GEMM wave's MFMA stream: 32 accumulators of 16 x 16 (or 8 of 32 x 32)
 * for a 128 x 64 sub-tile, 64 k per iteration; operands from registers,
 * stepped by an add each iteration so their bits (and the power drawn) move
 * as with real data. */
extern "C" __global__ __launch_bounds__(512) void probe_gemm_wave16(float *out, int iters) {
  const unsigned seed = 12345u + threadIdx.x;
  f32x4 acc[8][4] = {};
  u32x4 a[8], b[4];
  for (int i = 0; i < 8; ++i) a[i] = (u32x4){seed * (i + 1), seed + i, seed ^ 0x5a5a1234u, seed * 7u + i};
  for (int j = 0; j < 4; ++j) b[j] = (u32x4){seed * (j + 3), seed - j, seed ^ 0x3c3c4321u, seed * 5u + j};
  for (int it = 0; it < iters; ++it)
    for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
      for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, b[j]),
                                                              __builtin_bit_cast(bf16x8, a[i]), acc[i][j], 0, 0, 0);
#pragma unroll
      for (int i = 0; i < 8; ++i) a[i] += 0x9e3779b9u;
#pragma unroll
      for (int j = 0; j < 4; ++j) b[j] += 0x7f4a7c15u;
    }
  float s = 0;
  for (int i = 0; i < 8; ++i)
    for (int j = 0; j < 4; ++j) s += acc[i][j][0] + acc[i][j][3];
  if (s == 1234.5f) out[0] = 1;
}
extern "C" __global__ __launch_bounds__(512) void probe_gemm_wave32(float *out, int iters) {
  const unsigned seed = 12345u + threadIdx.x;
  f32x16 acc[4][2] = {};
  u32x4 a[4], b[2];
  for (int i = 0; i < 4; ++i) a[i] = (u32x4){seed * (i + 1), seed + i, seed ^ 0x5a5a1234u, seed * 7u + i};
  for (int j = 0; j < 2; ++j) b[j] = (u32x4){seed * (j + 3), seed - j, seed ^ 0x3c3c4321u, seed * 5u + j};
  for (int it = 0; it < iters; ++it)
    for (int ks = 0; ks < 4; ++ks) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, b[j]),
                                                              __builtin_bit_cast(bf16x8, a[i]), acc[i][j], 0, 0, 0);
#pragma unroll
      for (int i = 0; i < 4; ++i) a[i] += 0x9e3779b9u;
#pragma unroll
      for (int j = 0; j < 2; ++j) b[j] += 0x7f4a7c15u;
    }
  float s = 0;
  for (int i = 0; i < 4; ++i)
    for (int j = 0; j < 2; ++j) s += acc[i][j][0] + acc[i][j][15];
  if (s == 1234.5f) out[0] = 1;
}

/* Each workgroup adds into one [32 x 128] fp32 tile of a 64 MiB buffer `iters`
 * times: with atomics, or as a plain read-add-write. */
extern "C" __global__ __launch_bounds__(256) void probe_atomic(float *acc, int iters) {
  const long tile = (long)(blockIdx.x % 4096) * 4096;
  for (int r = 0; r < iters; ++r)
    for (int e = threadIdx.x; e < 4096; e += 256)
      __hip_atomic_fetch_add(acc + tile + e, 1.0f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
/* The dQ traffic of a fused single-kernel backward at config 5 (B4 H32
 * S4096 D128 causal, 128 keys per workgroup, 32-query steps): workgroup
 * (bh, kb) adds one [32 x 128] fp32 tile into dQ for every query block from
 * its first key to the end -- 1.107e9 atomic adds in all, nothing else. */
extern "C" __global__ __launch_bounds__(256) void probe_dq_atomics(float *dq, int seq) {
  const int nkb = seq / 128;
  const int bh = blockIdx.x / nkb, kb = blockIdx.x % nkb;
  float *head = dq + (long)bh * seq * 128;
  for (int q0 = kb * 128; q0 < seq; q0 += 32)
    for (int e = threadIdx.x; e < 32 * 128; e += 256)
      __hip_atomic_fetch_add(head + (long)q0 * 128 + e, 1.0f, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
}
extern "C" __global__ __launch_bounds__(256) void probe_rmw(float *acc, int iters) {
  const long tile = (long)(blockIdx.x % 4096) * 4096;
  for (int r = 0; r < iters; ++r)
    for (int e = threadIdx.x; e < 4096; e += 256) acc[tile + e] += 1.0f;
}
'''

#: name -> (kernel, work units per workgroup per iteration, unit)
_PROBES = {
    "mfma_16x16x32_bf16": ("probe_mfma16", 4 * 4 * 2 * 16 * 16 * 32, "FLOP"),
    "mfma_32x32x16_bf16": ("probe_mfma32", 4 * 4 * 2 * 32 * 32 * 16 / 2, "FLOP"),
    "exp2_f32": ("probe_exp2", 4 * 256, "exp"),
    "lds_b128": ("probe_lds_b128", 8 * 16 * 256, "B"),
    "lds_tr_b64": ("probe_lds_tr", 8 * 8 * 256, "B"),
    "atomic_add_f32": ("probe_atomic", 4096, "add"),
    "rmw_f32": ("probe_rmw", 4096, "add"),
}


def run(iters=4096, workgroups=CUS * 16):
    """Time every probe; returns {name: {ms, per_cu_clk, total_per_s, unit}}."""
    lib = _core.compile_msl(_SOURCE)
    scratch = _core.alloc_buffer(4096 * 4096 * 4)
    results = {}
    try:
        for name, (kernel_name, per_iter, unit) in _PROBES.items():
            kernel = _core.load_kernel(lib, kernel_name)
            n_iter = 8 if kernel_name in ("probe_atomic", "probe_rmw") else iters
            args = ([_core.ARG_BUFFER, _core.ARG_I32], [scratch, n_iter])
            grid = (workgroups, 1, 1)
            _core.launch(kernel, grid, 256, *args)
            ms = _core.launch_timed(kernel, grid, 256, args[0], args[1], 5) / 5
            total = workgroups * n_iter * per_iter / (ms * 1e-3)
            results[name] = {"ms": round(ms, 4), "unit": unit,
                             "total_per_s": float(f"{total:.4g}"),
                             "per_cu_clk": round(total / CUS / CLOCK_HZ, 2)}
            _core.release_kernel(kernel)
        results.update(_gemm_wave_mfma(lib))
        results["atomic_dq_config5"] = _dq_atomics(lib)
    finally:
        _core.free_buffer(scratch)
        _core.release_library(lib)
    return results


def _gemm_wave_mfma(lib, iters=2048, workgroups=CUS * 4):
    """The GEMM wave's MFMA stream at the GEMM's occupancy: 512-thread
    workgroups, 8 waves of 128 x 64 x 64 per iteration."""
    out = {}
    scratch = _core.alloc_buffer(4096)
    try:
        for name, kernel_name in (("gemm_wave_mfma_16x16x32_bf16", "probe_gemm_wave16"),
                                  ("gemm_wave_mfma_32x32x16_bf16", "probe_gemm_wave32")):
            kernel = _core.load_kernel(lib, kernel_name)
            grid = (workgroups, 1, 1)
            args = ([_core.ARG_BUFFER, _core.ARG_I32], [scratch, iters])
            _core.launch(kernel, grid, 512, *args)
            ms = _core.launch_timed(kernel, grid, 512, args[0], args[1], 5) / 5
            total = workgroups * iters * 8 * 128 * 64 * 64 * 2 / (ms * 1e-3)
            out[name] = {"ms": round(ms, 4), "unit": "FLOP", "total_per_s": float(f"{total:.4g}"),
                         "per_cu_clk": round(total / CUS / CLOCK_HZ, 2)}
            _core.release_kernel(kernel)
    finally:
        _core.free_buffer(scratch)
    return out


def _dq_atomics(lib, heads=128, seq=4096):
    """Time the dQ atomics alone of a fused backward at config 5: the lower
    bound such a kernel would pay on top of its dK/dV work."""
    kernel = _core.load_kernel(lib, "probe_dq_atomics")
    dq = _core.alloc_buffer(heads * seq * 128 * 4)
    try:
        grid = (heads * (seq // 128), 1, 1)
        args = ([_core.ARG_BUFFER, _core.ARG_I32], [dq, seq])
        _core.launch(kernel, grid, 256, *args)
        ms = _core.launch_timed(kernel, grid, 256, args[0], args[1], 3) / 3
        adds = heads * 128 * sum(seq - 128 * kb for kb in range(seq // 128))
    finally:
        _core.free_buffer(dq)
        _core.release_kernel(kernel)
    return {"ms": round(ms, 4), "unit": "add", "adds": adds,
            "total_per_s": float(f"{adds / (ms * 1e-3):.4g}")}


if __name__ == "__main__":
    print(json.dumps(run(), indent=1))
