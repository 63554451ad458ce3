/*
 * Specialised gfx950 GEMM for 16-bit element types: C = A @ B with A [M, K],
 * B [K, N], C [M, N] row-major (unit inner stride, 16-byte aligned rows),
 * M and N multiples of 256, K a multiple of 64; f32 accumulation, output
 * rounded to the element type (the reference's matmul_kernel semantics,
 * Sources/TritonMetalBench/GEMMKernel.swift:28-174).
 *
 * Tiling: one 512-thread workgroup (8 waves, 2 x 4) computes a 256 x 256 tile
 * of C; each wave a 128 x 64 sub-tile on v_mfma_f32_16x16x32_{bf16,f16}
 * (8 x 4 accumulators of 16 x 16).  Per K step of 64:
 *   - A [256 x 64] and B [64 x 256] tiles are copied HBM -> LDS with
 *     global_load_lds_dwordx4 (issued from inline assembly, so the compiler
 *     pipelines the operand reads behind it) in their natural row-major layouts (double
 *     buffered, 128 KB of LDS), 16-byte chunks XOR-swizzled by row;
 *   - the A operand (row m, 8 consecutive k) is one ds_read_b128;
 *   - the B operand (column n, 8 consecutive k) is two ds_read_b64_tr_b16:
 *     lane i of a 16-lane group receives element (i & 3) of the 8 bytes
 *     addressed by lane 4e + (i >> 2), so lane 4e + q addresses row k0 + e,
 *     columns n0 + 4q .. +3;
 *   - the MFMA takes B as its first operand, producing C^T tiles: each lane
 *     then holds 4 consecutive columns of one row, stored as one 8-byte write.
 * The 1-D grid is remapped so each XCD owns a contiguous range of tiles,
 * walked in groups of 8 tile rows so concurrently running tiles share A and B
 * panels in that XCD's L2.
 */
#include "common.h"

template <typename T> struct GVec8;
template <> struct GVec8<bf16_t> { typedef bf16x8 type; };
template <> struct GVec8<f16_t> { typedef f16x8 type; };

typedef short gs16x4 __attribute__((ext_vector_type(4)));

TM_DEV void g_global_to_lds16(const void *src, char *lds_wave_base) {
  lds_copy16_global(src, lds_addr(lds_wave_base));
}
TM_DEV void g_wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }

TM_DEV int g_xcd_remap(int wg, int nwg) {
  const int q = nwg >> 3, r = nwg & 7;
  const int xcd = wg & 7, slot = wg >> 3;
  return (xcd < r ? xcd * (q + 1) : r * (q + 1) + (xcd - r) * q) + slot;
}

constexpr int GBM = 256, GBN = 256, GBK = 64;
constexpr int A_TILE = GBM * GBK * 2; /* 32 KB: 256 rows of 128 bytes */
constexpr int B_TILE = GBK * GBN * 2; /* 32 KB: 64 rows of 512 bytes */

/* A tile: 128-byte rows (8 chunks), read only by ds_read_b128 of 16
 * consecutive rows at one chunk: the key row & 7 gives those reads no bank
 * conflicts (SQ_LDS_BANK_CONFLICT reads 0; the key shared with the transposed
 * B reads left 40% of the LDS cycles in conflicts and ran 3% slower). */
TM_DEV int a_swz(int row) { return row & 7; }
TM_DEV int a_off(int row, int chunk) { return row * 128 + ((chunk ^ a_swz(row)) << 4); }

/* B tile: 512-byte rows (32 chunks).  A transpose read touches rows
 * k0 + 8g + {0..3} (and +4) at one chunk pair; the even key separates the
 * pairs of the 8 rows served together. */
TM_DEV int b_swz(int row) { return ((row & 3) | ((row >> 1) & 4)) << 1; }
TM_DEV int b_off(int row, int chunk) { return row * 512 + ((chunk ^ b_swz(row)) << 4); }

template <typename T>
TM_DEV void stage_a(const T *A, int64_t lda, int m0, int k0, char *tile, int wave, int lane) {
  /* 32 instructions of 8 rows each, 4 per wave */
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int t = wave * 4 + i;
    const int row = t * 8 + (lane >> 3);
    const int chunk = (lane & 7) ^ a_swz(row);
    g_global_to_lds16(A + (int64_t)(m0 + row) * lda + k0 + chunk * 8, tile + t * 1024);
  }
}

template <typename T>
TM_DEV void stage_b(const T *B, int64_t ldb, int k0, int n0, char *tile, int wave, int lane) {
  /* 32 instructions of 2 rows each, 4 per wave */
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int t = wave * 4 + i;
    const int row = t * 2 + (lane >> 5);
    const int chunk = (lane & 31) ^ b_swz(row);
    g_global_to_lds16(B + (int64_t)(k0 + row) * ldb + n0 + chunk * 8, tile + t * 1024);
  }
}

/* B operand for k rows kbase + 8g .. +7 of column n0 + c. */
TM_DEV u32x4 read_b_operand(const char *tile, int kbase, int n0, int g, int c) {
  const int n = n0 + 4 * (c & 3);
  const int chunk = n >> 3, half = (n >> 2) & 1;
  const int ra = kbase + 8 * g + (c >> 2), rb = ra + 4;
  const gs16x4 a = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) gs16x4 *)(tile + b_off(ra, chunk) + (half << 3)));
  const gs16x4 b = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) gs16x4 *)(tile + b_off(rb, chunk) + (half << 3)));
  const u32x2 ua = __builtin_bit_cast(u32x2, a), ub = __builtin_bit_cast(u32x2, b);
  return (u32x4){ua[0], ua[1], ub[0], ub[1]};
}

template <typename T>
TM_DEV uint32_t g_pack2(float lo, float hi) {
  typedef float f2 __attribute__((ext_vector_type(2)));
  typedef T t2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f2){lo, hi}, t2));
}

template <typename T, int EPI>
TM_DEV void gemm_fast(const TmGemmArgs &p) {
  typedef typename GVec8<T>::type v8;
  __shared__ __align__(1024) char lds_a0[A_TILE];
  __shared__ __align__(1024) char lds_b0[B_TILE];
  __shared__ __align__(1024) char lds_a1[A_TILE];
  __shared__ __align__(1024) char lds_b1[B_TILE];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, c = lane & 15;
  const int wm = wave >> 2, wn = wave & 3; /* 2 x 4 waves */

  const int mt = p.m / GBM, nt = p.n / GBN;
  const int logical = g_xcd_remap(blockIdx.x, gridDim.x);
  constexpr int GROUP = 8;
  const int per_group = GROUP * nt;
  const int group = logical / per_group;
  const int first_m = group * GROUP;
  const int gm = min(mt - first_m, GROUP);
  const int in_group = logical - group * per_group;
  const int tile_m = first_m + in_group % gm;
  const int tile_n = in_group / gm;
  const int m0 = tile_m * GBM, n0 = tile_n * GBN;

  const T *A = (const T *)p.a;
  const T *B = (const T *)p.b;
  T *C = (T *)p.c;
  const int64_t lda = p.sam, ldb = p.sbk, ldc = p.scm;

  f32x4 acc[8][4];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = (f32x4){0.f, 0.f, 0.f, 0.f};

  const int ksteps = p.k / GBK;
  stage_a<T>(A, lda, m0, 0, lds_a0, wave, lane);
  stage_b<T>(B, ldb, 0, n0, lds_b0, wave, lane);
  g_wait_vmem();
  __syncthreads();

  auto step = [&](const char *ca, const char *cb, char *na, char *nb, int kb) {
    if (kb + 1 < ksteps) {
      stage_a<T>(A, lda, m0, (kb + 1) * GBK, na, wave, lane);
      stage_b<T>(B, ldb, (kb + 1) * GBK, n0, nb, wave, lane);
    }
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      v8 bf[4];
#pragma unroll
      for (int j = 0; j < 4; ++j)
        bf[j] = __builtin_bit_cast(v8, read_b_operand(cb, ks * 32, wn * 64 + j * 16, g, c));
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const v8 af = __builtin_bit_cast(
            v8, *(const u32x4 *)(ca + a_off(wm * 128 + i * 16 + c, ks * 4 + g)));
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = mfma_16x16x32(bf[j], af, acc[i][j]);
      }
    }
    g_wait_vmem();
    __syncthreads();
  };

  for (int kb = 0; kb < ksteps; kb += 2) {
    step(lds_a0, lds_b0, lds_a1, lds_b1, kb);
    if (kb + 1 < ksteps) step(lds_a1, lds_b1, lds_a0, lds_b0, kb + 1);
  }

  /* acc[i][j] is the C^T tile: lane holds row m0 + wm*128 + i*16 + c,
   * columns n0 + wn*64 + j*16 + 4g .. +3 */
  /* The bias of the wave's 16 columns, loaded once before any store (the
   * compiler cannot move the loads across stores to C that might alias). */
  float bias[4][4];
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int r = 0; r < 4; ++r)
      bias[j][r] = EPI == EPI_BIAS_RELU
                       ? to_f32(((const T *)p.bias)[n0 + wn * 64 + j * 16 + 4 * g + r])
                       : 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int m = m0 + wm * 128 + i * 16 + c;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int n = n0 + wn * 64 + j * 16 + 4 * g;
      float v[4];
#pragma unroll
      for (int r = 0; r < 4; ++r)
        v[r] = EPI == EPI_BIAS_RELU ? fmaxf(acc[i][j][r] + bias[j][r], 0.f) : acc[i][j][r];
      u32x2 w;
      w[0] = g_pack2<T>(v[0], v[1]);
      w[1] = g_pack2<T>(v[2], v[3]);
      *(u32x2 *)(C + (int64_t)m * ldc + n) = w;
    }
  }
}

#define TM_GEMM_FAST(T, TN)                                                                \
  extern "C" __global__ __launch_bounds__(512) void tm_gemm_fast_##TN(TmGemmArgs p) {        \
    gemm_fast<T, EPI_NONE>(p);                                                               \
  }                                                                                          \
  extern "C" __global__ __launch_bounds__(512) void tm_sae_fast_##TN(TmGemmArgs p) {         \
    gemm_fast<T, EPI_BIAS_RELU>(p);                                                          \
  }
TM_GEMM_FAST(bf16_t, bf16)
TM_GEMM_FAST(f16_t, f16)
