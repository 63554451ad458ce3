/*
 * Specialised gfx950 GEMM for fp32, the reference's own element type:
 * C = A @ B with A [M, K], B [K, N], C [M, N] row-major (unit inner stride,
 * 16-byte aligned rows, lda >= K, ldb >= N), M and N multiples of 128 and K a
 * multiple of 32; fp32 products and accumulation on v_mfma_f32_16x16x4_f32
 * (the reference's matmul_kernel semantics,
 * Sources/TritonMetalBench/GEMMKernel.swift:28-174, in fp32).
 *
 * Tiling: one 256-thread workgroup (4 waves, 2 x 2) computes a 128 x 128
 * tile of C; each wave a 64 x 64 sub-tile (4 x 4 accumulators of 16 x 16).
 * Per K step of 32:
 *   - A [128 x 32] and B [32 x 128] tiles are copied HBM -> LDS with
 *     global_load_lds_dwordx4 in their row-major layouts (double buffered,
 *     64 KB of LDS, two workgroups per CU), 16-byte chunks XOR-swizzled by row;
 *   - the MFMA's k index is permuted within each 16-wide k chunk: lane
 *     (g = l / 16, c = l % 16) feeds k = 4g + t to the t-th of four MFMAs, so
 *     one ds_read_b128 of A row c supplies all four, and B's element
 *     (k = 4g + t, column c) is one ds_read_b32;
 *   - B is the MFMA's first operand, producing C^T tiles: each lane holds 4
 *     consecutive columns of one row of C, stored as one 16-byte write.
 * Either operand may instead be stored transposed (tm_gemm_fast_nt_f32: B
 * with unit stride along K; tm_gemm_fast_tn_f32: A with unit stride along
 * M); its tile then has the other operand's layout and reads.
 */
#include "common.h"

namespace {

constexpr int FK = 32;

/* A tile: 128-byte rows, read by ds_read_b128 of 16 consecutive rows at one
 * chunk: the key row & 7 spreads them over the banks. */
TM_DEV int fa_off(int row, int chunk) { return row * 128 + ((chunk ^ (row & 7)) << 4); }

/* B tile: FT-float rows (512 or 256 bytes); a wave reads rows 4g + t
 * (g = 0..3) at 16 consecutive floats (four chunks): the key
 * 4 ((row >> 2) & 3) moves the four rows to different quarters of the
 * 256-byte bank row. */
template <int FT>
TM_DEV int fb_off(int row, int chunk) { return row * (4 * FT) + ((chunk ^ (((row >> 2) & 3) << 2)) << 4); }

TM_DEV void f_wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }

TM_DEV int f_xcd_remap(int wg, int nwg) {
  const int q = nwg >> 3, r = nwg & 7;
  const int xcd = wg & 7, slot = wg >> 3;
  return (xcd < r ? xcd * (q + 1) : r * (q + 1) + (xcd - r) * q) + slot;
}

/* A [FT x 32] tile at (m0, k0): FT / 8 instructions of 8 rows over 4 waves */
template <int FT>
TM_DEV void f_stage_a(const float *a, int64_t lda, int k0, char *tile, int wave, int lane) {
  constexpr int PER = FT / 32;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int t = wave * PER + i;
    const int row = t * 8 + (lane >> 3);
    const int chunk = (lane & 7) ^ (row & 7);
    lds_copy16_global(a + (int64_t)row * lda + k0 + chunk * 4, lds_addr(tile + t * 1024));
  }
}

/* B [32 x FT] tile at (k0, n0): FT / 8 instructions of 256 / FT rows over 4 waves */
template <int FT>
TM_DEV void f_stage_b(const float *b, int64_t ldb, int k0, char *tile, int wave, int lane) {
  constexpr int PER = FT / 32, RPI = 256 / FT, CPR = FT / 4;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int t = wave * PER + i;
    const int row = t * RPI + lane / CPR;
    const int chunk = (lane % CPR) ^ (((row >> 2) & 3) << 2);
    lds_copy16_global(b + (int64_t)(k0 + row) * ldb + chunk * 4, lds_addr(tile + t * 1024));
  }
}

/* AT / BT: A (B) stored transposed -- element (m, k) at k * lda + m, or
 * (k, n) at n * ldb + k.  A transposed operand's tile takes the other
 * operand's layout and reads: A^T is staged and read like B, B^T like A. */
/* KG: groups of 4 waves splitting the K loop inside the workgroup (1, 2 or
 * 4; 256 KG threads).  Group h computes k-steps h, h + KG, ... from its own
 * double-buffered tiles; at the end groups 1 .. KG-1 leave their
 * accumulators in LDS and group 0 adds them in order and stores.  For grids
 * with about one workgroup per CU, this puts KG waves on every SIMD instead
 * of one. */
template <int EPI, bool AT = false, bool BT = false, int FT = 128, int KG = 1>
TM_DEV void gemm_f32(const TmGemmArgs &p) {
  static_assert(!(AT && BT), "one transposed operand");
  static_assert(FT == 128 || FT == 64, "tile");
  static_assert(KG == 1 || KG == 2 || KG == 4, "K groups");
  constexpr int FA_TILE = FT * FK * 4; /* FT rows of 128 bytes */
  constexpr int FB_TILE = FK * FT * 4; /* 32 rows of 4 FT bytes */
  constexpr int WT = FT / 2, NI = WT / 16; /* a wave's sub-tile: WT x WT, NI x NI of 16 x 16 */
  constexpr int GROUP_BYTES = 2 * (FA_TILE + FB_TILE);
  static_assert(KG == 1 || GROUP_BYTES >= FT * FT * 4, "a group's tiles hold its accumulators");
  __shared__ __align__(1024) char lds[KG * GROUP_BYTES];

  const int tid = threadIdx.x, lane = tid & 63;
  const int kgrp = tid >> 8, wave = (tid >> 6) & 3; /* K group, wave within it */
  const int g = lane >> 4, c = lane & 15;
  char *const lds_a0 = lds + kgrp * GROUP_BYTES;
  char *const lds_b0 = lds_a0 + FA_TILE;
  char *const lds_a1 = lds_b0 + FB_TILE;
  char *const lds_b1 = lds_a1 + FA_TILE;
  const int wm = wave >> 1, wn = wave & 1; /* 2 x 2 waves */

  /* tile order: XCD-contiguous ranges, walked in groups of 8 tile rows */
  const int mt = p.m / FT, nt = p.n / FT;
  const int logical = f_xcd_remap(blockIdx.x, gridDim.x);
  constexpr int GROUP = 8;
  const int per_group = GROUP * nt;
  const int group = logical / per_group;
  const int first_m = group * GROUP;
  const int gm = min(mt - first_m, GROUP);
  const int in_group = logical - group * per_group;
  const int m0 = (first_m + in_group % gm) * FT, n0 = (in_group / gm) * FT;

  const int64_t lda = AT ? p.sak : p.sam, ldb = BT ? p.sbn : p.sbk, ldc = p.scm;
  const float *A = (const float *)p.a + (AT ? (int64_t)m0 : (int64_t)m0 * lda);
  const float *B = (const float *)p.b + (BT ? (int64_t)n0 * ldb : (int64_t)n0);
  auto stage = [&](char *ta, char *tb, int k0) {
    if (AT) f_stage_b<FT>(A, lda, k0, ta, wave, lane);
    else f_stage_a<FT>(A + k0, lda, 0, ta, wave, lane);
    if (BT) f_stage_a<FT>(B + k0, ldb, 0, tb, wave, lane);
    else f_stage_b<FT>(B, ldb, k0, tb, wave, lane);
  };
  float *C = (float *)p.c;

  f32x4 acc[NI][NI];
#pragma unroll
  for (int i = 0; i < NI; ++i)
#pragma unroll
    for (int j = 0; j < NI; ++j) acc[i][j] = (f32x4){0.f, 0.f, 0.f, 0.f};

  const int ksteps = p.k / FK;
  if (kgrp < ksteps) stage(lds_a0, lds_b0, kgrp * FK);
  f_wait_vmem();
  __syncthreads();

  /* every group meets the same barriers: the last rounds of a group with
   * no k-step left skip the work only */
  auto step = [&](const char *ca, const char *cb, char *na, char *nb, int kb) {
    if (kb + KG < ksteps) {
      stage(na, nb, (kb + KG) * FK);
    }
    if (kb < ksteps) {
#pragma unroll
    for (int kc = 0; kc < FK / 16; ++kc) {
      /* B (first operand): element (k = 16 kc + 4g + t, column n) */
      float bf[NI][4];
#pragma unroll
      for (int j = 0; j < NI; ++j) {
        const int n = wn * WT + j * 16 + c;
        if (BT) {
          const f32x4 v = *(const f32x4 *)(cb + fa_off(n, kc * 4 + g));
#pragma unroll
          for (int t = 0; t < 4; ++t) bf[j][t] = v[t];
        } else {
#pragma unroll
          for (int t = 0; t < 4; ++t)
            bf[j][t] = *(const float *)(cb + fb_off<FT>(kc * 16 + 4 * g + t, n >> 2) + ((n & 3) << 2));
        }
      }
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        /* A (second operand): row m, k = 16 kc + 4g .. +3 */
        const int m = wm * WT + i * 16 + c;
        f32x4 af;
        if (AT) {
#pragma unroll
          for (int t = 0; t < 4; ++t)
            af[t] = *(const float *)(ca + fb_off<FT>(kc * 16 + 4 * g + t, m >> 2) + ((m & 3) << 2));
        } else {
          af = *(const f32x4 *)(ca + fa_off(m, kc * 4 + g));
        }
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
          for (int j = 0; j < NI; ++j) acc[i][j] = mfma_f32_16x16x4(bf[j][t], af[t], acc[i][j]);
      }
    }
    }
    f_wait_vmem();
    __syncthreads();
  };

  const int rounds = (ksteps + KG - 1) / KG;
  for (int r = 0; r < rounds; r += 2) {
    step(lds_a0, lds_b0, lds_a1, lds_b1, r * KG + kgrp);
    if (r + 1 < rounds) step(lds_a1, lds_b1, lds_a0, lds_b0, (r + 1) * KG + kgrp);
  }
  if constexpr (KG > 1) {
    /* groups 1 .. KG-1 leave their partial C^T tiles in their own LDS (the
     * last barrier above ended every read of it); group 0 adds them */
    auto slot = [&](int grp, int i, int j) {
      return (f32x4 *)(lds + grp * GROUP_BYTES) + (((wave * NI + i) * NI + j) * 64 + lane);
    };
    if (kgrp > 0) {
#pragma unroll
      for (int i = 0; i < NI; ++i)
#pragma unroll
        for (int j = 0; j < NI; ++j) *slot(kgrp, i, j) = acc[i][j];
    }
    __syncthreads();
    if (kgrp > 0) return;
#pragma unroll
    for (int grp = 1; grp < KG; ++grp)
#pragma unroll
      for (int i = 0; i < NI; ++i)
#pragma unroll
        for (int j = 0; j < NI; ++j) acc[i][j] += *slot(grp, i, j);
  }

  /* acc[i][j] is the C^T tile: lane holds row m0 + wm*WT + i*16 + c,
   * columns n0 + wn*WT + j*16 + 4g .. +3 */
  f32x4 bias[NI];
#pragma unroll
  for (int j = 0; j < NI; ++j)
    bias[j] = EPI == EPI_BIAS_RELU
                  ? *(const f32x4 *)((const float *)p.bias + n0 + wn * WT + j * 16 + 4 * g)
                  : (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int m = m0 + wm * WT + i * 16 + c;
#pragma unroll
    for (int j = 0; j < NI; ++j) {
      f32x4 v = acc[i][j];
      if (EPI == EPI_BIAS_RELU) {
#pragma unroll
        for (int r = 0; r < 4; ++r) v[r] = fmaxf(v[r] + bias[j][r], 0.f);
      }
      *(f32x4 *)(C + (int64_t)m * ldc + n0 + wn * WT + j * 16 + 4 * g) = v;
    }
  }
}

} // namespace

extern "C" __global__ __launch_bounds__(256) void tm_gemm_fast_f32(TmGemmArgs p) {
  gemm_f32<EPI_NONE>(p);
}
extern "C" __global__ __launch_bounds__(256) void tm_sae_fast_f32(TmGemmArgs p) {
  gemm_f32<EPI_BIAS_RELU>(p);
}
extern "C" __global__ __launch_bounds__(256) void tm_gemm_fast_nt_f32(TmGemmArgs p) {
  gemm_f32<EPI_NONE, false, true>(p);
}
extern "C" __global__ __launch_bounds__(256) void tm_gemm_fast_tn_f32(TmGemmArgs p) {
  gemm_f32<EPI_NONE, true, false>(p);
}
/* The K loop split over 2 or 4 groups of waves, for grids of about one
 * workgroup per CU: 128 x 128 tiles at 512 threads, 64 x 64 at 512 or 1024 */
extern "C" __global__ __launch_bounds__(512) void tm_gemm_fast_k2_f32(TmGemmArgs p) {
  gemm_f32<EPI_NONE, false, false, 128, 2>(p);
}
extern "C" __global__ __launch_bounds__(512) void tm_gemm_fast_t64_k2_f32(TmGemmArgs p) {
  gemm_f32<EPI_NONE, false, false, 64, 2>(p);
}
extern "C" __global__ __launch_bounds__(1024) void tm_gemm_fast_t64_k4_f32(TmGemmArgs p) {
  gemm_f32<EPI_NONE, false, false, 64, 4>(p);
}
/* 64 x 64 tiles (4 waves of 32 x 32) for problems with too few 128 x 128 tiles */
extern "C" __global__ __launch_bounds__(256) void tm_gemm_fast_t64_f32(TmGemmArgs p) {
  gemm_f32<EPI_NONE, false, false, 64>(p);
}
extern "C" __global__ __launch_bounds__(256) void tm_sae_fast_t64_f32(TmGemmArgs p) {
  gemm_f32<EPI_BIAS_RELU, false, false, 64>(p);
}
extern "C" __global__ __launch_bounds__(256) void tm_gemm_fast_nt_t64_f32(TmGemmArgs p) {
  gemm_f32<EPI_NONE, false, true, 64>(p);
}
extern "C" __global__ __launch_bounds__(256) void tm_gemm_fast_tn_t64_f32(TmGemmArgs p) {
  gemm_f32<EPI_NONE, true, false, 64>(p);
}
