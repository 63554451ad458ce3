/*
 * Specialised gfx950 GEMM for 16-bit element types: C = A @ B with A [M, K],
 * B [K, N], C [M, N] (unit inner stride, 16-byte aligned rows of A and B,
 * rows no shorter than the matrix); f32 accumulation, output rounded to the
 * element type (the reference's matmul_kernel semantics,
 * Sources/TritonMetalBench/GEMMKernel.swift:28-174).  Instantiations:
 *   - aligned (whole tiles, K a multiple of 64) or ragged (any M, N, K: the
 *     copies clip at the matrix, the last k-step and the stores are masked);
 *   - 256 x 256 tiles (512 threads), 128 x 128 tiles ("t128", 256 threads,
 *     for problems with too few large tiles to fill the chip) or 64 x 64
 *     tiles ("t64", 128 threads, for fewer 128 x 128 tiles than CUs);
 *   - A and B row-major, or B stored transposed ("nt"), or A stored
 *     transposed ("tn");
 *   - plain, or with the SAE encoder's bias + ReLU epilogue (row-major only).
 *
 * Tiling (256 x 256; each smaller tile halves every count): one 512-thread
 * workgroup (8 waves, 2 x 4) computes a tile of C; each wave a 128 x 64
 * sub-tile on v_mfma_f32_16x16x32_{bf16,f16} (8 x 4 accumulators of 16 x 16).
 * Per K step of 64:
 *   - A [256 x 64] and B [64 x 256] tiles are copied HBM -> LDS with
 *     global_load_lds_dwordx4 (aligned) or buffer_load ... lds (ragged: the
 *     buffer range check turns rows past the matrix into zeros), issued from
 *     inline assembly so the compiler pipelines the operand reads behind
 *     them, in their natural row-major layouts (double buffered, 128 KB of
 *     LDS), 16-byte chunks XOR-swizzled by row;
 *   - the A operand (row m, 8 consecutive k) is one ds_read_b128;
 *   - the B operand (column n, 8 consecutive k) is two ds_read_b64_tr_b16:
 *     lane i of a 16-lane group receives element (i & 3) of the 8 bytes
 *     addressed by lane 4e + (i >> 2), so lane 4e + q addresses row k0 + e,
 *     columns n0 + 4q .. +3;
 *   - the MFMA takes B as its first operand, producing C^T tiles: each lane
 *     then holds 4 consecutive columns of one row, stored as one 8-byte write.
 * A transposed operand's tile has the other operand's layout and is copied
 * and read the same way.
 * Ragged K: the last step's k-contiguous fragments are zeroed past column K
 * in registers (the copies there read the next row, or the 16-byte rounding
 * of the last one), and k-major tiles' rows past K arrive as zeros, so no
 * value from outside the matrices reaches a stored element.  Columns of B past
 * N and rows of A past M feed only the outputs past N and M, which are not
 * stored.
 * The 1-D grid is remapped so each XCD owns a contiguous range of tiles,
 * walked in groups of 8 tile rows so concurrently running tiles share A and B
 * panels in that XCD's L2.
 */
#include "common.h"

template <typename T> struct GVec8;
template <> struct GVec8<bf16_t> { typedef bf16x8 type; };
template <> struct GVec8<f16_t> { typedef f16x8 type; };

typedef short gs16x4 __attribute__((ext_vector_type(4)));

TM_DEV void g_wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }

TM_DEV int g_xcd_remap(int wg, int nwg) {
  const int q = nwg >> 3, r = nwg & 7;
  const int xcd = wg & 7, slot = wg >> 3;
  return (xcd < r ? xcd * (q + 1) : r * (q + 1) + (xcd - r) * q) + slot;
}

constexpr int GBK = 64;

/* A tile: 128-byte rows (8 chunks), read only by ds_read_b128 of 16
 * consecutive rows at one chunk: the key row & 7 gives those reads no bank
 * conflicts (SQ_LDS_BANK_CONFLICT reads 0; the key shared with the transposed
 * B reads left 40% of the LDS cycles in conflicts and ran 3% slower). */
TM_DEV int a_swz(int row) { return row & 7; }
TM_DEV int a_off(int row, int chunk) { return row * 128 + ((chunk ^ a_swz(row)) << 4); }

/* B tile: BN-element rows (2 BN bytes: 32 or 16 chunks, a multiple of the
 * 256-byte bank width either way).  A transpose read touches rows
 * k0 + 8g + {0..3} (and +4) at one chunk pair; the even key separates the
 * pairs of the 8 rows served together. */
template <int BN>
TM_DEV int b_swz(int row) {
  /* 128-byte rows (BN = 64) have 8 chunks: the key keeps to 0..6 */
  return BN >= 128 ? ((row & 3) | ((row >> 1) & 4)) << 1 : (row & 3) << 1;
}
template <int BN>
TM_DEV int b_off(int row, int chunk) { return row * (2 * BN) + ((chunk ^ b_swz<BN>(row)) << 4); }

/* Each copy instruction moves a few whole rows of a tile through a buffer
 * resource based at its first row, whose range ends at the matrix's last
 * element (rounded up to 16 bytes, inside the allocation's 256-byte padding):
 * rows past the last row of A or B are read as zeros, and a lane's byte
 * offset is the same for every instruction and k-step, so the addresses cost
 * only scalar instructions.  `rows_left` counts the valid rows from `base`,
 * `width` the valid elements of a row. */
template <int ROWS>
TM_DEV void copy_rows(const void *base, int rows_left, int64_t ld, int width, int voff, char *slot) {
  const int rows = min(rows_left, ROWS);
  const int64_t bytes = rows > 0 ? ((int64_t)(rows - 1) * ld + ((width + 7) & ~7)) * 2 : 0;
  lds_copy16_buffer(raw_buffer_rsrc(base, bytes), voff, lds_addr(slot));
}

/* A [BM x 64] tile, k0 = 0 at `a`: BM / 8 instructions of 8 rows (4 per
 * wave); lane l copies row 8t + (l >> 3), source chunk (l & 7) ^ a_swz(row). */
template <typename T>
TM_DEV void stage_a(const T *a, int64_t lda, int rows_left, int width, int voff, char *tile, int wave) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int t = wave * 4 + i;
    copy_rows<8>(a + (int64_t)(t * 8) * lda, rows_left - t * 8, lda, width, voff, tile + t * 1024);
  }
}
TM_DEV int a_lane_offset(int64_t lda, int lane) {
  const int r = lane >> 3; /* a_swz(8t + r) = a_swz(r) */
  return r * (int)lda * 2 + (((lane & 7) ^ a_swz(r)) << 4);
}

/* B [64 x BN] tile: BN / 8 instructions of RPI = 512 / BN rows (4 per
 * wave); lane l copies row RPI t + l / CPR, source chunk (l % CPR) ^
 * b_swz(row), CPR = BN / 8 chunks per row.  For t = 4w + i the key depends on
 * the lane, w and i only, so each of the 4 offsets is fixed per lane. */
template <typename T, int BN>
TM_DEV void stage_b(const T *b, int64_t ldb, int rows_left, int width, const int (&voff)[4], char *tile,
                    int wave) {
  constexpr int RPI = 512 / BN;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int t = wave * 4 + i;
    copy_rows<RPI>(b + (int64_t)(t * RPI) * ldb, rows_left - t * RPI, ldb, width, voff[i],
                   tile + t * 1024);
  }
}
template <int BN>
TM_DEV void b_lane_offsets(int64_t ldb, int wave, int lane, int (&voff)[4]) {
  constexpr int RPI = 512 / BN, CPR = BN / 8;
  const int h = lane / CPR;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    voff[i] = h * (int)ldb * 2 + (((lane % CPR) ^ b_swz<BN>((wave * 4 + i) * RPI + h)) << 4);
}

/* The aligned kernel's copies: every row and column of a tile is inside the
 * matrix, and plain global addresses measured 1.5-3% faster at 8192^3 than
 * the buffer-resource copies above (the same tiles, the same LDS layout). */
TM_DEV void global_rows_to_lds(const void *src, char *slot) { lds_copy16_global(src, lds_addr(slot)); }

template <typename T>
TM_DEV void stage_a_global(const T *a, int64_t lda, int k0, char *tile, int wave, int lane) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int t = wave * 4 + i;
    const int row = t * 8 + (lane >> 3);
    const int chunk = (lane & 7) ^ a_swz(row);
    global_rows_to_lds(a + (int64_t)row * lda + k0 + chunk * 8, tile + t * 1024);
  }
}

template <typename T, int BN>
TM_DEV void stage_b_global(const T *b, int64_t ldb, int k0, char *tile, int wave, int lane) {
  constexpr int RPI = 512 / BN, CPR = BN / 8;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int t = wave * 4 + i;
    const int row = t * RPI + lane / CPR;
    const int chunk = (lane % CPR) ^ b_swz<BN>(row);
    global_rows_to_lds(b + (int64_t)(k0 + row) * ldb + chunk * 8, tile + t * 1024);
  }
}

/* Keep the first `valid` 16-bit elements of an operand fragment, zero the
 * rest (the k columns past K in the last k-step of a ragged GEMM). */
TM_DEV u32x4 keep_first(u32x4 v, int valid) {
#pragma unroll
  for (int w = 0; w < 4; ++w)
    v[w] &= 2 * w + 1 < valid ? 0xffffffffu : 2 * w < valid ? 0x0000ffffu : 0u;
  return v;
}

/* B operand for k rows kbase + 8g .. +7 of column n0 + c. */
template <int BN>
TM_DEV u32x4 read_b_operand(const char *tile, int kbase, int n0, int g, int c) {
  const int n = n0 + 4 * (c & 3);
  const int chunk = n >> 3, half = (n >> 2) & 1;
  const int ra = kbase + 8 * g + (c >> 2), rb = ra + 4;
  const gs16x4 a = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) gs16x4 *)(tile + b_off<BN>(ra, chunk) + (half << 3)));
  const gs16x4 b = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) gs16x4 *)(tile + b_off<BN>(rb, chunk) + (half << 3)));
  const u32x2 ua = __builtin_bit_cast(u32x2, a), ub = __builtin_bit_cast(u32x2, b);
  return (u32x4){ua[0], ua[1], ub[0], ub[1]};
}

template <typename T>
TM_DEV uint32_t g_pack2(float lo, float hi) {
  typedef float f2 __attribute__((ext_vector_type(2)));
  typedef T t2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f2){lo, hi}, t2));
}

/* BM x BN tiles: 256 x 256 with 8 waves (2 x 4) of 128 x 64, 128 x 128 with
 * 4 waves (2 x 2) of 64 x 64, or 64 x 64 with 2 waves (2 x 1) of 32 x 64.  A
 * wave's sub-tile is (BM / 2) x 64.
 * BT: B is stored transposed (element (k, n) at n * ldb + k, the layout of
 * x @ W^T with W [N, K] row-major).  Its tile is then [BN x 64] k-contiguous
 * like A's, copied and read the same way: the B operand is one
 * ds_read_b128 instead of two transposed reads.
 * AT: A is stored transposed (element (m, k) at k * lda + m, the layout of
 * dY^T X in a linear layer's weight gradient).  Its tile is then [64 x BM]
 * m-contiguous like B's, copied and read the same way (transposed reads). */
/* KG: groups of 2 WN waves splitting the K loop inside the workgroup (1, 2
 * or 4; whole tiles only).  Group h contracts k-steps h, h + KG, ... from its
 * own double-buffered tiles; at the end groups 1 .. KG-1 leave their
 * accumulators in LDS and group 0 adds them in order and stores.  For grids
 * of about one workgroup per CU (128 x 128 tiles at 2048^3, 64 x 64 at
 * 1024^3), this puts more waves on every SIMD. */
/* KSPLIT: the K range of the workgroup comes from grid y and p.splits, and
 * the result is an fp32 partial (64 x 64 tiles only: the instantiations the
 * planner uses when the tiles alone leave the chip idle). */
template <typename T, int EPI, bool RAGGED, int BM, int BN, bool BT = false, bool AT = false,
          int KG = 1, bool KSPLIT = false>
TM_DEV void gemm_fast(const TmGemmArgs &p) {
  typedef typename GVec8<T>::type v8;
  constexpr int GBM = BM, GBN = BN;
  constexpr int A_TILE = BM * GBK * 2; /* BM rows of 128 bytes */
  constexpr int B_TILE = GBK * BN * 2; /* 64 rows of 2 BN bytes */
  constexpr int WN = BN / 64;          /* waves across N */
  constexpr int MI = BM / 32;          /* 16-row tiles per wave */
  static_assert((BM == 256 && BN == 256) || (BM == 128 && BN == 128) || (BM == 64 && BN == 64),
                "tile shapes");
  constexpr int GROUP_BYTES = 2 * (A_TILE + B_TILE);
  static_assert(KG == 1 || (!RAGGED && GROUP_BYTES >= 2 * WN * MI * 4 * 64 * 16),
                "K groups: whole tiles, and a group's tiles hold its accumulators");
  const int tid = threadIdx.x, lane = tid & 63;
  const int kgrp = KG == 1 ? 0 : (tid >> 6) / (2 * WN); /* K group */
  /* the kernel body over its LDS: one workgroup-wide group takes four
   * separate tile arrays (the compiler then knows they do not alias), K
   * groups one array carved per group (`lds`, also where the groups'
   * accumulators meet) */
  auto body = [&](char *const lds_a0, char *const lds_b0, char *const lds_a1, char *const lds_b1,
                  char *const lds) __attribute__((always_inline)) {
  /* uniform in the ragged kernel, whose copy ranges are scalar arithmetic */
  const int wave = RAGGED ? __builtin_amdgcn_readfirstlane(tid >> 6) : KG == 1 ? tid >> 6 : (tid >> 6) % (2 * WN);
  const int g = lane >> 4, c = lane & 15;
  const int wm = wave / WN, wn = wave % WN; /* 2 x WN waves */

  const int mt = (p.m + GBM - 1) / GBM, nt = (p.n + GBN - 1) / GBN;
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

  static_assert(!(AT && BT), "one transposed operand");
  const int64_t lda = AT ? p.sak : p.sam, ldb = BT ? p.sbn : p.sbk, ldc = p.scm;
  const T *A = (const T *)p.a + (AT ? (int64_t)m0 : (int64_t)m0 * lda);
  const T *B = (const T *)p.b + (BT ? (int64_t)n0 * ldb : (int64_t)n0);
  T *C = (T *)p.c;
  const int a_rows = RAGGED ? min(p.m - m0, GBM) : GBM;
  const int b_cols = RAGGED ? min(p.n - n0, GBN) : GBN;

  int va[4];
  if (AT) b_lane_offsets<BM>(lda, wave, lane, va);
  else va[0] = a_lane_offset(lda, lane);
  int vb[4];
  if (BT) vb[0] = a_lane_offset(ldb, lane);
  else b_lane_offsets<BN>(ldb, wave, lane, vb);
  auto stage = [&](char *ta, char *tb, int kb) {
    const int k0 = kb * GBK;
    if (RAGGED) {
      if (AT) stage_b<T, BM>(A + (int64_t)k0 * lda, lda, p.k - k0, a_rows, va, ta, wave);
      else stage_a(A + k0, lda, a_rows, p.k - k0, va[0], ta, wave);
      if (BT) stage_a(B + k0, ldb, b_cols, p.k - k0, vb[0], tb, wave);
      else stage_b<T, BN>(B + (int64_t)k0 * ldb, ldb, p.k - k0, b_cols, vb, tb, wave);
    } else {
      if (AT) stage_b_global<T, BM>(A, lda, k0, ta, wave, lane);
      else stage_a_global(A, lda, k0, ta, wave, lane);
      if (BT) stage_a_global(B, ldb, k0, tb, wave, lane);
      else stage_b_global<T, BN>(B, ldb, k0, tb, wave, lane);
    }
  };

  f32x4 acc[MI][4];
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = (f32x4){0.f, 0.f, 0.f, 0.f};

  /* this workgroup's k-steps: all of them, or (KSPLIT) the split-th of
   * p.splits contiguous ranges (grid y) */
  static_assert(!KSPLIT || (BM == 64 && EPI == EPI_NONE), "K ranges: 64 x 64 GEMM tiles");
  const int ksteps = (p.k + GBK - 1) / GBK;
  const int splits = KSPLIT && p.splits > 1 ? p.splits : 1;
  const int split = splits > 1 ? (int)blockIdx.y : 0;
  const int kbeg = splits > 1 ? (int)((unsigned)(split * ksteps) / (unsigned)splits) : 0;
  const int kend = splits > 1 ? (int)((unsigned)((split + 1) * ksteps) / (unsigned)splits) : ksteps;
  if (kbeg + kgrp < kend) stage(lds_a0, lds_b0, kbeg + kgrp);
  g_wait_vmem();
  __syncthreads();

  /* LAST (ragged K only): A's k columns at or past K are zeroed in registers
   * (and B's, when B is transposed); B's rows past K were copied as zeros by
   * the range check. */
  auto step = [&](auto last_tag, const char *ca, const char *cb, char *na, char *nb, int kb) {
    constexpr bool LAST = decltype(last_tag)::value;
    if (!LAST && kb + KG < kend) stage(na, nb, kb + KG);
    /* a group with no k-step left in the last round still meets its barrier */
#pragma unroll
    for (int ks = 0; ks < 2 && (KG == 1 || kb < kend); ++ks) {
      v8 bf[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (BT) {
          u32x4 b = *(const u32x4 *)(cb + a_off(wn * 64 + j * 16 + c, ks * 4 + g));
          if (LAST) b = keep_first(b, p.k - kb * GBK - ks * 32 - 8 * g);
          bf[j] = __builtin_bit_cast(v8, b);
        } else {
          bf[j] = __builtin_bit_cast(v8, read_b_operand<BN>(cb, ks * 32, wn * 64 + j * 16, g, c));
        }
      }
#pragma unroll
      for (int i = 0; i < MI; ++i) {
        u32x4 a;
        if (AT) {
          /* rows past K arrived as zeros */
          a = read_b_operand<BM>(ca, ks * 32, wm * (BM / 2) + i * 16, g, c);
        } else {
          a = *(const u32x4 *)(ca + a_off(wm * (BM / 2) + i * 16 + c, ks * 4 + g));
          if (LAST) a = keep_first(a, p.k - kb * GBK - ks * 32 - 8 * g);
        }
        const v8 af = __builtin_bit_cast(v8, a);
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = mfma_16x16x32(bf[j], af, acc[i][j]);
      }
      /* the last step has no copy in flight to pace it: keep its operand
       * reads from all being hoisted ahead of the MFMAs (registers) */
      if (LAST) __builtin_amdgcn_sched_barrier(0);
    }
    if (!LAST) {
      g_wait_vmem();
      __syncthreads();
    }
  };
  using Full = std::integral_constant<bool, false>;
  using Last = std::integral_constant<bool, true>;

  /* with a ragged K the last step (in the last range) runs masked */
  const int kfull = RAGGED && p.k % GBK && kend == ksteps ? kend - 1 : kend;
  if constexpr (KG == 1) {
    for (int kb = kbeg; kb < kfull; kb += 2) {
      step(Full{}, lds_a0, lds_b0, lds_a1, lds_b1, kb);
      if (kb + 1 < kfull) step(Full{}, lds_a1, lds_b1, lds_a0, lds_b0, kb + 1);
    }
    if (RAGGED && kfull < kend) {
      const bool odd = (kfull - kbeg) & 1;
      step(Last{}, odd ? lds_a1 : lds_a0, odd ? lds_b1 : lds_b0, nullptr, nullptr, kfull);
    }
  } else {
    const int rounds = (kend - kbeg + KG - 1) / KG;
    for (int r = 0; r < rounds; r += 2) {
      step(Full{}, lds_a0, lds_b0, lds_a1, lds_b1, kbeg + r * KG + kgrp);
      if (r + 1 < rounds) step(Full{}, lds_a1, lds_b1, lds_a0, lds_b0, kbeg + (r + 1) * KG + kgrp);
    }
    /* groups 1 .. KG-1 leave their partial C^T tiles in their own LDS (the
     * last barrier above ended every read of it); group 0 adds them */
    auto slot = [&](int grp, int i, int j) {
      return (f32x4 *)(lds + grp * GROUP_BYTES) + (((wave * MI + i) * 4 + j) * 64 + lane);
    };
    if (kgrp > 0) {
#pragma unroll
      for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) *slot(kgrp, i, j) = acc[i][j];
    }
    __syncthreads();
    if (kgrp > 0) return;
#pragma unroll
    for (int grp = 1; grp < KG; ++grp)
#pragma unroll
      for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] += *slot(grp, i, j);
  }

  /* acc[i][j] is the C^T tile: lane holds row m0 + wm*BM/2 + i*16 + c,
   * columns n0 + wn*64 + j*16 + 4g .. +3 */
  if constexpr (EPI == EPI_NONE) {
    if (splits > 1) {
      /* this range's fp32 partial: rows of round4(n) floats */
      const int64_t np = (p.n + 3) & ~3;
      float *part = p.part + (int64_t)split * p.m * np;
#pragma unroll
      for (int i = 0; i < MI; ++i) {
        const int m = m0 + wm * (BM / 2) + i * 16 + c;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int n = n0 + wn * 64 + j * 16 + 4 * g;
          if (m < p.m && n < p.n) *(f32x4 *)(part + m * np + n) = acc[i][j];
        }
      }
      return;
    }
  }
  /* The bias of the wave's 16 columns, loaded once before any store (the
   * compiler cannot move the loads across stores to C that might alias). */
  float bias[4][4];
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int n = n0 + wn * 64 + j * 16 + 4 * g + r;
      bias[j][r] = EPI == EPI_BIAS_RELU && (!RAGGED || n < p.n) ? to_f32(((const T *)p.bias)[n]) : 0.f;
    }
#pragma unroll
  for (int i = 0; i < MI; ++i) {
    const int m = m0 + wm * (BM / 2) + i * 16 + c;
    if (RAGGED && m >= p.m) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int n = n0 + wn * 64 + j * 16 + 4 * g;
      float v[4];
#pragma unroll
      for (int r = 0; r < 4; ++r)
        v[r] = EPI == EPI_BIAS_RELU ? fmaxf(acc[i][j][r] + bias[j][r], 0.f) : acc[i][j][r];
      T *dst = C + (int64_t)m * ldc + n;
      if (!RAGGED || n + 4 <= p.n) {
        u32x2 w;
        w[0] = g_pack2<T>(v[0], v[1]);
        w[1] = g_pack2<T>(v[2], v[3]);
        *(u32x2 *)dst = w;
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (n + r < p.n) dst[r] = (T)v[r];
      }
    }
  }
  };
  if constexpr (KG == 1) {
    __shared__ __align__(1024) char tile_a0[A_TILE];
    __shared__ __align__(1024) char tile_b0[B_TILE];
    __shared__ __align__(1024) char tile_a1[A_TILE];
    __shared__ __align__(1024) char tile_b1[B_TILE];
    body(tile_a0, tile_b0, tile_a1, tile_b1, nullptr);
  } else {
    __shared__ __align__(1024) char lds[KG * GROUP_BYTES];
    char *const mine = lds + kgrp * GROUP_BYTES;
    body(mine, mine + A_TILE, mine + A_TILE + B_TILE, mine + 2 * A_TILE + B_TILE, lds);
  }
}

/* The K ranges' partials summed in range order (deterministic) into C in the
 * element type: one thread per four columns of a row. */
template <typename T>
TM_DEV void gemm_split_reduce(const TmGemmArgs &p) {
  const int64_t np4 = (p.n + 3) >> 2;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)p.m * np4) return;
  const int64_t m = idx / np4;
  const int n = (int)(idx - m * np4) * 4;
  const int64_t plane = (int64_t)p.m * np4 * 4;
  f32x4 sum = {0.f, 0.f, 0.f, 0.f};
  for (int s = 0; s < p.splits; ++s) sum += *(const f32x4 *)(p.part + s * plane + m * np4 * 4 + n);
  T *dst = (T *)p.c + m * p.scm + n;
  if (n + 4 <= p.n) {
    u32x2 w;
    w[0] = g_pack2<T>(sum[0], sum[1]);
    w[1] = g_pack2<T>(sum[2], sum[3]);
    *(u32x2 *)dst = w;
  } else {
    for (int r = 0; n + r < p.n; ++r) dst[r] = (T)sum[r];
  }
}
extern "C" __global__ __launch_bounds__(256) void tm_gemm_split_reduce_bf16(TmGemmArgs p) {
  gemm_split_reduce<bf16_t>(p);
}
extern "C" __global__ __launch_bounds__(256) void tm_gemm_split_reduce_f16(TmGemmArgs p) {
  gemm_split_reduce<f16_t>(p);
}

#define TM_GEMM_ONE(NAME, T, EPI, RAGGED, TILE, BT, AT)                                     \
  extern "C" __global__ __launch_bounds__(TILE * 2) void NAME(TmGemmArgs p) {                 \
    gemm_fast<T, EPI, RAGGED, TILE, TILE, BT, AT>(p);                                          \
  }
/* the 64 x 64-tile GEMMs with K ranges across workgroups ("_ks") */
#define TM_GEMM_KS(NAME, T, RAGGED, BT, AT, KG)                                               \
  extern "C" __global__ __launch_bounds__(128 * KG) void NAME(TmGemmArgs p) {                 \
    gemm_fast<T, EPI_NONE, RAGGED, 64, 64, BT, AT, KG, true>(p);                               \
  }
#define TM_GEMM_KS_ALL(T, TN)                                                  \
  TM_GEMM_KS(tm_gemm_fast_t64_ks_##TN, T, false, false, false, 1)              \
  TM_GEMM_KS(tm_gemm_ragged_t64_ks_##TN, T, true, false, false, 1)             \
  TM_GEMM_KS(tm_gemm_fast_nt_t64_ks_##TN, T, false, true, false, 1)            \
  TM_GEMM_KS(tm_gemm_ragged_nt_t64_ks_##TN, T, true, true, false, 1)           \
  TM_GEMM_KS(tm_gemm_fast_tn_t64_ks_##TN, T, false, false, true, 1)            \
  TM_GEMM_KS(tm_gemm_ragged_tn_t64_ks_##TN, T, true, false, true, 1)           \
  TM_GEMM_KS(tm_gemm_fast_t64_k2_ks_##TN, T, false, false, false, 2)           \
  TM_GEMM_KS(tm_gemm_fast_t64_k4_ks_##TN, T, false, false, false, 4)
TM_GEMM_KS_ALL(bf16_t, bf16)
TM_GEMM_KS_ALL(f16_t, f16)
/* whole 128 x 128 (64 x 64) tiles, row-major, the K loop over 2 (2 or 4) wave groups */
#define TM_GEMM_KSPLIT(T, TN)                                                                   \
  extern "C" __global__ __launch_bounds__(512) void tm_gemm_fast_t128_k2_##TN(TmGemmArgs p) {   \
    gemm_fast<T, EPI_NONE, false, 128, 128, false, false, 2>(p);                                \
  }                                                                                             \
  extern "C" __global__ __launch_bounds__(256) void tm_gemm_fast_t64_k2_##TN(TmGemmArgs p) {    \
    gemm_fast<T, EPI_NONE, false, 64, 64, false, false, 2>(p);                                  \
  }                                                                                             \
  extern "C" __global__ __launch_bounds__(512) void tm_gemm_fast_t64_k4_##TN(TmGemmArgs p) {    \
    gemm_fast<T, EPI_NONE, false, 64, 64, false, false, 4>(p);                                  \
  }
TM_GEMM_KSPLIT(bf16_t, bf16)
TM_GEMM_KSPLIT(f16_t, f16)
#define TM_GEMM_FAST(T, TN)                                                       \
  TM_GEMM_ONE(tm_gemm_fast_##TN, T, EPI_NONE, false, 256, false, false)           \
  TM_GEMM_ONE(tm_gemm_ragged_##TN, T, EPI_NONE, true, 256, false, false)          \
  TM_GEMM_ONE(tm_sae_fast_##TN, T, EPI_BIAS_RELU, false, 256, false, false)       \
  TM_GEMM_ONE(tm_sae_ragged_##TN, T, EPI_BIAS_RELU, true, 256, false, false)      \
  TM_GEMM_ONE(tm_gemm_fast_t128_##TN, T, EPI_NONE, false, 128, false, false)      \
  TM_GEMM_ONE(tm_gemm_ragged_t128_##TN, T, EPI_NONE, true, 128, false, false)     \
  TM_GEMM_ONE(tm_sae_fast_t128_##TN, T, EPI_BIAS_RELU, false, 128, false, false)  \
  TM_GEMM_ONE(tm_sae_ragged_t128_##TN, T, EPI_BIAS_RELU, true, 128, false, false) \
  TM_GEMM_ONE(tm_gemm_fast_nt_##TN, T, EPI_NONE, false, 256, true, false)         \
  TM_GEMM_ONE(tm_gemm_ragged_nt_##TN, T, EPI_NONE, true, 256, true, false)        \
  TM_GEMM_ONE(tm_gemm_fast_nt_t128_##TN, T, EPI_NONE, false, 128, true, false)    \
  TM_GEMM_ONE(tm_gemm_ragged_nt_t128_##TN, T, EPI_NONE, true, 128, true, false)   \
  TM_GEMM_ONE(tm_gemm_fast_tn_##TN, T, EPI_NONE, false, 256, false, true)         \
  TM_GEMM_ONE(tm_gemm_ragged_tn_##TN, T, EPI_NONE, true, 256, false, true)        \
  TM_GEMM_ONE(tm_gemm_fast_tn_t128_##TN, T, EPI_NONE, false, 128, false, true)    \
  TM_GEMM_ONE(tm_gemm_ragged_tn_t128_##TN, T, EPI_NONE, true, 128, false, true)   \
  TM_GEMM_ONE(tm_gemm_fast_t64_##TN, T, EPI_NONE, false, 64, false, false)        \
  TM_GEMM_ONE(tm_gemm_ragged_t64_##TN, T, EPI_NONE, true, 64, false, false)       \
  TM_GEMM_ONE(tm_sae_fast_t64_##TN, T, EPI_BIAS_RELU, false, 64, false, false)    \
  TM_GEMM_ONE(tm_sae_ragged_t64_##TN, T, EPI_BIAS_RELU, true, 64, false, false)   \
  TM_GEMM_ONE(tm_gemm_fast_nt_t64_##TN, T, EPI_NONE, false, 64, true, false)      \
  TM_GEMM_ONE(tm_gemm_ragged_nt_t64_##TN, T, EPI_NONE, true, 64, true, false)     \
  TM_GEMM_ONE(tm_gemm_fast_tn_t64_##TN, T, EPI_NONE, false, 64, false, true)      \
  TM_GEMM_ONE(tm_gemm_ragged_tn_t64_##TN, T, EPI_NONE, true, 64, false, true)
TM_GEMM_FAST(bf16_t, bf16)
TM_GEMM_FAST(f16_t, f16)
