/*
 * Specialised gfx950 FlashAttention-2 kernels for 16-bit element types (bf16,
 * f16) at head_dim 64 and 128, contiguous head dimension, 16-byte aligned rows.
 * Same maths as the generic kernels (and the reference's
 * AttentionKernel.swift:40-250 / AttentionBackwardKernel.swift): f32 scores and
 * accumulators, P rounded to the element type before P V, exp2 with sm_scale
 * folded into log2(e), L = m + log2(l) in log2 units.  The forward's row sum l
 * is the fp32 sum of the rounded P that P V uses (the reference sums the
 * unrounded P; the two differ by at most the element type's rounding unit,
 * relative).
 *
 * Forward tiling (one workgroup = 4 waves = 128 queries of one head):
 *   - each wave owns 32 queries, held in registers as the B operand of
 *     S^T = K Q^T on v_mfma_f32_16x16x32_{bf16,f16}: a lane then owns one query
 *     (column l%16) and 4 keys of every 16-key tile;
 *   - O^T = V^T P^T keeps the lane <-> query ownership, so P goes from the
 *     softmax straight into the B operand; a ones tile beside V^T gives l;
 *   - K and V tiles [64 keys][D] are double-buffered in LDS in their natural
 *     row order, 16-byte chunks XOR-swizzled by row (KEY_BOTH); K feeds the
 *     A operand by ds_read_b128, V^T by the transposing ds_read_b64_tr_b16;
 *   - causal: key blocks past the workgroup's last query are never visited,
 *     masking only runs on blocks that straddle the diagonal or n_ctx (a wave
 *     whose queries all lie below a block computes it fully masked: skipping
 *     it measured no faster, since the wave then waits at the barrier);
 *   - the 1-D grid is remapped so that each XCD (workgroups are dealt to the
 *     8 XCDs round-robin) runs a contiguous range of heads, keeping one head's
 *     K and V in that XCD's L2; within a head, causal blocks run heaviest first.
 */
#include "common.h"

#include <type_traits>
#include <utility>

#define TM_NEG_INF (-__builtin_inff())

template <typename T> struct Vec8;
template <> struct Vec8<bf16_t> { typedef bf16x8 type; };
template <> struct Vec8<f16_t> { typedef f16x8 type; };

template <typename T>
TM_DEV typename Vec8<T>::type as_vec8(u32x4 x) {
  return __builtin_bit_cast(typename Vec8<T>::type, x);
}

/* Two f32 -> one dword of two 16-bit values (lo first), round to nearest even. */
typedef float f32x2 __attribute__((ext_vector_type(2)));
template <typename T>
TM_DEV uint32_t pack2(float lo, float hi) {
  typedef T t2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){lo, hi}, t2));
}

/* Workgroup index remapped so consecutive logical ids share an XCD. */
TM_DEV int xcd_remap(int wg, int nwg) {
  const int q = nwg >> 3, r = nwg & 7;
  const int xcd = wg & 7, slot = wg >> 3;
  return (xcd < r ? xcd * (q + 1) : r * (q + 1) + (xcd - r) * q) + slot;
}

/* Logical id -> (head, rank of the block's work, 0 = heaviest) for the
 * causal kernels, whose blocks differ in work by up to the number of blocks
 * per head.  Heads are walked in groups of G and, within a group, every
 * head's heaviest block before any head's next one, so each group ends on the
 * light blocks of all its heads instead of the last head's heavy ones
 * starting late.  Measured at B4 H32 S4096 D128 (16 heads per XCD): G = 4
 * runs the forward, dq and dkdv 4-5% faster than head by head (G = 1); G = 2
 * and 8 gain less, G = 3 and 6 (not dividing an XCD's heads) and 16 nothing. */
#ifndef TM_CAUSAL_GROUP
#define TM_CAUSAL_GROUP 4
#endif
TM_DEV void causal_order(int logical, int nb, int heads, int &bh, int &rank) {
  constexpr int G = TM_CAUSAL_GROUP;
  const int group = logical / (G * nb);
  const int r = logical - group * G * nb;
  const int gsize = min(G, heads - group * G);
  rank = r / gsize;
  bh = group * G + (r - rank * gsize);
}


/* ---- LDS staging ----------------------------------------------------------
 * K and V tiles are copied HBM -> LDS by buffer_load_dwordx4 ... lds, which
 * writes each lane's 16 bytes to (wave-uniform LDS base) + 16 * lane: one
 * instruction fills 1 KB.  Rows keep their natural [key][d] order; the 16-byte chunk c of
 * row r is stored at chunk position c ^ (r & 7), so the 16-row MFMA operand
 * reads (K: 16 bytes per lane; V: ds_read_b64_tr_b16, 8 bytes per lane) spread
 * over all banks. */

typedef short s16x4 __attribute__((ext_vector_type(4)));


/* Per-row statistics of one block of BM queries, HBM -> LDS with the tiles:
 * wave w < BM/32 copies L[q0 + 32w .. +31] then Delta[q0 + 32w .. +31] to
 * bytes [256w, 256w + 256) (one 4-byte element per lane; rows past n repeat
 * row n-1 and are masked by the caller), so the block's L and Delta arrive
 * under the same wait as its Q and dO rows. */
template <int BM = 32>
TM_DEV void stage_stats(const float *L, const float *Dl, int q0, int n, char *lds, int wave,
                        int lane) {
  if (wave >= BM / 32) return;
  const int q = min(q0 + wave * 32 + (lane & 31), n - 1);
  const float *src = lane < 32 ? L + q : Dl + q;
  lds_copy4_global(src, lds_addr(lds + wave * 256));
}

/* wait for this wave's outstanding vector-memory operations (vmcnt = 0) */
TM_DEV void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }

/* 16-byte chunk position of logical chunk `chunk` in row `row`: the chunk
 * XORed with a key of the row.  Two read patterns meet the tiles: 16
 * consecutive rows at one chunk (ds_read_b128 of an MFMA operand) and 8
 * consecutive rows at a chunk pair (ds_read_b64_tr_b16 of a k-major operand).
 * KEY_BOTH serves both at full LDS rate; it was found by timing every
 * GF(2)-linear key of the row's low four bits (3 bits at D = 64) on both
 * patterns at once (8 waves per CU, 16 reads in flight per wave): at D = 128
 * it reads within 1% of the best key for each pattern (the row-index key
 * loses 5% on 16-row reads and 30% on transposed reads, the rotate key of the
 * transposed reads 50% on 16-row reads); at D = 64 within 1%.
 * KEY_B128 (the row index) and KEY_TR (a rotation of it) are the
 * per-pattern keys, kept for comparison. */
enum SwizzleKey {
  KEY_TR = 0,   /* transposed reads only */
  KEY_B128 = 1, /* ds_read_b128 of 16 consecutive rows only */
  KEY_BOTH = 2  /* both */
};

template <int D, int KEY = KEY_BOTH>
TM_DEV int swz(int row) {
  if (KEY == KEY_BOTH) {
    /* linear over GF(2) in row bits 0..3: the key of each bit */
    if (D == 128) return ((row & 1) ? 5 : 0) ^ ((row & 2) ? 9 : 0) ^ ((row & 4) ? 10 : 0) ^ ((row & 8) ? 7 : 0);
    return ((row & 1) ? 7 : 0) ^ ((row & 2) ? 4 : 0) ^ ((row & 4) ? 4 : 0) ^ ((row & 8) ? 6 : 0);
  }
  if (KEY == KEY_B128) return D == 128 ? (row & 15) : (row & 7);
  if (D == 128) return ((row & 7) << 1) | ((row >> 3) & 1);
  const int t = row >> 1;
  return ((t & 3) << 1) | ((t >> 2) & 1);
}

template <int D, int KEY = KEY_BOTH>
TM_DEV int tile_off(int row, int chunk) {
  return row * (D * 2) + ((chunk ^ swz<D, KEY>(row)) << 4);
}

/* Copy rows [k0, k0 + ROWS) of a [n, D] tensor (row stride ss elements) into an
 * LDS tile, the four waves sharing the work, by buffer_load ... lds through a
 * buffer resource based at row k0: the lane offsets are loop-invariant, the
 * per-block base is scalar arithmetic, and rows at or past n lie outside the
 * resource, so the hardware delivers zeros for them (finite values that the
 * caller masks: scores to -inf, P to 0).  The host only takes this path when a
 * head's rows span fewer than 2^31 bytes. */
template <typename T, int D, int ROWS, int KEY = KEY_BOTH>
TM_DEV void stage_rows(const T *src, int64_t ss, int k0, int n, char *tile, int wave, int lane) {
  constexpr int CPR = D / 8;                      /* 16-byte chunks per row */
  constexpr int RPI = 64 / CPR;                   /* rows per wave instruction */
  constexpr int INSTR = ROWS / RPI / 4;           /* instructions per wave */
  static_assert(INSTR >= 1 && ROWS % (RPI * 4) == 0, "tile rows");
  const int64_t bytes = (int64_t)(n - k0 - 1) * ss * 2 + D * 2;
  const u32x4 rs = raw_buffer_rsrc(src + (int64_t)k0 * ss, bytes);
#pragma unroll
  for (int i = 0; i < INSTR; ++i) {
    const int t = wave * INSTR + i;
    const int row = t * RPI + lane / CPR;
    const int chunk = (lane % CPR) ^ swz<D, KEY>(row);
    lds_copy16_buffer(rs, (int)(row * ss * 2) + chunk * 16, lds_addr(tile + t * 1024));
  }
}

/* A 16x16x32 MFMA operand whose k index runs down the rows of an LDS tile
 * (the V^T operand of O^T = V^T P^T): lane (c, g) receives rows
 * r0 + 4g + {0..3} and r0 + 16 + 4g + {0..3} of column d0 + c.
 * ds_read_b64_tr_b16 gives lane i of a 16-lane group element (i & 3) of the
 * 8 bytes addressed by lane 4e + (i >> 2), for e = 0..3; so lane j addresses
 * row r0 + 4g + (j >> 2), columns d0 + 4 (j & 3) .. +3. */
template <int D>
TM_DEV u32x4 read_kmajor_operand(const char *tile, int r0, int d0, int g, int c) {
  const int d = d0 + 4 * (c & 3);
  const int chunk = d >> 3, half = (d >> 2) & 1;
  const int ra = r0 + 4 * g + (c >> 2), rb = ra + 16;
  const s16x4 a = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) s16x4 *)(tile + tile_off<D>(ra, chunk) + (half << 3)));
  const s16x4 b = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) s16x4 *)(tile + tile_off<D>(rb, chunk) + (half << 3)));
  const u32x2 ua = __builtin_bit_cast(u32x2, a), ub = __builtin_bit_cast(u32x2, b);
  return (u32x4){ua[0], ua[1], ub[0], ub[1]};
}

TM_DEV float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

/* ---- forward ----------------------------------------------------------------
 * Software-pipelined over key blocks.  Iteration j of a wave issues the P V
 * MFMAs of block j-1 and then the S MFMAs of block j+1, and in their shadow runs
 * the softmax VALU work of block j: fma and exp2 of every score, the packing of
 * P into the B operands of the next P V, and an OR over the packed words.  None
 * of it depends on the MFMAs of the same iteration (the scores of block j
 * completed during iteration j-1).  A gfx950 wave issues about two fp32 VALU
 * operations (or one exp) in the shadow of each 16x16x32 MFMA; the softmax
 * work is spread evenly over the iteration's MFMAs, with every dependent
 * operation at least one MFMA after the one it waits for.
 *
 * Row sums come from the MFMA pipe: a seventeenth d tile whose A operand is all
 * ones accumulates sum_k P[q][k] of the rounded P that the P V product uses, so
 * O = acc / l is normalised by exactly the weights it was built from.
 *
 * Offsets: P = exp2(S * qk_scale - mb) with mb = m + B, m a running row maximum
 * that moves only when it must (PBias below).  Block 0 sets m from its exact
 * row maxima.
 *
 * LDS: K and V tiles double-buffered, in their natural row order with the
 * 16-byte chunks XOR-swizzled with KEY_BOTH (K is read by ds_read_b128, V
 * transposed).  Iteration j reads V(j-1) and K(j+1) and copies
 * V(j) and K(j+2) into the buffers that V(j-2) and K(j) left; the copy
 * instructions are spread over the MFMA stream (issued back to back they stall
 * the wave on the memory pipeline for hundreds of cycles).
 *
 * The interleave is fixed with __builtin_amdgcn_sched_barrier fences between
 * MFMAs and empty volatile asm "pins" on the VALU values, which keep the
 * compiler from sinking each computation to its use or hoisting it to where
 * its inputs become available. */

template <typename F, int... I>
TM_DEV void static_for_impl(F &&f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
TM_DEV void static_for(F &&f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}
template <int LO, typename F, int... I>
TM_DEV void static_range_impl(F &&f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, LO + I>{}), ...);
}
template <int LO, int HI, typename F>
TM_DEV void static_range(F &&f) {
  if constexpr (HI > LO) static_range_impl<LO>(f, std::make_integer_sequence<int, HI - LO>{});
}
#define TM_FENCE() __builtin_amdgcn_sched_barrier(0)

/* An empty volatile asm that reads and redefines a register: it emits nothing
 * but keeps the value's computation on its side of the surrounding fences. */
TM_DEV void pin(float &x) { asm volatile("" : "+v"(x)); }
TM_DEV void pin(uint32_t &x) { asm volatile("" : "+v"(x)); }

typedef __attribute__((address_space(3))) char lds_char_t;
TM_DEV u32x4 lds_read16(uint32_t addr) {
  return *(const __attribute__((address_space(3))) u32x4 *)(lds_char_t *)(uintptr_t)addr;
}
/* the two ds_read_b64_tr_b16 of a k-major operand (read_kmajor_operand) at LDS
 * byte addresses base + off_a, base + off_b */
TM_DEV u32x4 lds_read_kmajor(uint32_t base, int off_a, int off_b) {
  const s16x4 a = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) s16x4 *)(lds_char_t *)(uintptr_t)(base + off_a));
  const s16x4 b = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) s16x4 *)(lds_char_t *)(uintptr_t)(base + off_b));
  const u32x2 ua = __builtin_bit_cast(u32x2, a), ub = __builtin_bit_cast(u32x2, b);
  return (u32x4){ua[0], ua[1], ub[0], ub[1]};
}

/* Copies of [ROWS, D] tiles into XOR-swizzled LDS tiles (key KEY), the four
 * waves sharing the work, one instruction at a time: the lane offsets are
 * computed once; the buffer resource is based at the block's first row, so
 * rows at or past n (and every row of a block at or past n) arrive as zeros. */
template <typename T, int D, int ROWS, int KEY>
struct TileCopy {
  static constexpr int CPR = D / 8, RPI = 64 / CPR;     /* chunks per row, rows per instruction */
  static constexpr int PER_WAVE = ROWS / RPI / 4;
  static_assert(PER_WAVE >= 1 && ROWS % (RPI * 4) == 0, "tile rows");
  int voff[PER_WAVE];
  TM_DEV void init(int64_t ss, int wave, int lane) {
#pragma unroll
    for (int i = 0; i < PER_WAVE; ++i) {
      const int row = (wave * PER_WAVE + i) * RPI + lane / CPR;
      voff[i] = (int)(row * ss * 2) + (((lane % CPR) ^ swz<D, KEY>(row)) << 4);
    }
  }
  static TM_DEV u32x4 rsrc(const T *src, int64_t ss, int k0, int n) {
    const int64_t bytes = k0 < n ? (int64_t)(n - k0 - 1) * ss * 2 + D * 2 : 0;
    return raw_buffer_rsrc(src + (int64_t)k0 * ss, bytes);
  }
  TM_DEV void issue(u32x4 rs, int i, uint32_t tile, int wave) const {
    lds_copy16_buffer(rs, voff[i], tile + (uint32_t)((wave * PER_WAVE + i) * 1024));
  }
  TM_DEV void copy(const T *src, int64_t ss, int k0, int n, uint32_t tile, int wave) const {
    const u32x4 rs = rsrc(src, ss, k0, n);
#pragma unroll
    for (int i = 0; i < PER_WAVE; ++i) issue(rs, i, tile, wave);
  }
};

/* Exponent bias of P.  P = exp2(S * qk_scale - m - B) keeps a row's values at
 * or below 2^-B while its offset m is current, so the exponent field of every
 * rounded P stays below the bit that marks 2.0 (bit 14 of a bf16 or an f16
 * half), and an OR over the packed P words tells whether any value reached 2:
 * a score more than B + 1 (log2 units) above the offset.  Only then does a
 * block take its exact row maxima, move the offsets and redo its P.  bf16 has
 * fp32's exponent range, so B = 32 lets the offset lag the maximum by 33 with
 * no value near overflow; f16's range allows B = 2.  O = acc / l and
 * L = mb + log2(l) are unchanged by any choice of offsets. */
template <typename T> struct PBias;
template <> struct PBias<bf16_t> { static constexpr float B = 32.f; };
template <> struct PBias<f16_t> { static constexpr float B = 2.f; };

template <typename T, int D, bool CAUSAL>
TM_DEV void attn_fwd_fast(const TmAttnFwdArgs &p) {
  constexpr int QT = 2, BM = 128, QW = 32, BN = 64; /* query tiles per wave, queries per workgroup / wave, keys per block */
  constexpr int KT = BN / 16, KK = BN / 32;         /* 16-key tiles of S^T, 32-key halves of P V */
  constexpr int KS = D / 32;            /* k-steps of the S^T contraction */
  constexpr int DT = D / 16;            /* 16-wide d tiles of O^T */
  constexpr int TILE = BN * D * 2;
  constexpr int NM1 = KT * KS * QT;     /* S MFMAs per block */
  constexpr int NM2 = (DT + 1) * KK * QT; /* P V MFMAs per block, row sums included */
  constexpr int VS = QT * BN / 2;       /* softmax slots per iteration (4 per element pair) */
  constexpr int LA = 2;                 /* operands read ahead */
  constexpr float BIAS = PBias<T>::B;
  __shared__ __align__(1024) char lds[4 * TILE];
  const uint32_t kb0 = lds_addr(lds), kb1 = kb0 + TILE, vb0 = kb0 + 2 * TILE, vb1 = kb0 + 3 * TILE;

  typedef typename Vec8<T>::type v8;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4, c = lane & 15;
  const int n = p.n_ctx;
  const int nqb = (n + BM - 1) / BM;
  const int logical = xcd_remap(blockIdx.x, gridDim.x);
  int bh, qb;
  if (CAUSAL) {
    causal_order(logical, nqb, p.heads, bh, qb);
    qb = nqb - 1 - qb;
  } else {
    bh = logical / nqb;
    qb = logical - bh * nqb;
  }
  const int q0 = qb * BM;
  const int qw0 = q0 + wave * QW;
  const int64_t base = (int64_t)bh * p.stride_head;
  const int64_t ss = p.stride_seq;
  const T *Qg = (const T *)p.q + base;
  const T *Kg = (const T *)p.k + base;
  const T *Vg = (const T *)p.v + base;
  T *Og = (T *)p.o + base;

  const int kend = CAUSAL ? min(n, q0 + BM) : n;
  const int nblocks = (kend + BN - 1) / BN;
  /* blocks [0, first_edge) need no mask */
  const int first_edge = CAUSAL ? min(q0 / BN, n / BN) : n / BN;

  TileCopy<T, D, BN, KEY_BOTH> kcp;
  TileCopy<T, D, BN, KEY_BOTH> vcp;
  kcp.init(ss, wave, lane);
  vcp.init(ss, wave, lane);
  if (nblocks > 0) kcp.copy(Kg, ss, 0, n, kb0, wave);
  if (nblocks > 1) kcp.copy(Kg, ss, BN, n, kb1, wave);
  u32x4 qf[QT][KS];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    const int qi = min(qw0 + qt * 16 + c, n - 1);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      qf[qt][ks] = *(const u32x4 *)(Qg + (int64_t)qi * ss + ks * 32 + 8 * g);
  }
  /* lane parts of the operand addresses: K fragment (row c, k-step ks) and
   * V^T fragment (d tile dt); the row offsets of kt, kk and the second
   * transposed read are immediates */
  uint32_t koff[KS], voff[DT];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) koff[ks] = (uint32_t)tile_off<D>(c, ks * 4 + g);
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
    voff[dt] = (uint32_t)(tile_off<D>(4 * g + (c >> 2), 2 * dt + ((c & 3) >> 1)) + ((c & 1) << 3));
  /* the A operand of the row-sum MFMAs: sixteen rows of ones */
  const uint32_t one2 = pack2<T>(1.f, 1.f);
  const u32x4 ones = (u32x4){one2, one2, one2, one2};
  const float qk_scale = p.sm_scale * TM_LOG2E;
  float mb[QT];                 /* offsets m + B */
  f32x4 acc[DT + 1][QT];        /* O^T tiles, then the row sums (four equal rows) */
#pragma unroll
  for (int dt = 0; dt <= DT; ++dt)
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) acc[dt][qt] = (f32x4){0.f, 0.f, 0.f, 0.f};
  /* scores of the block whose softmax runs next and the packed P^T B operands
   * [qt][kk] of the block whose P V runs next, each in two sets that the
   * iterations of the interior loop alternate */
  f32x4 s[KT][QT], s2[KT][QT];
  u32x4 pf[QT][KK], pf2[QT][KK];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt)
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) pf[qt][kk] = (u32x4){0u, 0u, 0u, 0u};

  auto mask_block = [&](f32x4 (&sc)[KT][QT], int k0) {
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      const int qi = qw0 + qt * 16 + c;
#pragma unroll
      for (int kt = 0; kt < KT; ++kt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int key = k0 + kt * 16 + 4 * g + r;
          sc[kt][qt][r] = (key >= n || (CAUSAL && key > qi)) ? TM_NEG_INF : sc[kt][qt][r];
        }
    }
  };
  /* exact row maxima of a block times qk_scale, reduced over the 4 lane groups */
  auto row_max = [&](const f32x4 (&sc)[KT][QT], float (&out)[QT]) {
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      float mx = vmax(sc[0][qt][0], sc[0][qt][1]);
#pragma unroll
      for (int e = 2; e < 4 * KT; e += 2)
        mx = vmax(vmax(mx, sc[e >> 2][qt][e & 3]), sc[e >> 2][qt][(e & 3) + 1]);
      out[qt] = group4_max(mx) * qk_scale;
    }
  };
  /* S^T of one block from K fragments read by `kfrag(kt, ks)` */
  auto scores = [&](f32x4 (&sc)[KT][QT], auto kfrag) {
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) {
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) sc[kt][qt] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const v8 a = as_vec8<T>(kfrag(kt, ks));
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) sc[kt][qt] = mfma_16x16x32(a, as_vec8<T>(qf[qt][ks]), sc[kt][qt]);
      }
    }
  };

  wait_vmem();
  __syncthreads();
  if (nblocks == 0) return;

  /* block 0: scores, and the offsets from its exact row maxima */
  scores(s, [&](int kt, int ks) { return lds_read16(kb0 + koff[ks] + kt * 16 * D * 2); });
  if (first_edge == 0) mask_block(s, 0);
  {
    float mx[QT];
    row_max(s, mx);
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) mb[qt] = mx[qt] + BIAS;
  }
  /* every wave has read kb0 before iteration 0 copies K(2) into it */
  __syncthreads();

  /* Iteration j.  PV: the P V of block j-1; SM: the softmax of block j; SN: the
   * scores of block j+1 (the tail computes them even for a block that does not
   * exist, from stale LDS; they are never used); EDGE: block j takes the mask.
   * vrd/krd: LDS addresses of the V(j-1) and K(j+1) tiles; vdst/kdst: where
   * V(j) and K(j+2) are copied. */
  auto iteration = [&](auto pv_tag, auto sm_tag, auto sn_tag, auto edge_tag, uint32_t vrd,
                       uint32_t krd, uint32_t vdst, uint32_t kdst, int j, f32x4 (&s)[KT][QT],
                       f32x4 (&sn)[KT][QT], u32x4 (&pf)[QT][KK], u32x4 (&pn)[QT][KK]) {
    constexpr bool PV = decltype(pv_tag)::value;
    constexpr bool SM = decltype(sm_tag)::value;
    constexpr bool SN = decltype(sn_tag)::value;
    constexpr bool EDGE = decltype(edge_tag)::value;
    constexpr int NA = PV ? NM2 : 0, NB = SN ? NM1 : 0, NM = NA + NB;
    const int k0 = j * BN;
    /* copies of V(j) and K(j+2), one instruction every CSTRIDE MFMAs (a K
     * block past the end copies zeros) */
    constexpr int NCV = SM ? decltype(vcp)::PER_WAVE : 0, NCK = decltype(kcp)::PER_WAVE;
    constexpr int NC = NCV + NCK;
    constexpr int CSTRIDE = NM >= 4 * NC ? 4 : (NM >= 2 * NC ? 2 : 1);
    const u32x4 rsv = decltype(vcp)::rsrc(Vg, ss, k0, n);
    const u32x4 rsk = decltype(kcp)::rsrc(Kg, ss, k0 + 2 * BN, n);
    auto copy_at = [&](auto cc) {
      constexpr int cidx = decltype(cc)::value;
      if constexpr (cidx < NCV) vcp.issue(rsv, cidx, vdst, wave);
      else if constexpr (cidx < NC) kcp.issue(rsk, cidx - NCV, kdst, wave);
    };

    /* operand o: (kk, dt) of the P V part for o < NA/QT, the row-sum ones
     * first in each kk (no LDS wait behind them), then (ks, kt) of the S part:
     * k-step-major, so consecutive score MFMAs feed eight independent
     * accumulators (kt-major gave two; 0.5-1% slower at configs 4 and 5) */
    u32x4 opnd[NM > 0 ? NM / QT : 1];
    auto read_op = [&](auto oo) {
      constexpr int o = decltype(oo)::value;
      if constexpr (o < NA / QT) {
        constexpr int kk = o / (DT + 1), dt = (o % (DT + 1) + DT) % (DT + 1);
        if constexpr (dt == DT) opnd[o] = ones;
        else opnd[o] = lds_read_kmajor(vrd + voff[dt], 32 * kk * D * 2, (32 * kk + 16) * D * 2);
      } else if constexpr (o < NM / QT) {
        constexpr int b = o - NA / QT, kt = b % KT, ks = b / KT;
        opnd[o] = lds_read16(krd + koff[ks] + kt * 16 * D * 2);
      }
    };
    /* softmax slot v: element pair u = v / 4 (elements 2w, 2w+1 of [qt][kk])
     * as fma, exp, pack and OR on four consecutive slots */
    uint32_t big = 0;       /* OR of the packed P words */
    float px[2], pe[2];
    uint32_t wd = 0, wprev = 0;
    auto vslot = [&](auto vv) {
      constexpr int v = decltype(vv)::value;
      constexpr int u = v / 4, beat = v % 4, qt = u / (BN / 8), kk = (u / 4) % KK, w = u % 4;
      constexpr int e0 = 2 * w, e1 = 2 * w + 1;
      if constexpr (beat == 0) {
        px[0] = __builtin_fmaf(s[2 * kk + (e0 >> 2)][qt][e0 & 3], qk_scale, -mb[qt]);
        px[1] = __builtin_fmaf(s[2 * kk + (e1 >> 2)][qt][e1 & 3], qk_scale, -mb[qt]);
        pin(px[0]);
        pin(px[1]);
      } else if constexpr (beat == 1) {
        pe[0] = fast_exp2(px[0]);
        pe[1] = fast_exp2(px[1]);
        pin(pe[0]);
        pin(pe[1]);
      } else if constexpr (beat == 2) {
        wd = pack2<T>(pe[0], pe[1]);
        pin(wd);
        pn[qt][kk][w] = wd;
      } else if constexpr (u % 2 == 0) {
        wprev = wd; /* ORed with the next pair's word: one v_or3 per two words */
      } else {
        big = big | wprev | wd;
        pin(big);
      }
    };

    if constexpr (SM) {
      if (EDGE) mask_block(s, k0);
    }
    if constexpr (SN) {
#pragma unroll
      for (int kt = 0; kt < KT; ++kt)
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) sn[kt][qt] = (f32x4){0.f, 0.f, 0.f, 0.f};
    }
    static_for<(LA < NM / QT ? LA : NM / QT)>([&](auto o) { read_op(o); });
    if constexpr (SM && NM == 0) static_for<VS>([&](auto vv) { vslot(vv); });
    if constexpr (NM < NC) static_for<NC>([&](auto cc) { copy_at(cc); });
    static_for<NM>([&](auto ii) {
      constexpr int i = decltype(ii)::value;
      constexpr int o = i / QT, qt = i % QT;
      if constexpr (qt == 0 && o + LA < NM / QT) read_op(std::integral_constant<int, o + LA>{});
      if constexpr (NM >= NC && i % CSTRIDE == 1 && i / CSTRIDE < NC)
        copy_at(std::integral_constant<int, i / CSTRIDE>{});
      if constexpr (i < NA) {
        constexpr int kk = o / (DT + 1), dt = (o % (DT + 1) + DT) % (DT + 1);
        acc[dt][qt] = mfma_16x16x32(as_vec8<T>(opnd[o]), as_vec8<T>(pf[qt][kk]), acc[dt][qt]);
      } else {
        constexpr int b = o - NA / QT, kt = b % KT, ks = b / KT;
        sn[kt][qt] = mfma_16x16x32(as_vec8<T>(opnd[o]), as_vec8<T>(qf[qt][ks]), sn[kt][qt]);
      }
      if constexpr (SM)
        static_range<(i * VS + NM - 1) / NM, ((i + 1) * VS + NM - 1) / NM>([&](auto vv) { vslot(vv); });
      TM_FENCE();
    });
    if constexpr (SM) {
      /* some P reached 2: recompute this block's scores with K fragments read
       * straight from HBM (its tile is being overwritten and its scores are no
       * longer in registers), take the exact row maxima, move the offsets,
       * redo P, and scale O and the row sums, which hold the P V of every
       * block computed under the old offsets (all issued above) */
      if (__builtin_amdgcn_ballot_w64((big & 0x40004000u) != 0) != 0) {
        f32x4 sr[KT][QT];
        scores(sr, [&](int kt, int ks) {
          const int key = min(k0 + kt * 16 + c, n - 1);
          return *(const u32x4 *)(Kg + (int64_t)key * ss + ks * 32 + 8 * g);
        });
        mask_block(sr, k0);
        float mx[QT];
        row_max(sr, mx);
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) {
          const float m_new = fmaxf(mb[qt], mx[qt] + BIAS);
          const float alpha = fast_exp2(mb[qt] - m_new);
          mb[qt] = m_new;
#pragma unroll
          for (int kk = 0; kk < KK; ++kk)
#pragma unroll
            for (int w = 0; w < 4; ++w) {
              const int e0 = 2 * w, e1 = 2 * w + 1;
              const float p0 = fast_exp2(__builtin_fmaf(sr[2 * kk + (e0 >> 2)][qt][e0 & 3], qk_scale, -m_new));
              const float p1 = fast_exp2(__builtin_fmaf(sr[2 * kk + (e1 >> 2)][qt][e1 & 3], qk_scale, -m_new));
              pn[qt][kk][w] = pack2<T>(p0, p1);
            }
#pragma unroll
          for (int dt = 0; dt <= DT; ++dt) acc[dt][qt] *= alpha;
        }
      }
    }
    wait_vmem();
    __syncthreads();
  };
  using T_ = std::integral_constant<bool, true>;
  using F_ = std::integral_constant<bool, false>;
  auto take_second_set = [&]() {
#pragma unroll
    for (int kt = 0; kt < KT; ++kt)
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) s[kt][qt] = s2[kt][qt];
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) pf[qt][kk] = pf2[qt][kk];
    }
  };

  /* iteration j reads V(j-1) from vb[(j-1)&1] and K(j+1) from kb[(j+1)&1], and
   * copies V(j) into vb[j&1] and K(j+2) into kb[j&1] */
  iteration(F_{}, T_{}, T_{}, T_{}, vb1, kb1, vb0, kb0, 0, s, s2, pf, pf2);
  take_second_set();
  int j = 1;
  /* interior pairs: blocks j-1 .. j+2 exist and j, j+1 need no mask */
  for (; j + 2 < nblocks && j + 1 < first_edge; j += 2) {
    iteration(T_{}, T_{}, T_{}, F_{}, vb0, kb0, vb1, kb1, j, s, s2, pf, pf2);
    iteration(T_{}, T_{}, T_{}, F_{}, vb1, kb1, vb0, kb0, j + 1, s2, s, pf2, pf);
  }
  /* the rest, masked; j is odd here */
  uint32_t vr = vb0, kr = kb0, vc = vb1, kc = kb1;
  for (; j < nblocks; ++j) {
    iteration(T_{}, T_{}, T_{}, T_{}, vr, kr, vc, kc, j, s, s2, pf, pf2);
    take_second_set();
    const uint32_t t0 = vr, t1 = kr;
    vr = vc;
    kr = kc;
    vc = t0;
    kc = t1;
  }
  iteration(T_{}, F_{}, F_{}, F_{}, vr, kr, vc, kc, j, s, s2, pf, pf2);

#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    const int qi = qw0 + qt * 16 + c;
    const float l = acc[DT][qt][0];
    if (qi < n) {
      const float inv = 1.f / l;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        u32x2 w;
        w[0] = pack2<T>(acc[dt][qt][0] * inv, acc[dt][qt][1] * inv);
        w[1] = pack2<T>(acc[dt][qt][2] * inv, acc[dt][qt][3] * inv);
        *(u32x2 *)(Og + (int64_t)qi * ss + dt * 16 + 4 * g) = w;
      }
      if (p.lse && g == 0) p.lse[(int64_t)bh * p.stride_lse + qi] = mb[qt] + log2f(l);
    }
  }
}

/* ---- backward: Delta ------------------------------------------------------
 * Delta_i = sum_d dO[i, d] O[i, d] in fp32 (AttentionBackwardKernel.swift:
 * 119-124).  HBM-bound: each lane loads 16 bytes of O and of dO per row
 * (D / 8 lanes per row), a wave covers 64 rows with all its loads issued
 * before the first reduction, and each row reduces over its D / 8 lanes. */
template <typename T, int D>
TM_DEV void attn_pre_fast(const TmAttnPreArgs &p) {
  constexpr int LPR = D / 8;        /* lanes per row */
  constexpr int RPI = 64 / LPR;     /* rows per wave instruction */
  constexpr int NI = 64 / RPI;      /* instructions per wave (64 rows) */
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6); /* uniform: LDS bases are scalar */
  const int n = p.n_ctx;
  const int nrb = (n + 255) / 256;
  const int bh = blockIdx.x / nrb;
  const int r0 = (blockIdx.x - bh * nrb) * 256 + wave * 64 + lane / LPR;
  const int64_t base = (int64_t)bh * p.stride_head + (lane % LPR) * 8;
  const T *O = (const T *)p.o + base;
  const T *dO = (const T *)p.dout + base;
  u32x4 o[NI], d[NI];
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int64_t row = min(r0 + i * RPI, n - 1);
    o[i] = *(const u32x4 *)(O + row * p.stride_seq);
    d[i] = *(const u32x4 *)(dO + row * p.stride_seq);
  }
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const typename Vec8<T>::type ov = as_vec8<T>(o[i]), dv = as_vec8<T>(d[i]);
    float acc = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc = __builtin_fmaf(to_f32(ov[e]), to_f32(dv[e]), acc);
#pragma unroll
    for (int off = LPR / 2; off >= 1; off >>= 1) acc += __shfl_xor(acc, off, 64);
    const int row = r0 + i * RPI;
    if ((lane % LPR) == 0 && row < n) p.delta[(int64_t)bh * p.stride_lse + row] = acc;
  }
}

#define TM_PRE_FAST(T, TN, D) \
  extern "C" __global__ __launch_bounds__(256) void tm_attn_pre_fast_##TN##_d##D(TmAttnPreArgs p) { \
    attn_pre_fast<T, D>(p); \
  }
TM_PRE_FAST(bf16_t, bf16, 64)
TM_PRE_FAST(bf16_t, bf16, 128)
TM_PRE_FAST(f16_t, f16, 64)
TM_PRE_FAST(f16_t, f16, 128)

/* ---- backward: dQ ------------------------------------------------------
 * One workgroup = 4 waves = 128 queries; each wave owns 32 queries and walks
 * the key blocks (64 keys) of its head.  Per block, with the lane owning one
 * query as in the forward:
 *   S^T  = K Q^T, dP^T = V dO^T            (K, V: ds_read_b128 of the tiles)
 *   P^T  = exp2(qk_scale S^T - L), dS^T = P^T (dP^T - Delta)
 *   dQ^T += K^T dS^T                       (K^T: ds_read_b64_tr_b16 of the K tile)
 * dS is rounded to the element type before its dot, as the reference does
 * (AttentionBackwardKernel.swift:155-160).  The dP^T MFMAs start from -Delta
 * (a lane's four values share its query) instead of zero, so they deliver
 * dP^T - Delta with no subtraction per element.  LDS is addressed by 32-bit
 * offsets whose lane parts are computed once: with flat tile pointers (and a
 * branch between the two buffer phases in the masked loop) the kernel needed
 * 256 registers and spilled; so it needs 234 and runs 3% faster. */
template <int D> struct DqLds { static constexpr int BYTES = 4 * 64 * D * 2; };
template <typename T, int D, bool CAUSAL>
TM_DEV void attn_dq_fast(const TmAttnDqArgs &p, char *lds, int wg, int nwg) {
  constexpr int BM = 128, BN = 64, QW = 32;
  constexpr int KS = D / 32;
  constexpr int TILE = BN * D * 2;
  const uint32_t buf_a = lds_addr(lds), buf_b = buf_a + 2 * TILE;

  typedef typename Vec8<T>::type v8;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6); /* uniform: LDS bases are scalar */
  const int g = lane >> 4, c = lane & 15;
  const int n = p.n_ctx;
  const int nqb = (n + BM - 1) / BM;
  const int logical = xcd_remap(wg, nwg);
  int bh, qb;
  if (CAUSAL) {
    causal_order(logical, nqb, p.heads, bh, qb);
    qb = nqb - 1 - qb;
  } else {
    bh = logical / nqb;
    qb = logical - bh * nqb;
  }
  const int q0 = qb * BM;
  const int qw0 = q0 + wave * QW;
  const int64_t base = (int64_t)bh * p.stride_head;
  const int64_t ss = p.stride_seq;
  const T *Qg = (const T *)p.q + base;
  const T *Kg = (const T *)p.k + base;
  const T *Vg = (const T *)p.v + base;
  const T *dOg = (const T *)p.dout + base;
  T *dQg = (T *)p.dq + base;
  const float *Lg = p.lse + (int64_t)bh * p.stride_lse;
  const float *Dg = p.delta + (int64_t)bh * p.stride_lse;

  const int kend = CAUSAL ? min(n, q0 + BM) : n;
  const int nblocks = (kend + BN - 1) / BN;
  TileCopy<T, D, BN, KEY_BOTH> kvcp; /* K and V rows share the lane offsets */
  kvcp.init(ss, wave, lane);
  if (nblocks > 0) {
    kvcp.copy(Kg, ss, 0, n, buf_a, wave);
    kvcp.copy(Vg, ss, 0, n, buf_a + TILE, wave);
  }
  /* lane parts of the operand offsets (row offsets of kt are immediates) */
  uint32_t koff[KS], kmoff[D / 16];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) koff[ks] = (uint32_t)tile_off<D>(c, ks * 4 + g);
#pragma unroll
  for (int dt = 0; dt < D / 16; ++dt)
    kmoff[dt] = (uint32_t)(tile_off<D>(4 * g + (c >> 2), 2 * dt + ((c & 3) >> 1)) + ((c & 1) << 3));

  u32x4 qf[2][KS], df[2][KS];
  float lse[2], dlt[2];
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    const int qi = min(qw0 + qt * 16 + c, n - 1);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      qf[qt][ks] = *(const u32x4 *)(Qg + (int64_t)qi * ss + ks * 32 + 8 * g);
      df[qt][ks] = *(const u32x4 *)(dOg + (int64_t)qi * ss + ks * 32 + 8 * g);
    }
    lse[qt] = Lg[qi];
    dlt[qt] = Dg[qi];
  }
  const float qk_scale = p.sm_scale * TM_LOG2E;
  const f32x4 ndlt[2] = {(f32x4){-dlt[0], -dlt[0], -dlt[0], -dlt[0]},
                         (f32x4){-dlt[1], -dlt[1], -dlt[1], -dlt[1]}};
  f32x4 acc[D / 16][2];
#pragma unroll
  for (int dt = 0; dt < D / 16; ++dt) acc[dt][0] = acc[dt][1] = (f32x4){0.f, 0.f, 0.f, 0.f};

  wait_vmem();
  __syncthreads();

  auto step = [&](auto edge_tag, uint32_t cur, uint32_t nxt, int j) {
    constexpr bool EDGE = decltype(edge_tag)::value;
    const int k0 = j * BN;
    if (j + 1 < nblocks) {
      kvcp.copy(Kg, ss, k0 + BN, n, nxt, wave);
      kvcp.copy(Vg, ss, k0 + BN, n, nxt + TILE, wave);
    }
    /* two 32-key halves: scores, dS, then the dQ MFMAs of that half, so only
     * half of S^T and dP^T is live at a time */
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      f32x4 s[2][2], dp[2][2];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int kt = 2 * kk + h;
        s[h][0] = s[h][1] = (f32x4){0.f, 0.f, 0.f, 0.f};
        dp[h][0] = ndlt[0];
        dp[h][1] = ndlt[1];
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          const v8 ka = as_vec8<T>(lds_read16(cur + koff[ks] + kt * 16 * D * 2));
          const v8 va = as_vec8<T>(lds_read16(cur + TILE + koff[ks] + kt * 16 * D * 2));
          s[h][0] = mfma_16x16x32(ka, as_vec8<T>(qf[0][ks]), s[h][0]);
          s[h][1] = mfma_16x16x32(ka, as_vec8<T>(qf[1][ks]), s[h][1]);
          dp[h][0] = mfma_16x16x32(va, as_vec8<T>(df[0][ks]), dp[h][0]);
          dp[h][1] = mfma_16x16x32(va, as_vec8<T>(df[1][ks]), dp[h][1]);
        }
      }
      u32x4 dsf[2];
#pragma unroll
      for (int qt = 0; qt < 2; ++qt) {
        const int qi = qw0 + qt * 16 + c;
        float ds[2][4];
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            float x = __builtin_fmaf(s[h][qt][r], qk_scale, -lse[qt]);
            if (EDGE) {
              const int key = k0 + (2 * kk + h) * 16 + 4 * g + r;
              x = (key >= n || (CAUSAL && key > qi)) ? TM_NEG_INF : x;
            }
            ds[h][r] = fast_exp2(x) * dp[h][qt][r];
          }
        dsf[qt] = (u32x4){pack2<T>(ds[0][0], ds[0][1]), pack2<T>(ds[0][2], ds[0][3]),
                          pack2<T>(ds[1][0], ds[1][1]), pack2<T>(ds[1][2], ds[1][3])};
      }
      /* dQ^T += K^T dS^T over this half's 32 keys */
#pragma unroll
      for (int dt = 0; dt < D / 16; ++dt) {
        const v8 a = as_vec8<T>(lds_read_kmajor(cur + kmoff[dt], 32 * kk * D * 2, (32 * kk + 16) * D * 2));
        acc[dt][0] = mfma_16x16x32(a, as_vec8<T>(dsf[0]), acc[dt][0]);
        acc[dt][1] = mfma_16x16x32(a, as_vec8<T>(dsf[1]), acc[dt][1]);
      }
      /* keep the next half's loads below this point (register pressure) */
      __builtin_amdgcn_sched_barrier(0);
    }
    wait_vmem();
    __syncthreads();
  };
  using Interior = std::integral_constant<bool, false>;
  using Edge = std::integral_constant<bool, true>;

  const int n_interior = CAUSAL ? min(q0 / BN, n / BN) : n / BN;
  int j = 0;
  for (; j + 1 < n_interior; j += 2) {
    step(Interior{}, buf_a, buf_b, j);
    step(Interior{}, buf_b, buf_a, j + 1);
  }
  for (; j < nblocks; ++j) step(Edge{}, (j & 1) ? buf_b : buf_a, (j & 1) ? buf_a : buf_b, j);

#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    const int qi = qw0 + qt * 16 + c;
    if (qi < n) {
#pragma unroll
      for (int dt = 0; dt < D / 16; ++dt) {
        u32x2 w;
        w[0] = pack2<T>(acc[dt][qt][0] * p.sm_scale, acc[dt][qt][1] * p.sm_scale);
        w[1] = pack2<T>(acc[dt][qt][2] * p.sm_scale, acc[dt][qt][3] * p.sm_scale);
        *(u32x2 *)(dQg + (int64_t)qi * ss + dt * 16 + 4 * g) = w;
      }
    }
  }
}

/* ---- backward: dK, dV ---------------------------------------------------
 * One workgroup = 4 waves = 128 keys; each wave owns 32 keys, held in
 * registers (K^T and V^T as B operands), and walks the query blocks (BM = 32
 * queries at D = 128, 64 at D = 64) of its head.  Per block, with the lane owning one key:
 *   S  = Q K^T, dP = dO V^T                (Q, dO: ds_read_b128 of the tiles)
 *   P  = exp2(qk_scale S - L), dS = P (dP - Delta)
 *   dV^T += dO^T P, dK^T += Q^T dS         (dO^T, Q^T: ds_read_b64_tr_b16)
 * (carried as -dS, see below)
 * P and dS are rounded to the element type before their dots
 * (AttentionBackwardKernel.swift:357-369).  Causal: the heaviest key blocks
 * (lowest keys) run first and the query walk starts at the block's first key.
 *
 * Software pipeline over query blocks, three LDS buffers in rotation: step i
 * issues the copy of block i+2, computes S, dP, P and dS of block i+1, and
 * accumulates dV, dK from block i's P and dS (kept in registers since step
 * i-1).  The softmax of one block and the gradient MFMAs of the previous one
 * are independent, so the wave's VALU work overlaps its MFMA work.  Buffer
 * indices are compile-time (PH = i mod 3) so the compiler sees that the
 * in-flight copy never aliases the tiles being read. */
template <typename T, int D, bool CAUSAL, bool FUSED = false>
TM_DEV void attn_dkdv_fast(const TmAttnDkdvArgs &p, float *dq_acc = nullptr) {
  /* query rows per step: 64 at D = 64 (twice the MFMA work per barrier and
   * per softmax pass; measured 7% faster), 32 at D = 128, where 64 would not
   * fit the registers */
  constexpr int BN = 128, KW = 32, BM = D == 64 ? 64 : 32;
  /* The kernel carries -dS = P (Delta - dP): the dP MFMAs run on -V and start
   * from Delta, so no subtraction per element.  dK accumulates -dK and flips
   * the sign at the store; FUSED adds dQ with -K. */
  constexpr int QT = BM / 16, KK = BM / 32;
  constexpr int KS = D / 32;
  constexpr int TILE = BM * D * 2;
  constexpr int STATS = 2 * TILE; /* per 32 queries: L[32] then Delta[32], fp32 */
  constexpr int BUF = 2 * TILE + BM * 8;
  __shared__ __align__(1024) char lds_0[BUF];
  __shared__ __align__(1024) char lds_1[BUF];
  __shared__ __align__(1024) char lds_2[BUF];
  /* FUSED: dS of two query blocks, [BN keys][BM queries] each, so that every
   * wave can read all 128 keys of it (ds_off) */
  constexpr int DS_TILE = BN * BM * 2;
  __shared__ __align__(1024) char lds_ds[FUSED ? 2 * DS_TILE : 16];

  typedef typename Vec8<T>::type v8;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6); /* uniform: LDS bases are scalar */
  const int g = lane >> 4, c = lane & 15;
  const int n = p.n_ctx;
  const int nkb = (n + BN - 1) / BN;
  const int logical = xcd_remap(blockIdx.x, gridDim.x);
  int bh, kb;
  if (CAUSAL) {
    causal_order(logical, nkb, p.heads, bh, kb);
  } else {
    bh = logical / nkb;
    kb = logical - bh * nkb;
  }
  const int k0 = kb * BN;
  const int kw0 = k0 + wave * KW;
  const int64_t base = (int64_t)bh * p.stride_head;
  const int64_t ss = p.stride_seq;
  const T *Qg = (const T *)p.q + base;
  const T *Kg = (const T *)p.k + base;
  const T *Vg = (const T *)p.v + base;
  const T *dOg = (const T *)p.dout + base;
  T *dKg = (T *)p.dk + base;
  T *dVg = (T *)p.dv + base;
  const float *Lg = p.lse + (int64_t)bh * p.stride_lse;
  const float *Dg = p.delta + (int64_t)bh * p.stride_lse;

  const int q_start = CAUSAL ? k0 : 0;
  const int nblocks = (n - q_start + BM - 1) / BM;

  auto stage = [&](char *buf, int blk) {
    const int qs = q_start + blk * BM;
    stage_rows<T, D, BM>(Qg, ss, qs, n, buf, wave, lane);
    stage_rows<T, D, BM>(dOg, ss, qs, n, buf + TILE, wave, lane);
    stage_stats<BM>(Lg, Dg, qs, n, buf + STATS, wave, lane);
  };

  u32x4 kf[2][KS], vf[2][KS];
#pragma unroll
  for (int kt = 0; kt < 2; ++kt) {
    const int key = min(kw0 + kt * 16 + c, n - 1);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      kf[kt][ks] = *(const u32x4 *)(Kg + (int64_t)key * ss + ks * 32 + 8 * g);
      vf[kt][ks] = *(const u32x4 *)(Vg + (int64_t)key * ss + ks * 32 + 8 * g);
      /* -V: every element's sign bit flipped (exact) */
      vf[kt][ks] ^= (u32x4){0x80008000u, 0x80008000u, 0x80008000u, 0x80008000u};
    }
  }
  /* FUSED: K as the B operand of dQ[:, wave's D/4 columns] = dS K, for the
   * 128 keys in four 32-key steps; element j of a lane holds key
   * 32 ks + 4g + j (j < 4) or 32 ks + 16 + 4g + j - 4, the order in which the
   * transposing read of dS delivers them.  Keys at or past n are zero, so the
   * (finite) dS of those padding keys adds nothing. */
  constexpr int NT = FUSED ? D / 64 : 1;
  u32x4 kq[FUSED ? 4 : 1][NT];
  if constexpr (FUSED) {
    const uint16_t *Kh = (const uint16_t *)Kg;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        const int col = wave * (D / 4) + nt * 16 + c;
        uint32_t h[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int key = k0 + ks * 32 + (j < 4 ? 4 * g + j : 16 + 4 * g + j - 4);
          h[j] = key < n ? Kh[(int64_t)key * ss + col] : 0u;
        }
        /* -K (sign bits flipped, exact): dS K = (-dS)(-K) */
        kq[ks][nt] = (u32x4){h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16),
                             h[6] | (h[7] << 16)} ^
                     (u32x4){0x80008000u, 0x80008000u, 0x80008000u, 0x80008000u};
      }
  }
  const float qk_scale = p.sm_scale * TM_LOG2E;
  const float dk_scale = -p.sm_scale; /* dk holds -dK / sm_scale */
  f32x4 dk[D / 16][2], dv[D / 16][2];
#pragma unroll
  for (int dt = 0; dt < D / 16; ++dt)
    dk[dt][0] = dk[dt][1] = dv[dt][0] = dv[dt][1] = (f32x4){0.f, 0.f, 0.f, 0.f};

  /* S, dP, then P and dS (rounded, packed as MFMA B operands) of block `blk`
   * from its tile.  EDGE blocks (the diagonal band, a ragged end) apply the
   * mask; interior blocks run straight-line code. */
  auto scores = [&](auto edge_tag, const char *cur, int blk, u32x4 (&pf)[2][KK], u32x4 (&dsf)[2][KK]) {
    constexpr bool EDGE = decltype(edge_tag)::value;
    const int qs = q_start + blk * BM;
    /* L and Delta of queries qs + qt*16 + 4g + {0..3} */
    f32x4 lse[QT], dlt[QT];
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      lse[qt] = *(const f32x4 *)(cur + STATS + (qt >> 1) * 256 + ((qt & 1) * 16 + 4 * g) * 4);
      dlt[qt] = *(const f32x4 *)(cur + STATS + (qt >> 1) * 256 + 128 + ((qt & 1) * 16 + 4 * g) * 4);
    }
    f32x4 s[2][QT], dp[2][QT];
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      s[0][qt] = s[1][qt] = (f32x4){0.f, 0.f, 0.f, 0.f};
      /* Delta - dP: started from Delta, on -V */
      dp[0][qt] = dp[1][qt] = dlt[qt];
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const v8 qa = as_vec8<T>(*(const u32x4 *)(cur + tile_off<D>(qt * 16 + c, ks * 4 + g)));
        const v8 da =
            as_vec8<T>(*(const u32x4 *)(cur + TILE + tile_off<D>(qt * 16 + c, ks * 4 + g)));
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
          s[kt][qt] = mfma_16x16x32(qa, as_vec8<T>(kf[kt][ks]), s[kt][qt]);
          dp[kt][qt] = mfma_16x16x32(da, as_vec8<T>(vf[kt][ks]), dp[kt][qt]);
        }
      }
    }
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      const int key = kw0 + kt * 16 + c;
      float pr[QT][4], ds[QT][4];
#pragma unroll
      for (int qt = 0; qt < QT; ++qt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float x = __builtin_fmaf(s[kt][qt][r], qk_scale, -lse[qt][r]);
          if (EDGE) {
            const int qi = qs + qt * 16 + 4 * g + r;
            x = (qi >= n || (CAUSAL && qi < key)) ? TM_NEG_INF : x;
          }
          pr[qt][r] = fast_exp2(x);
          ds[qt][r] = pr[qt][r] * dp[kt][qt][r]; /* -dS */
        }
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) {
        pf[kt][kk] = (u32x4){pack2<T>(pr[2 * kk][0], pr[2 * kk][1]), pack2<T>(pr[2 * kk][2], pr[2 * kk][3]),
                             pack2<T>(pr[2 * kk + 1][0], pr[2 * kk + 1][1]),
                             pack2<T>(pr[2 * kk + 1][2], pr[2 * kk + 1][3])};
        dsf[kt][kk] = (u32x4){pack2<T>(ds[2 * kk][0], ds[2 * kk][1]), pack2<T>(ds[2 * kk][2], ds[2 * kk][3]),
                              pack2<T>(ds[2 * kk + 1][0], ds[2 * kk + 1][1]),
                              pack2<T>(ds[2 * kk + 1][2], ds[2 * kk + 1][3])};
      }
    }
  };

  /* dV^T += dO^T P, dK^T += Q^T dS for the block whose tile is `cur` */
  auto grads = [&](const char *cur, const u32x4 (&pf)[2][KK], const u32x4 (&dsf)[2][KK]) {
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt) {
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) {
        const v8 doa = as_vec8<T>(read_kmajor_operand<D>(cur + TILE, 32 * kk, dt * 16, g, c));
        const v8 qa = as_vec8<T>(read_kmajor_operand<D>(cur, 32 * kk, dt * 16, g, c));
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
          dv[dt][kt] = mfma_16x16x32(doa, as_vec8<T>(pf[kt][kk]), dv[dt][kt]);
          dk[dt][kt] = mfma_16x16x32(qa, as_vec8<T>(dsf[kt][kk]), dk[dt][kt]);
        }
      }
    }
  };

  /* FUSED: byte offset of queries q .. q+3 (q a multiple of 4) of key row
   * `key` in a dS tile; 16-byte chunks XOR-swizzled so that the 16 rows one
   * transposing read spans fall on distinct banks */
  auto ds_off = [&](int key, int q) {
    constexpr int CPR = BM / 8, RP = 256 / (BM * 2);
    return key * (BM * 2) + (((q >> 3) ^ ((key / RP) % CPR)) << 4) + (((q >> 2) & 1) << 3);
  };
  auto put_ds = [&](int blk, const u32x4 (&dsv)[2][KK]) {
    char *t = lds_ds + (blk & 1) * DS_TILE;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) {
        const int key = wave * KW + kt * 16 + c;
        *(u32x2 *)(t + ds_off(key, 32 * kk + 4 * g)) = (u32x2){dsv[kt][kk][0], dsv[kt][kk][1]};
        *(u32x2 *)(t + ds_off(key, 32 * kk + 16 + 4 * g)) = (u32x2){dsv[kt][kk][2], dsv[kt][kk][3]};
      }
  };
  /* dQ[block rows, this wave's D/4 columns] += dS K over the workgroup's 128
   * keys, added to the fp32 accumulator with one atomic per element: the
   * order in which workgroups reach an address varies, so dQ's rounding does */
  auto dq_block = [&](int blk) {
    const char *t = lds_ds + (blk & 1) * DS_TILE;
    const int qs = q_start + blk * BM;
    f32x4 acc[QT][NT];
#pragma unroll
    for (int qt = 0; qt < QT; ++qt)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) acc[qt][nt] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) {
        const int ra = ks * 32 + 4 * g + (c >> 2), qc = qt * 16 + 4 * (c & 3);
        const s16x4 a0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) s16x4 *)(t + ds_off(ra, qc)));
        const s16x4 a1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) s16x4 *)(t + ds_off(ra + 16, qc)));
        const u32x2 ua = __builtin_bit_cast(u32x2, a0), ub = __builtin_bit_cast(u32x2, a1);
        const v8 a = as_vec8<T>((u32x4){ua[0], ua[1], ub[0], ub[1]});
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) acc[qt][nt] = mfma_16x16x32(a, as_vec8<T>(kq[ks][nt]), acc[qt][nt]);
      }
    float *dst = dq_acc + ((int64_t)bh * n + qs) * D + wave * (D / 4) + c;
#pragma unroll
    for (int qt = 0; qt < QT; ++qt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = qt * 16 + 4 * g + r;
        if (qs + row < n) {
#pragma unroll
          for (int nt = 0; nt < NT; ++nt) unsafeAtomicAdd(dst + (int64_t)row * D + nt * 16, acc[qt][nt][r]);
        }
      }
  };

  char *const bufs[3] = {lds_0, lds_1, lds_2};
  u32x4 pf[2][KK], dsf[2][KK]; /* P and dS of the block whose gradients are pending */

  /* Step i with buffer phase PH = i mod 3.  CHECKED steps test whether blocks
   * i+1 and i+2 exist; unchecked (interior) steps know they do. */
  auto step = [&](auto ph_tag, auto edge_tag, auto checked_tag, int i) {
    constexpr int PH = decltype(ph_tag)::value;
    constexpr bool CHECKED = decltype(checked_tag)::value;
    char *cur = bufs[PH];
    char *nx1 = bufs[(PH + 1) % 3];
    char *nx2 = bufs[(PH + 2) % 3];
    if (!CHECKED || i + 2 < nblocks) stage(nx2, i + 2);
    u32x4 pf2[2][KK], ds2[2][KK];
    if (!CHECKED || i + 1 < nblocks) {
      scores(edge_tag, nx1, i + 1, pf2, ds2);
      if constexpr (FUSED) put_ds(i + 1, ds2);
    }
    grads(cur, pf, dsf);
    if constexpr (FUSED) dq_block(i);
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) {
        pf[kt][kk] = pf2[kt][kk];
        dsf[kt][kk] = ds2[kt][kk];
      }
    wait_vmem();
    __syncthreads();
  };
  using Interior = std::integral_constant<bool, false>;
  using Edge = std::integral_constant<bool, true>;
  using P0 = std::integral_constant<int, 0>;
  using P1 = std::integral_constant<int, 1>;
  using P2 = std::integral_constant<int, 2>;
  auto checked_step = [&](auto edge_tag, int i) {
    switch (i % 3) {
      case 0: step(P0{}, edge_tag, Edge{}, i); break;
      case 1: step(P1{}, edge_tag, Edge{}, i); break;
      default: step(P2{}, edge_tag, Edge{}, i); break;
    }
  };

  if (nblocks > 0) {
    stage(lds_0, 0);
    if (nblocks > 1) stage(lds_1, 1);
  }
  /* Unconditional: the compiler then knows the K/V fragment loads are complete
   * on every path into the step loop.  Left inside the branch, its wait-count
   * pass kept them pending at the loop header and waited vmcnt(N) inside every
   * step, where the hardware count also holds the step's own tile copies (which
   * the compiler does not see), so the waits stalled on those copies. */
  wait_vmem();
  __syncthreads();
  if (nblocks > 0) scores(Edge{}, lds_0, 0, pf, dsf);
  if constexpr (FUSED) {
    if (nblocks > 0) put_ds(0, dsf);
    __syncthreads();
  }

  /* Block b is masked if it lies in the diagonal band (b < band) or runs past
   * n (b >= full).  Step i masks the softmax of block i+1. */
  const int band = CAUSAL ? (BN + BM - 1) / BM : 0;
  const int full = (n - q_start) / BM;
  int i = 0;
  /* front: steps whose next block is masked */
  for (; i < nblocks && i + 1 < band; ++i) checked_step(Edge{}, i);
  /* interior: next block unmasked, blocks i+1 and i+2 exist; peel to phase 0,
   * then whole rotations */
  const int interior_end = min(full - 1, nblocks - 2); /* last i with i+1 < full, i+2 < nblocks */
  for (; i < interior_end && (i % 3) != 0; ++i) checked_step(Interior{}, i);
  for (; i + 2 < interior_end; i += 3) {
    step(P0{}, Interior{}, Interior{}, i);
    step(P1{}, Interior{}, Interior{}, i + 1);
    step(P2{}, Interior{}, Interior{}, i + 2);
  }
  for (; i < interior_end; ++i) checked_step(Interior{}, i);
  /* tail: the rest, masked where needed */
  for (; i < nblocks; ++i) {
    if (i + 1 < full) checked_step(Interior{}, i);
    else checked_step(Edge{}, i);
  }

#pragma unroll
  for (int kt = 0; kt < 2; ++kt) {
    const int key = kw0 + kt * 16 + c;
    if (key < n) {
#pragma unroll
      for (int dt = 0; dt < D / 16; ++dt) {
        u32x2 wk, wv;
        wk[0] = pack2<T>(dk[dt][kt][0] * dk_scale, dk[dt][kt][1] * dk_scale);
        wk[1] = pack2<T>(dk[dt][kt][2] * dk_scale, dk[dt][kt][3] * dk_scale);
        wv[0] = pack2<T>(dv[dt][kt][0], dv[dt][kt][1]);
        wv[1] = pack2<T>(dv[dt][kt][2], dv[dt][kt][3]);
        *(u32x2 *)(dKg + (int64_t)key * ss + dt * 16 + 4 * g) = wk;
        *(u32x2 *)(dVg + (int64_t)key * ss + dt * 16 + 4 * g) = wv;
      }
    }
  }
}


/* ---- backward: dK, dV at two waves per SIMD -------------------------------
 * The same work split as attn_dkdv_fast (a workgroup of 4 waves owns 128 keys,
 * a wave 32 of them, and walks 32-query blocks), built for two waves per SIMD
 * so that the other workgroup's wave fills the MFMA pipe while this one runs
 * its softmax.  To fit 256 registers the wave keeps only K^T in registers;
 * the workgroup's 128 V rows are copied to LDS once and read per block.
 * Q/dO tiles are double-buffered.  LDS is addressed by 32-bit offsets whose
 * lane parts are computed once (row offsets within a tile are immediates).
 * Scheduling fences sit only between the three phases of a block (score
 * MFMAs, softmax, gradient MFMAs): without them the compiler hoists the whole
 * block's operand reads and spills; finer fences (per k-step or per two d
 * tiles) measured 2-3% slower.  The masked and the interior blocks run in
 * separate loops: a branch between the two forms inside one loop body made
 * the register allocator spill the accumulators.
 * As in attn_dkdv_fast, the dP MFMAs run on -V (negated once in LDS) and
 * start from Delta, so they deliver Delta - dP, and the kernel carries
 * -dS = P (Delta - dP) with one multiply; the arithmetic is the same as that
 * kernel's (and its fused form's), so dK and dV are bit-identical. */
struct Dkdv2wLds { static constexpr int BYTES = 128 * 128 * 2 + 2 * (2 * 32 * 128 * 2 + 32 * 8); };
template <typename T, int D, bool CAUSAL>
TM_DEV void attn_dkdv_2w(const TmAttnDkdvArgs &p, char *lds, int wg, int nwg) {
  static_assert(D == 128, "two-wave dK/dV is built for head_dim 128");
  constexpr int BN = 128, KW = 32, BM = 32;
  constexpr int KS = D / 32, DT = D / 16;
  constexpr int TILE = BM * D * 2;
  constexpr int VT = BN * D * 2;
  constexpr int STATS = 2 * TILE;
  constexpr int BUF = 2 * TILE + BM * 8;
  static_assert(VT + 2 * BUF <= Dkdv2wLds::BYTES, "LDS");
  const uint32_t vbase = lds_addr(lds), buf0 = vbase + VT, buf1 = buf0 + BUF;

  typedef typename Vec8<T>::type v8;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4, c = lane & 15;
  const int n = p.n_ctx;
  const int nkb = (n + BN - 1) / BN;
  const int logical = xcd_remap(wg, nwg);
  int bh, kb;
  if (CAUSAL) {
    causal_order(logical, nkb, p.heads, bh, kb);
  } else {
    bh = logical / nkb;
    kb = logical - bh * nkb;
  }
  const int k0 = kb * BN;
  const int kw0 = k0 + wave * KW;
  const int64_t base = (int64_t)bh * p.stride_head;
  const int64_t ss = p.stride_seq;
  const T *Qg = (const T *)p.q + base;
  const T *Kg = (const T *)p.k + base;
  const T *Vg = (const T *)p.v + base;
  const T *dOg = (const T *)p.dout + base;
  T *dKg = (T *)p.dk + base;
  T *dVg = (T *)p.dv + base;
  const float *Lg = p.lse + (int64_t)bh * p.stride_lse;
  const float *Dg = p.delta + (int64_t)bh * p.stride_lse;

  const int q_start = CAUSAL ? k0 : 0;
  const int nblocks = (n - q_start + BM - 1) / BM;

  TileCopy<T, D, BM, KEY_BOTH> qcp;  /* Q and dO rows share the lane offsets */
  TileCopy<T, D, BN, KEY_B128> vcp;
  qcp.init(ss, wave, lane);
  vcp.init(ss, wave, lane);
  auto stage = [&](uint32_t buf, int blk) {
    const int qs = q_start + blk * BM;
    qcp.copy(Qg, ss, qs, n, buf, wave);
    qcp.copy(dOg, ss, qs, n, buf + TILE, wave);
    if (wave == 0) {
      const int q = min(qs + (lane & 31), n - 1);
      lds_copy4_global(lane < 32 ? Lg + q : Dg + q, buf + STATS);
    }
  };
  vcp.copy(Vg, ss, k0, n, vbase, wave);
  if (nblocks > 0) stage(buf0, 0);

  u32x4 kf[2][KS];
#pragma unroll
  for (int kt = 0; kt < 2; ++kt) {
    const int key = min(kw0 + kt * 16 + c, n - 1);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      kf[kt][ks] = *(const u32x4 *)(Kg + (int64_t)key * ss + ks * 32 + 8 * g);
  }
  /* lane parts of the operand offsets: rows c (+16 qt or kt immediates) at
   * chunk 4 ks + g of a KEY_BOTH tile (Q, dO) or a KEY_B128 tile (V); and the
   * k-major reads of d tile dt (rows 4g + c/4, +16 immediate) */
  uint32_t qoff[KS], voff[KS], kmoff[DT];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    qoff[ks] = (uint32_t)tile_off<D>(c, ks * 4 + g);
    voff[ks] = (uint32_t)tile_off<D, KEY_B128>(c, ks * 4 + g) + (uint32_t)(wave * KW * D * 2);
  }
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
    kmoff[dt] = (uint32_t)(tile_off<D>(4 * g + (c >> 2), 2 * dt + ((c & 3) >> 1)) + ((c & 1) << 3));
  const float qk_scale = p.sm_scale * TM_LOG2E;
  f32x4 dk[DT][2], dv[DT][2];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
    dk[dt][0] = dk[dt][1] = dv[dt][0] = dv[dt][1] = (f32x4){0.f, 0.f, 0.f, 0.f};

  auto block = [&](auto edge_tag, uint32_t cur, int blk) {
    constexpr bool EDGE = decltype(edge_tag)::value;
    const int qs = q_start + blk * BM;
    f32x4 s[2][2], dp[2][2];
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
      const f32x4 dl = __builtin_bit_cast(f32x4, lds_read16(cur + STATS + 128 + (qt * 16 + 4 * g) * 4));
      s[0][qt] = s[1][qt] = (f32x4){0.f, 0.f, 0.f, 0.f};
      dp[0][qt] = dp[1][qt] = dl;
    }
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
      for (int qt = 0; qt < 2; ++qt) {
        const v8 qa = as_vec8<T>(lds_read16(cur + qoff[ks] + qt * 16 * D * 2));
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) s[kt][qt] = mfma_16x16x32(qa, as_vec8<T>(kf[kt][ks]), s[kt][qt]);
      }
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
        const v8 vb = as_vec8<T>(lds_read16(vbase + voff[ks] + kt * 16 * D * 2));
#pragma unroll
        for (int qt = 0; qt < 2; ++qt) {
          const v8 da = as_vec8<T>(lds_read16(cur + TILE + qoff[ks] + qt * 16 * D * 2));
          dp[kt][qt] = mfma_16x16x32(da, vb, dp[kt][qt]);
        }
      }
    }
    TM_FENCE();
    u32x4 pf[2], dsf[2];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      const int key = kw0 + kt * 16 + c;
      float pr[2][4], ds[2][4];
#pragma unroll
      for (int qt = 0; qt < 2; ++qt) {
        const f32x4 lse = __builtin_bit_cast(f32x4, lds_read16(cur + STATS + (qt * 16 + 4 * g) * 4));
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float x = __builtin_fmaf(s[kt][qt][r], qk_scale, -lse[r]);
          if (EDGE) {
            const int qi = qs + qt * 16 + 4 * g + r;
            x = (qi >= n || (CAUSAL && qi < key)) ? TM_NEG_INF : x;
          }
          pr[qt][r] = fast_exp2(x);
          ds[qt][r] = pr[qt][r] * dp[kt][qt][r]; /* -dS */
        }
      }
      pf[kt] = (u32x4){pack2<T>(pr[0][0], pr[0][1]), pack2<T>(pr[0][2], pr[0][3]),
                       pack2<T>(pr[1][0], pr[1][1]), pack2<T>(pr[1][2], pr[1][3])};
      dsf[kt] = (u32x4){pack2<T>(ds[0][0], ds[0][1]), pack2<T>(ds[0][2], ds[0][3]),
                        pack2<T>(ds[1][0], ds[1][1]), pack2<T>(ds[1][2], ds[1][3])};
    }
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      const v8 doa = as_vec8<T>(lds_read_kmajor(cur + TILE + kmoff[dt], 0, 16 * D * 2));
      const v8 qa = as_vec8<T>(lds_read_kmajor(cur + kmoff[dt], 0, 16 * D * 2));
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
        dv[dt][kt] = mfma_16x16x32(doa, as_vec8<T>(pf[kt]), dv[dt][kt]);
        dk[dt][kt] = mfma_16x16x32(qa, as_vec8<T>(dsf[kt]), dk[dt][kt]);
      }
    }
    TM_FENCE();
  };
  using Interior = std::integral_constant<bool, false>;
  using Edge = std::integral_constant<bool, true>;

  wait_vmem();
  __syncthreads();
  /* -V in LDS: every sign bit flipped once (exact) */
#pragma unroll
  for (int e = 0; e < VT / (256 * 16); ++e) {
    const uint32_t a = vbase + (uint32_t)(e * 256 + tid) * 16;
    const u32x4 x = lds_read16(a) ^ (u32x4){0x80008000u, 0x80008000u, 0x80008000u, 0x80008000u};
    *(__attribute__((address_space(3))) u32x4 *)(lds_char_t *)(uintptr_t)a = x;
  }
  __syncthreads();
  const int band = CAUSAL ? BN / BM : 0;
  const int full = (n - q_start) / BM;
  /* block i reads buffer i mod 2 while block i+1 is copied into the other;
   * the masked blocks (the diagonal band, a ragged end) and the interior run
   * in loops of their own */
  auto step = [&](auto edge_tag, int i) {
    const uint32_t cur = (i & 1) ? buf1 : buf0, nxt = (i & 1) ? buf0 : buf1;
    if (i + 1 < nblocks) stage(nxt, i + 1);
    /* causal: a block whose every query precedes the wave's first key adds
     * exact zeros; the wave skips its arithmetic (not its copies and barrier),
     * which changes no bit of dK or dV (0.5-1% faster at config 5) */
    if (!CAUSAL || q_start + (i + 1) * BM > kw0) block(edge_tag, cur, i);
    wait_vmem();
    __syncthreads();
  };
  const int interior_end = min(full, nblocks);
  int i = 0;
  for (; i < nblocks && i < band; ++i) step(Edge{}, i);
  for (; i < interior_end; ++i) step(Interior{}, i);
  for (; i < nblocks; ++i) step(Edge{}, i);

  const float dk_scale = -p.sm_scale; /* dk holds -dK / sm_scale */
#pragma unroll
  for (int kt = 0; kt < 2; ++kt) {
    const int key = kw0 + kt * 16 + c;
    if (key < n) {
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        u32x2 wk, wv;
        wk[0] = pack2<T>(dk[dt][kt][0] * dk_scale, dk[dt][kt][1] * dk_scale);
        wk[1] = pack2<T>(dk[dt][kt][2] * dk_scale, dk[dt][kt][3] * dk_scale);
        wv[0] = pack2<T>(dv[dt][kt][0], dv[dt][kt][1]);
        wv[1] = pack2<T>(dv[dt][kt][2], dv[dt][kt][3]);
        *(u32x2 *)(dKg + (int64_t)key * ss + dt * 16 + 4 * g) = wk;
        *(u32x2 *)(dVg + (int64_t)key * ss + dt * 16 + 4 * g) = wv;
      }
    }
  }
}


#define TM_BWD_FAST(T, TN, D, CAUSAL, CN)                                                     \
  extern "C" __global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void  \
  tm_attn_dq_fast_##TN##_d##D##CN(TmAttnDqArgs p) {                                           \
    __shared__ __align__(1024) char lds[DqLds<D>::BYTES];                                     \
    attn_dq_fast<T, D, CAUSAL>(p, lds, blockIdx.x, gridDim.x);                                \
  }                                                                                           \
  TM_DKDV_FAST_##D(T, TN, CAUSAL, CN)
/* head_dim 128: the two-waves-per-SIMD kernel (0.99-1.03 ms at B4 H32 S4096
 * causal against 1.11-1.16 ms for attn_dkdv_fast at one wave per SIMD, whose
 * dK, dV accumulators plus K^T and V^T fragments need more than 256
 * registers); head_dim 64: attn_dkdv_fast, one wave per SIMD */
#define TM_DKDV_FAST_128(T, TN, CAUSAL, CN)                                                   \
  extern "C" __global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void  \
  tm_attn_dkdv_fast_##TN##_d128##CN(TmAttnDkdvArgs p) {                                       \
    __shared__ __align__(1024) char lds[Dkdv2wLds::BYTES];                                    \
    attn_dkdv_2w<T, 128, CAUSAL>(p, lds, blockIdx.x, gridDim.x);                              \
  }
#define TM_DKDV_FAST_64(T, TN, CAUSAL, CN)                                                    \
  extern "C" __global__ __launch_bounds__(256) void tm_attn_dkdv_fast_##TN##_d64##CN(         \
      TmAttnDkdvArgs p) {                                                                     \
    attn_dkdv_fast<T, 64, CAUSAL>(p);                                                         \
  }
/* Single-pass backward with atomic dQ (opt-in: bwd=atomic): the dK/dV
 * kernel plus dQ = dS K per query block, and the passes around it. */
#define TM_BWD_FUSED(T, TN, D, CAUSAL, CN)                                                    \
  extern "C" __global__ __launch_bounds__(256) void tm_attn_fused_fast_##TN##_d##D##CN(       \
      TmAttnFusedArgs p) {                                                                    \
    attn_dkdv_fast<T, D, CAUSAL, true>(p.kv, p.dq_acc);                                       \
  }
#define TM_BWD_FAST_ALL(T, TN)           \
  TM_BWD_FUSED(T, TN, 64, false, )       \
  TM_BWD_FUSED(T, TN, 64, true, _causal) \
  TM_BWD_FUSED(T, TN, 128, false, )      \
  TM_BWD_FUSED(T, TN, 128, true, _causal) \
  TM_BWD_FAST(T, TN, 64, false, )        \
  TM_BWD_FAST(T, TN, 64, true, _causal)  \
  TM_BWD_FAST(T, TN, 128, false, )       \
  TM_BWD_FAST(T, TN, 128, true, _causal)
TM_BWD_FAST_ALL(bf16_t, bf16)
TM_BWD_FAST_ALL(f16_t, f16)

#define TM_FWD_FAST(T, TN, D, CAUSAL, CN)                                                     \
  extern "C" __global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void  \
  tm_attn_fwd_fast_##TN##_d##D##CN(TmAttnFwdArgs p) {                                         \
    attn_fwd_fast<T, D, CAUSAL>(p);                                                           \
  }
#define TM_FWD_FAST_ALL(T, TN)           \
  TM_FWD_FAST(T, TN, 64, false, )        \
  TM_FWD_FAST(T, TN, 64, true, _causal)  \
  TM_FWD_FAST(T, TN, 128, false, )       \
  TM_FWD_FAST(T, TN, 128, true, _causal)
TM_FWD_FAST_ALL(bf16_t, bf16)
TM_FWD_FAST_ALL(f16_t, f16)

/* dq_acc = 0 (count a multiple of 4), before the fused backward */
extern "C" __global__ __launch_bounds__(256) void tm_attn_dq_acc_zero(TmAttnDqAccArgs p) {
  const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (i < p.count) *(f32x4 *)(p.acc + i) = (f32x4){0.f, 0.f, 0.f, 0.f};
}

/* dq[bh, q, :] = sm_scale * dq_acc[bh, q, :] in the element type, after it:
 * D / 8 lanes per row, 8 elements (one 16-byte store) per lane */
template <typename T, int D>
TM_DEV void attn_dq_convert(const TmAttnDqAccArgs &p) {
  constexpr int LPR = D / 8, RPB = 256 / LPR;
  const int64_t row = (int64_t)blockIdx.x * RPB + threadIdx.x / LPR;
  if (row >= (int64_t)p.heads * p.n_ctx) return;
  const int col = (threadIdx.x % LPR) * 8;
  const int bh = (int)(row / p.n_ctx), q = (int)(row - (int64_t)bh * p.n_ctx);
  const f32x4 a = *(const f32x4 *)(p.acc + row * D + col);
  const f32x4 b = *(const f32x4 *)(p.acc + row * D + col + 4);
  const float s = p.sm_scale;
  *(u32x4 *)((T *)p.dq + (int64_t)bh * p.stride_head + (int64_t)q * p.stride_seq + col) =
      (u32x4){pack2<T>(a[0] * s, a[1] * s), pack2<T>(a[2] * s, a[3] * s), pack2<T>(b[0] * s, b[1] * s),
              pack2<T>(b[2] * s, b[3] * s)};
}
#define TM_DQ_CONVERT(T, TN, D) \
  extern "C" __global__ __launch_bounds__(256) void tm_attn_dq_convert_##TN##_d##D(TmAttnDqAccArgs p) { \
    attn_dq_convert<T, D>(p); \
  }
TM_DQ_CONVERT(bf16_t, bf16, 64)
TM_DQ_CONVERT(bf16_t, bf16, 128)
TM_DQ_CONVERT(f16_t, f16, 64)
TM_DQ_CONVERT(f16_t, f16, 128)
