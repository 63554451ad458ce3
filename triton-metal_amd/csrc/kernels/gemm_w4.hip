/*
 * gfx950 GEMM for large whole-tile 16-bit problems: C = A @ B, A [M, K] and
 * B [K, N] row-major, or one of them stored transposed (B as [N, K]: the
 * x @ W^T layout; A as [K, M]: the dY^T X layout), M and N multiples of 256,
 * K a multiple of 64; f32
 * accumulation, output rounded to the element type (the reference's
 * matmul_kernel semantics, Sources/TritonMetalBench/GEMMKernel.swift:28-174),
 * optionally with the SAE encoder's bias + ReLU epilogue
 * (Sources/TritonMetalMLX/SAEEncoder.swift:1-20).
 *
 * One 256-thread workgroup (4 waves, 2 x 2) per 256 x 256 tile of C, one
 * workgroup per CU; each wave owns a 128 x 128 sub-tile as 4 x 4
 * accumulators of v_mfma_f32_32x32x16_{bf16,f16} (256 accumulator registers:
 * the kernel is built for one wave per SIMD and 512 registers).  Against the
 * 8-wave kernel of gemm_fast.hip (128 x 64 per wave, 16x16x32) this reads a
 * third less LDS per K step (each wave's operands cover twice the columns),
 * and the 32x32x16 instruction issues closer to the MFMA peak.
 *
 * Per K step of 64: A [256 x 64] and B [64 x 256] tiles are copied HBM -> LDS
 * by buffer_load_dwordx4 ... lds (double buffered, 128 KB), through buffer
 * resources rebased at each step's first element with scalar arithmetic, the
 * lane parts of the offsets fixed for the whole loop, so a copy costs no
 * vector instruction.  A wave's 16 copy instructions of a step are spread
 * one every two MFMAs from the barrier two steps earlier (see the loop).  The
 * step's four k-substeps of 16 read their operands one substep ahead of the
 * MFMAs (two register sets), and the first substep of the next step is read
 * right after the step's barrier, ahead of the current step's last 16 MFMAs,
 * which hide its LDS latency.  C goes out through LDS in whole row segments.
 *
 * Measured at 8192^3 on one MI355X (alternating runs, TFLOP/s): this kernel
 * 1311-1342 against 1291-1341 for gemm_fast.hip's 8-wave kernel, the SAE
 * encoder shape (8192 x 2048 -> 16384) 1166 against 1080, and short K
 * (4096^2 x 64 / 128) 11.6 / 12.7 us against 14.1 / 15.3; B transposed
 * 1315-1321 against 1289-1298, A transposed 1297-1304 against 1218-1222.
 * Without its copies
 * (timing only) it runs 1690 (constant operands): one wave per SIMD cannot
 * hide the issue of the copy instructions behind another wave's MFMAs.
 *
 * Operands (lane l, h = l / 32): the MFMA's first operand is a B fragment
 * (C column n0 + (l % 32), k = 8h .. 8h + 7), the second an A fragment (C row
 * m0 + (l % 32), the same k).  A K-contiguous operand (A row-major, B
 * transposed) keeps its stored rows in a [256][64] tile of 128-byte rows and
 * gives a fragment by one ds_read_b128; the other kind a [64][256] tile of
 * 512-byte rows and two ds_read_b64_tr_b16 (W4Operand).  The product is then
 * C^T: a lane holds 4 consecutive columns of one row per group of 4
 * accumulator floats.  Tiles keep gemm_fast.hip's layouts with XOR keys for
 * this kernel's 32-row reads.
 */
#include "common.h"

#include <type_traits>

namespace {

template <typename T> struct W4Vec8;
template <> struct W4Vec8<bf16_t> { typedef bf16x8 type; };
template <> struct W4Vec8<f16_t> { typedef f16x8 type; };

typedef short w4s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) char w4lds_t;

constexpr int W4_TILE = 256, W4_BK = 64;
constexpr int W4_A_BYTES = W4_TILE * W4_BK * 2; /* 32 KB */
constexpr int W4_B_BYTES = W4_BK * W4_TILE * 2; /* 32 KB */
constexpr int W4_STAGE = W4_A_BYTES + W4_B_BYTES;

TM_DEV int w4_xcd_remap(int wg, int nwg) {
  const int q = nwg >> 3, r = nwg & 7;
  const int xcd = wg & 7, slot = wg >> 3;
  return (xcd < r ? xcd * (q + 1) : r * (q + 1) + (xcd - r) * q) + slot;
}

/* A tile [256 rows][64 k], 128-byte rows, chunk c of row r at
 * c ^ ((r >> 1) & 7).  A ds_read_b128 of 32 lanes reads 32 consecutive rows
 * at one chunk: two rows share each 256-byte bank line, so the row's parity
 * and the key give 16 distinct 16-byte slots (the row & 7 key of
 * gemm_fast.hip, made for 16 rows, gives 8 here: 2-way conflicts). */
TM_DEV int w4_a_swz(int row) { return (row >> 1) & 7; }
TM_DEV int w4_a_off(int row, int chunk) { return row * 128 + ((chunk ^ w4_a_swz(row)) << 4); }
/* B tile [64 k][256 n], 512-byte rows.  A transposed read of 32 lanes
 * touches 4 consecutive rows at 4 consecutive chunks (two 16-lane groups
 * side by side); the key 4 (row & 3) puts the 4 rows' chunks in 4 disjoint
 * blocks of the 256-byte bank width.  (gemm_fast.hip's key, made for 8 rows
 * at one chunk pair, leaves these reads 2-way conflicted.) */
TM_DEV int w4_b_swz(int row) { return (row & 3) << 2; }
TM_DEV int w4_b_off(int row, int chunk) { return row * 512 + ((chunk ^ w4_b_swz(row)) << 4); }

/* 16 bytes per lane to LDS at M0 + 16 * lane from buffer `rsrc` at byte
 * offset voffset + soffset.  Issued from inline assembly so the compiler does
 * not serialise LDS reads behind it (see common.h); the caller waits vmcnt(0)
 * and barriers before any wave reads the tile.  s_nop 4: the wait states a
 * VALU-written SGPR operand needs before a memory instruction reads it. */
TM_DEV void w4_copy16(u32x4 rsrc, int voffset, int soffset, uint32_t lds_base) {
  asm volatile("s_nop 4\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
               :: "{m0}"(lds_base), "v"(voffset), "s"(rsrc), "s"(soffset) : "memory");
}

TM_DEV u32x4 w4_rsrc(const void *base, uint32_t bytes) {
  const uint64_t a = (uint64_t)base;
  return (u32x4){(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)a),
                 (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(a >> 32)) & 0xffffu,
                 bytes, 0x00020000u};
}

TM_DEV u32x4 w4_lds_read16(uint32_t addr) {
  return *(const __attribute__((address_space(3))) u32x4 *)(w4lds_t *)(uintptr_t)addr;
}
TM_DEV u32x4 w4_lds_read_tr(uint32_t addr_a, uint32_t addr_b) {
  const w4s16x4 a = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) w4s16x4 *)(w4lds_t *)(uintptr_t)addr_a);
  const w4s16x4 b = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) w4s16x4 *)(w4lds_t *)(uintptr_t)addr_b);
  const u32x2 ua = __builtin_bit_cast(u32x2, a), ub = __builtin_bit_cast(u32x2, b);
  return (u32x4){ua[0], ua[1], ub[0], ub[1]};
}

template <typename T>
TM_DEV uint32_t w4_pack2(float lo, float hi) {
  typedef float f2 __attribute__((ext_vector_type(2)));
  typedef T t2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f2){lo, hi}, t2));
}

#define W4_FENCE() __builtin_amdgcn_sched_barrier(0)

/* One operand's tiles.  KC (K-contiguous: A row-major, or B stored
 * transposed): [256 rows][64 k], 128-byte rows, keyed by w4_a_swz, copied 8
 * rows per instruction and read by ds_read_b128.  MC (M- or N-contiguous: B
 * row-major, or A stored transposed): [64 k][256 columns], 512-byte rows,
 * keyed by w4_b_swz, copied 2 rows per instruction and read by two
 * ds_read_b64_tr_b16.  Either way a fragment f (0..3) of substep s (k 16s ..
 * 16s + 15) gives lane l the 8 values k = 16s + 8h .. + 7 (h = l / 32) of
 * tile row or column half * 128 + 32 f + l % 32, the operand layout of
 * v_mfma_f32_32x32x16. */
template <typename T, bool KC>
struct W4Operand {
  const T *base;  /* the tile's origin at k = 0 */
  int64_t ld;     /* elements between the tile's stored rows */
  uint32_t bytes; /* a step's buffer range */
  int voff[2];    /* copy lane offsets by instruction parity */
  uint32_t rd[4]; /* read lane offsets: per substep (KC) or per fragment (MC) */
  TM_DEV void init(const T *origin, int64_t stride, int lane, int half) {
    base = origin;
    ld = stride;
    if constexpr (KC) {
      bytes = (uint32_t)((int64_t)(W4_TILE - 1) * ld * 2 + W4_BK * 2);
#pragma unroll
      for (int par = 0; par < 2; ++par)
        voff[par] = (lane >> 3) * (int)ld * 2 + (((lane & 7) ^ w4_a_swz(8 * par + (lane >> 3))) << 4);
      const int row = half * 128 + (lane & 31), h = lane >> 5;
#pragma unroll
      for (int s = 0; s < 4; ++s) rd[s] = (uint32_t)w4_a_off(row, 2 * s + h);
    } else {
      bytes = (uint32_t)((int64_t)(W4_BK - 1) * ld * 2 + W4_TILE * 2);
#pragma unroll
      for (int par = 0; par < 2; ++par)
        voff[par] = (lane >> 5) * (int)ld * 2 +
                    (((lane & 31) ^ w4_b_swz(2 * par + (lane >> 5))) << 4);
      const int q = lane >> 4, i = lane & 15;
      const int krow = 8 * (q >> 1) + (i >> 2);
#pragma unroll
      for (int f = 0; f < 4; ++f) {
        const int col = half * 128 + 32 * f + 16 * (q & 1) + 4 * (i & 3);
        rd[f] = (uint32_t)(w4_b_off(krow, col >> 3) + (((col >> 2) & 1) << 3));
      }
    }
  }
  TM_DEV u32x4 rsrc(int kb) const {
    return w4_rsrc(KC ? base + kb * W4_BK : base + (int64_t)kb * W4_BK * ld, bytes);
  }
  /* copy instruction t (0..31) of a step's tile into `region` */
  TM_DEV void copy(const u32x4 &rs, int t, uint32_t region) const {
    w4_copy16(rs, voff[t & 1], t * (KC ? 8 : 2) * (int)ld * 2, region + t * 1024);
  }
  TM_DEV u32x4 read(uint32_t region, int s, int f) const {
    if constexpr (KC) return w4_lds_read16(region + rd[s] + f * 32 * 128);
    const uint32_t ad = region + rd[f] + s * 16 * 512;
    return w4_lds_read_tr(ad, ad + 4 * 512);
  }
};

/* AK: A row-major [M, K] (else stored transposed, element (m, k) at
 * k * stride_ak + m); BK: B stored transposed, element (k, n) at
 * n * stride_bn + k (else row-major [K, N]). */
template <typename T, int EPI, bool AK, bool BK>
TM_DEV void gemm_w4(const TmGemmArgs &p) {
  typedef typename W4Vec8<T>::type v8;
  __shared__ __align__(1024) char lds[2 * W4_STAGE];
  const uint32_t st0 = (uint32_t)(uintptr_t)(w4lds_t *)lds;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;

  /* tile order: each XCD a contiguous range, walked 4 tile rows at a time
   * (measured against 2, 8 and 16 on one box, alternating runs, TFLOP/s:
   * 8192^3 1309 / 1271-1275 / 1299 / 1275-1277, SAE 1171-1172 / 1176-1177 /
   * 1150-1152 / 1127-1128, 4096^3 1254-1255 / 1251-1253 / 1241-1243 / 1248) */
  const int mt = p.m / W4_TILE, nt = p.n / W4_TILE;
  const int logical = w4_xcd_remap(blockIdx.x, gridDim.x);
  constexpr int GROUP = 4;
  const int per_group = GROUP * nt;
  const int group = logical / per_group;
  const int first_m = group * GROUP;
  const int gm = min(mt - first_m, GROUP);
  const int in_group = logical - group * per_group;
  const int m0 = (first_m + in_group % gm) * W4_TILE, n0 = (in_group / gm) * W4_TILE;

  const int64_t ldc = p.scm;
  W4Operand<T, AK> opa;
  W4Operand<T, BK> opb;
  opa.init(AK ? (const T *)p.a + (int64_t)m0 * p.sam : (const T *)p.a + m0, AK ? p.sam : p.sak,
           lane, wm);
  opb.init(BK ? (const T *)p.b + (int64_t)n0 * p.sbn : (const T *)p.b + n0, BK ? p.sbn : p.sbk,
           lane, wn);

  /* copies: each tile is 32 instructions of 1 KB; wave w issues instructions
   * 8w .. 8w + 7 of each: copy i of 16 is A's (i < 8) or B's */
  auto copy = [&](uint32_t stage, int i, const u32x4 &ra, const u32x4 &rb) {
    const int t = wave * 8 + (i & 7);
    if (i < 8) opa.copy(ra, t, stage);
    else opb.copy(rb, t, stage + W4_A_BYTES);
  };
  auto read_ops = [&](uint32_t stage, int s, u32x4 (&af)[4], u32x4 (&bf)[4]) {
#pragma unroll
    for (int f = 0; f < 4; ++f) bf[f] = opb.read(stage + W4_A_BYTES, s, f);
#pragma unroll
    for (int f = 0; f < 4; ++f) af[f] = opa.read(stage, s, f);
  };

  f32x16 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;
  auto mfmas = [&](const u32x4 (&af)[4], const u32x4 (&bf)[4], auto between) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        acc[i][j] = mfma_32x32x16(__builtin_bit_cast(v8, bf[j]), __builtin_bit_cast(v8, af[i]),
                                  acc[i][j]);
        between(j * 4 + i);
        W4_FENCE();
      }
  };
  auto nothing = [](int) {};

  const int ksteps = p.k / W4_BK;
  /* SAE epilogue: this lane's 16 bias words, loaded before the K loop (loaded
   * in the epilogue, each waited for its load: SAE 1173-1180 against
   * 1190-1194 TFLOP/s on one box) */
  u32x2 biasw[4][4];
  if constexpr (EPI == EPI_BIAS_RELU) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        biasw[j][e] = *(const u32x2 *)((const T *)p.bias + n0 + wn * 128 + 32 * j + 8 * e + 4 * (lane >> 5));
  }
  /* Copy x (0..15) of step s is issued after MFMA 2x of a 64-MFMA window
   * that opens at the barrier ending step s - 2: window MFMAs 0-15 are the
   * last substep of step s - 2 (issued after that barrier, which ends every
   * read of the buffer the copies overwrite), 16-63 substeps 0-2 of step
   * s - 1, whose barrier waits for them.  So a copy has at least a step's
   * MFMAs to land, and the four waves' 64 copies of a step are spread over
   * 32 MFMAs (measured at 8192^3 against the other placements on one box:
   * all 16 in the first 16 MFMAs of step s - 1, 1249 TFLOP/s; one every two
   * MFMAs of the window, 1342; every three, 1286; every four, 1190).
   * Copies 0-7 of step 1 (window MFMAs 0-15) go out in the prologue. */
  constexpr int SPREAD = 2, PRE1 = 16 / SPREAD;
  auto copy_step = [&](uint32_t stage, int kb, int x) { copy(stage, x, opa.rsrc(kb), opb.rsrc(kb)); };
#pragma unroll
  for (int x = 0; x < 16; ++x) copy_step(st0, 0, x);
  if (ksteps > 1) {
#pragma unroll
    for (int x = 0; x < PRE1; ++x) copy_step(st0 + W4_STAGE, 1, x);
    /* vmcnt(PRE1): step 0's copies (issued first) have landed */
    __builtin_amdgcn_s_waitcnt(0x0F70 | PRE1);
  } else {
    __builtin_amdgcn_s_waitcnt(0x0F70); /* vmcnt(0) */
  }
  __syncthreads();
  u32x4 a0[4], b0[4], a1[4], b1[4];
  read_ops(st0, 0, a0, b0);
  /* One K step.  NEXT: step kb + 1 exists (wait for its tile, read its first
   * substep after the barrier); NEXT2: step kb + 2 exists.  Separate
   * instantiations keep the loop body free of branches (a branch around the
   * MFMA groups made the register allocator shuffle the accumulators). */
  auto kstep = [&](auto next_tag, auto next2_tag, int kb) {
    constexpr bool NEXT = decltype(next_tag)::value;
    constexpr bool NEXT2 = decltype(next2_tag)::value;
    const uint32_t cur = st0 + (uint32_t)((kb & 1) * W4_STAGE);
    const uint32_t nxt = st0 + (uint32_t)(((kb + 1) & 1) * W4_STAGE);
    const u32x4 ra = opa.rsrc(kb + 1), rb = opb.rsrc(kb + 1);
    /* step kb + 1's copies at window MFMAs 16-63 */
    auto copies_in = [&](int sub) {
      return [&, sub](int at) {
        if constexpr (NEXT) {
          const int pos = 16 + sub * 16 + at;
          if (pos % SPREAD == 0 && pos / SPREAD < 16) copy(nxt, pos / SPREAD, ra, rb);
        }
      };
    };
    read_ops(cur, 1, a1, b1);
    W4_FENCE();
    mfmas(a0, b0, copies_in(0));
    read_ops(cur, 2, a0, b0);
    W4_FENCE();
    mfmas(a1, b1, copies_in(1));
    read_ops(cur, 3, a1, b1);
    W4_FENCE();
    mfmas(a0, b0, copies_in(2));
    if constexpr (NEXT) {
      __builtin_amdgcn_s_waitcnt(0x0F70); /* this wave's copies of step kb + 1 */
      __syncthreads();                    /* everyone's; every read of `cur` issued */
      read_ops(nxt, 0, a0, b0);
      W4_FENCE();
    }
    if constexpr (NEXT2) {
      /* step kb + 2's copies at window MFMAs 0-15, into `cur` */
      const u32x4 ra2 = opa.rsrc(kb + 2), rb2 = opb.rsrc(kb + 2);
      mfmas(a1, b1, [&](int at) {
        if (at % SPREAD == 0) copy(cur, at / SPREAD, ra2, rb2);
      });
    } else {
      mfmas(a1, b1, nothing);
    }
  };
  using Y = std::true_type;
  using N = std::false_type;
  int kb = 0;
  for (; kb + 2 < ksteps; ++kb) kstep(Y{}, Y{}, kb);
  if (kb + 1 < ksteps) kstep(Y{}, N{}, kb++);
  kstep(N{}, N{}, kb);

  /* acc[i][j] = C^T tile: float 4e + r of a lane is C[row][col] with
   * row = wm*128 + 32i + l%32, col = wn*128 + 32j + 8e + 4h + r (tile
   * relative).  Stored through LDS: each wave writes its 128 x 128 sub-tile
   * (rounded, 32 KB) into its own quarter of the stage buffers, then reads it
   * back 16 bytes per lane along rows, so every global store covers whole
   * 256-byte row segments (stored straight from the accumulators, a store
   * instruction wrote 16 bytes in each of 32 rows, and the kernel's fixed
   * cost doubled).  Chunk c of sub-tile row r sits at c ^ (r & 15). */
  const int h = lane >> 5;
  /* every copy has landed on every feasible path already; the wait makes
   * that visible on every path of the control-flow graph */
  __builtin_amdgcn_s_waitcnt(0x0F70);
  __syncthreads(); /* every wave's last operand reads are done */
  const uint32_t mine = st0 + (uint32_t)(wave * 128 * 256);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float bias[4] = {0.f, 0.f, 0.f, 0.f};
      if constexpr (EPI == EPI_BIAS_RELU) {
        const u32x2 bw = biasw[j][e];
        const T *bt = (const T *)&bw;
#pragma unroll
        for (int r = 0; r < 4; ++r) bias[r] = to_f32(bt[r]);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float v[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          v[r] = acc[i][j][4 * e + r];
          if constexpr (EPI == EPI_BIAS_RELU) v[r] = fmaxf(v[r] + bias[r], 0.f);
        }
        u32x2 w;
        w[0] = w4_pack2<T>(v[0], v[1]);
        w[1] = w4_pack2<T>(v[2], v[3]);
        const int row = 32 * i + (lane & 31);
        const uint32_t addr = mine + (uint32_t)(row * 256 + (((4 * j + e) ^ (row & 15)) << 4) + 8 * h);
        *(__attribute__((address_space(3))) u32x2 *)(w4lds_t *)(uintptr_t)addr = w;
      }
    }
  }
  T *C = (T *)p.c + (int64_t)(m0 + wm * 128) * ldc + n0 + wn * 128;
#pragma unroll
  for (int t = 0; t < 32; ++t) {
    const int row = 4 * t + (lane >> 4), chunk = lane & 15;
    const u32x4 x = w4_lds_read16(mine + (uint32_t)(row * 256 + ((chunk ^ (row & 15)) << 4)));
    *(u32x4 *)(C + (int64_t)row * ldc + 8 * chunk) = x;
  }
}

}  // namespace

#define TM_GEMM_W4(NAME, T, EPI, AK, BK)                                                       \
  extern "C" __global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1))) void \
  NAME(TmGemmArgs p) {                                                                         \
    gemm_w4<T, EPI, AK, BK>(p);                                                                \
  }
TM_GEMM_W4(tm_gemm_w4_bf16, bf16_t, EPI_NONE, true, false)
TM_GEMM_W4(tm_gemm_w4_f16, f16_t, EPI_NONE, true, false)
TM_GEMM_W4(tm_gemm_w4_nt_bf16, bf16_t, EPI_NONE, true, true)
TM_GEMM_W4(tm_gemm_w4_nt_f16, f16_t, EPI_NONE, true, true)
TM_GEMM_W4(tm_gemm_w4_tn_bf16, bf16_t, EPI_NONE, false, false)
TM_GEMM_W4(tm_gemm_w4_tn_f16, f16_t, EPI_NONE, false, false)
TM_GEMM_W4(tm_sae_w4_bf16, bf16_t, EPI_BIAS_RELU, true, false)
TM_GEMM_W4(tm_sae_w4_f16, f16_t, EPI_BIAS_RELU, true, false)
