/*
 * Generic gfx950 kernels for the dense hot path: every element type the
 * reference supports (f32, f16, bf16), arbitrary strides, ragged shapes, any
 * head dimension up to 128, causal or not.  They stage tiles through LDS as
 * f32 and contract on v_mfma_f32_16x16x4_f32, which multiplies exactly for all
 * three element types, so one code path serves them all.  The hot shapes run
 * on the specialised kernels in gemm_fast.hip / attn_fast.hip; these cover
 * everything else with the reference's numerics:
 *   - f32 accumulation everywhere (GEMMKernel.swift:46, AttentionKernel.swift:59-65);
 *   - P and dS rounded to the element type before the dot they feed
 *     (AttentionKernel.swift:59-65, AttentionBackwardKernel.swift:155-160, :357-369);
 *   - exp2 with sm_scale folded into log2(e) (AttentionKernel.swift:79-80);
 *   - the log2-unit row statistic L = m + log2(l) (AttentionKernel.swift:33-39).
 */
#include "common.h"

#define TM_NEG_INF (-__builtin_inff())

/* ---------------------------------------------------------------------------
 * matmul_kernel: C = A @ B, masked in M, N and K, f32 accumulation, output in
 * the element type (GEMMKernel.swift:28-174; matmul.py:20-44).
 * 64x64 output tile per 256-thread workgroup, 4 waves in 2x2, 32x32 per wave.
 * K advances 32 at a time; the next k-slice's global loads are issued into
 * registers before the current slice's MFMAs, so their latency overlaps the
 * contraction (one barrier-separated LDS store per slice).
 * ------------------------------------------------------------------------- */
template <typename T, int EPI>
TM_DEV void gemm_generic(const TmGemmArgs &p) {
  constexpr int BM = 64, BN = 64, BK = 32;
  constexpr int PER = BM * BK / 256; /* elements of A (and of B) per thread per slice */
  __shared__ float As[BM][BK + 1];
  __shared__ float Bs[BK][BN + 4];
  const T *A = (const T *)p.a;
  const T *B = (const T *)p.b;
  T *C = (T *)p.c;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, c = lane & 15;
  const int wm = wave >> 1, wn = wave & 1;
  const int m0 = blockIdx.x * BM, n0 = blockIdx.y * BN;

  f32x4 acc[2][2];
  for (int i = 0; i < 2; ++i)
    for (int j = 0; j < 2; ++j) acc[i][j] = (f32x4){0.f, 0.f, 0.f, 0.f};

  /* element e = tid + 256 * i of a slice: A row e / BK, column e % BK (k
   * fastest, so a wave reads runs along A's rows); B row e / BN, column e % BN */
  float ra[PER], rb[PER];
  auto load = [&](int k0) {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int e = tid + 256 * i;
      const int gm = m0 + e / BK, gk = k0 + e % BK;
      ra[i] = (gm < p.m && gk < p.k) ? to_f32(A[(int64_t)gm * p.sam + (int64_t)gk * p.sak]) : 0.f;
      const int kk = k0 + e / BN, gn = n0 + e % BN;
      rb[i] = (kk < p.k && gn < p.n) ? to_f32(B[(int64_t)kk * p.sbk + (int64_t)gn * p.sbn]) : 0.f;
    }
  };
  auto store = [&]() {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int e = tid + 256 * i;
      As[e / BK][e % BK] = ra[i];
      Bs[e / BN][e % BN] = rb[i];
    }
  };

  if (p.k > 0) load(0);
  for (int k0 = 0; k0 < p.k; k0 += BK) {
    store();
    __syncthreads();
    if (k0 + BK < p.k) load(k0 + BK);
#pragma unroll
    for (int kk = 0; kk < BK; kk += 4) {
      float a[2], b[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) a[i] = As[wm * 32 + i * 16 + c][kk + g];
#pragma unroll
      for (int j = 0; j < 2; ++j) b[j] = Bs[kk + g][wn * 32 + j * 16 + c];
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = mfma_f32_16x16x4(a[i], b[j], acc[i][j]);
    }
    __syncthreads();
  }

  /* the bias of this lane's two columns, loaded before any store to C */
  float bias[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int col = n0 + wn * 32 + j * 16 + c;
    bias[j] = (EPI == EPI_BIAS_RELU && col < p.n) ? to_f32(((const T *)p.bias)[col]) : 0.f;
  }
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = m0 + wm * 32 + i * 16 + 4 * g + r;
        const int col = n0 + wn * 32 + j * 16 + c;
        const float v = EPI == EPI_BIAS_RELU ? fmaxf(acc[i][j][r] + bias[j], 0.f) : acc[i][j][r];
        if (row < p.m && col < p.n) C[(int64_t)row * p.scm + (int64_t)col * p.scn] = from_f32<T>(v);
      }
}

/* Two [ROWS x DP] row tiles of one head (rows r0 .., columns < D, zeros
 * outside the sequence and the head dimension) staged HBM -> registers -> LDS
 * as f32 with row stride DP + 1.  The attention loops call load() for the
 * next block right after the current block is in LDS, so the global reads'
 * latency overlaps the current block's MFMAs; store() writes them out after
 * the barrier that ends the current block. */
template <typename T, int ROWS, int DP>
struct TileStager {
  static constexpr int PER = ROWS * DP / 256;
  static_assert(ROWS * DP % 1024 == 0, "four consecutive elements per thread");
  /* DP <= 64: a thread's elements come in runs of four consecutive ones,
   * e = 4 (tid + 256 (i / 4)) + i % 4, loaded together when they can be
   * (measured: fp32 D = 64 backward 5% faster; at DP = 128 the forward ran
   * 11% slower, so wider tiles keep e = tid + 256 i, one load each) */
  static constexpr bool RUNS = DP <= 64;
  float ra[PER], rb[PER];
  static TM_DEV int elem(int tid, int i) { return RUNS ? 4 * (tid + 256 * (i / 4)) + i % 4 : tid + 256 * i; }
  /* RUNS, with D and the row stride multiples of 4 and both bases aligned:
   * one 16-byte (f32) or 8-byte load per run; else one load per element */
  TM_DEV void load(const T *a, const T *b, int r0, int n, int D, int64_t ss, int tid) {
    const bool vec = RUNS && D % 4 == 0 && ss % 4 == 0 &&
                     ((uintptr_t)a | (uintptr_t)b) % (4 * sizeof(T)) == 0;
    if (vec) {
      typedef T t4 __attribute__((ext_vector_type(4)));
#pragma unroll
      for (int i = 0; i < PER; i += 4) {
        const int e = elem(tid, i);
        const int r = r0 + e / DP, cc = e % DP;
        const bool ok = r < n && cc < D;
        const int64_t off = (int64_t)r * ss + cc;
        const t4 x = ok ? *(const t4 *)(a + off) : (t4){};
        const t4 y = ok ? *(const t4 *)(b + off) : (t4){};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          ra[i + j] = to_f32(x[j]);
          rb[i + j] = to_f32(y[j]);
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        const int e = elem(tid, i);
        const int r = r0 + e / DP, cc = e % DP;
        const bool ok = r < n && cc < D;
        const int64_t off = (int64_t)r * ss + cc;
        ra[i] = ok ? to_f32(a[off]) : 0.f;
        rb[i] = ok ? to_f32(b[off]) : 0.f;
      }
    }
  }
  TM_DEV void store(float *as, float *bs, int tid) const {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int e = elem(tid, i);
      as[(e / DP) * (DP + 1) + e % DP] = ra[i];
      bs[(e / DP) * (DP + 1) + e % DP] = rb[i];
    }
  }
  /* the forward's layouts: a row-major with 16-byte aligned rows of DP + 4,
   * b transposed ([DP][ROWS + 4]), so a lane's four consecutive d (of a) or
   * keys (of b) are one 16-byte read */
  TM_DEV void store_rows_cols(float *as, float *bt, int tid) const {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int e = elem(tid, i);
      as[(e / DP) * (DP + 4) + e % DP] = ra[i];
      bt[(e % DP) * (ROWS + 4) + e / DP] = rb[i];
    }
  }
};

/* ---------------------------------------------------------------------------
 * attn_fwd: FlashAttention-2 forward with the online softmax in the exp2
 * domain (AttentionKernel.swift:40-250; attention_training.py:37-71).
 * 64 queries per workgroup (16 per wave), keys in blocks of 64 (32 at DP = 96 and 128).
 * Each wave computes S^T = K Q^T so that a lane owns one query (column l%16)
 * and four keys per 16-key tile; the row statistics are then lane-local up to
 * a reduction over the four lane groups, and O^T = V^T P^T keeps the same
 * lane <-> query ownership for the rescale.
 * Operands come four MFMAs at a time from one 16-byte LDS read: the S^T
 * contraction takes d in the order 16 j + 4 g + t (lane group g, MFMA t of
 * chunk j), so a lane reads K[key][16 j + 4 g .. +3] at once and Q holds the
 * same d order; V is staged transposed, so the four keys 4 g + m of MFMAs
 * m = 0..3 of a P V step are adjacent in a V^T row.
 * ------------------------------------------------------------------------- */
template <typename T, int DP, bool CAUSAL>
TM_DEV void attn_fwd_generic(const TmAttnFwdArgs &p) {
  /* 64-key blocks; 32 at DP = 96 and 128, where the staged tiles and the
   * operands of 64 keys would need more registers than two waves per SIMD
   * leave */
  constexpr int BM = 64, BN = DP >= 96 ? 32 : 64, LDK = DP + 4, LDV = BN + 4, KT = BN / 16;
  __shared__ __align__(16) float Ks[BN * LDK];
  __shared__ __align__(16) float Vt[DP * LDV];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, c = lane & 15;
  const int bh = blockIdx.y;
  const int q0 = blockIdx.x * BM;
  const int n = p.n_ctx, D = p.head_dim;
  const int64_t base = (int64_t)bh * p.stride_head;
  const T *Q = (const T *)p.q + base;
  const T *K = (const T *)p.k + base;
  const T *V = (const T *)p.v + base;
  T *O = (T *)p.o + base;

  const int qi = q0 + wave * 16 + c;
  float q[DP / 16][4];
#pragma unroll
  for (int j = 0; j < DP / 16; ++j)
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int d = 16 * j + 4 * g + t;
      q[j][t] = (qi < n && d < D) ? to_f32(Q[(int64_t)qi * p.stride_seq + d]) : 0.f;
    }
  const float qk_scale = p.sm_scale * TM_LOG2E;
  float m_i = TM_NEG_INF, l_i = 0.f;
  f32x4 acc[DP / 16];
#pragma unroll
  for (int i = 0; i < DP / 16; ++i) acc[i] = (f32x4){0.f, 0.f, 0.f, 0.f};

  /* the key blocks this workgroup walks: all of them, or the split-th of
   * `splits` contiguous ranges */
  const int kend_all = CAUSAL ? min(n, q0 + BM) : n;
  const int nkb = (kend_all + BN - 1) / BN;
  const int split = blockIdx.z;
  const int kbeg = p.splits > 1 ? (int)((int64_t)split * nkb / p.splits) * BN : 0;
  const int kend = p.splits > 1 ? min(kend_all, (int)((int64_t)(split + 1) * nkb / p.splits) * BN) : kend_all;
  TileStager<T, BN, DP> kv;
  if (kbeg < kend) kv.load(K, V, kbeg, n, D, p.stride_seq, tid);
  for (int k0 = kbeg; k0 < kend; k0 += BN) {
    __syncthreads();
    kv.store_rows_cols(Ks, Vt, tid);
    __syncthreads();
    if (k0 + BN < kend) kv.load(K, V, k0 + BN, n, D, p.stride_seq, tid);

    float sc[KT][4];
    float mx = TM_NEG_INF;
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) {
      f32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < DP / 16; ++j) {
        const f32x4 ka = *(const f32x4 *)&Ks[(kt * 16 + c) * LDK + 16 * j + 4 * g];
#pragma unroll
        for (int t = 0; t < 4; ++t) s = mfma_f32_16x16x4(ka[t], q[j][t], s);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int kj = k0 + kt * 16 + 4 * g + r;
        float v = s[r] * qk_scale;
        if (kj >= n || (CAUSAL && kj > qi)) v = TM_NEG_INF;
        sc[kt][r] = v;
        mx = fmaxf(mx, v);
      }
    }
    mx = group4_max(mx);
    const float m_new = fmaxf(m_i, mx);
    /* a row whose keys so far are all masked (the first blocks of a key
     * range above a causal query) keeps P = 0 and l = 0 instead of
     * exp2(-inf - -inf) */
    const float m_use = m_new == TM_NEG_INF ? 0.f : m_new;
    float rs = 0.f;
#pragma unroll
    for (int kt = 0; kt < KT; ++kt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        sc[kt][r] = exp2f(sc[kt][r] - m_use);
        rs += sc[kt][r];
      }
    rs = group4_sum(rs);
    const float alpha = exp2f(m_i - m_use);
    l_i = l_i * alpha + rs;
    m_i = m_new;
#pragma unroll
    for (int dt = 0; dt < DP / 16; ++dt) {
      acc[dt] *= alpha;
#pragma unroll
      for (int kt = 0; kt < KT; ++kt) {
        const f32x4 va = *(const f32x4 *)&Vt[(dt * 16 + c) * LDV + kt * 16 + 4 * g];
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[dt] = mfma_f32_16x16x4(va[r], round_through<T>(sc[kt][r]), acc[dt]);
      }
    }
  }

  if (qi < n && p.splits > 1) {
    /* partials of this key range: unnormalised O, then (m, l) */
    float *po = p.part + (((int64_t)split * p.heads + bh) * n + qi) * D;
#pragma unroll
    for (int dt = 0; dt < DP / 16; ++dt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int d = dt * 16 + 4 * g + r;
        if (d < D) po[d] = acc[dt][r];
      }
    if (g == 0) {
      float *pml = p.part + (int64_t)p.splits * p.heads * n * D +
                   (((int64_t)split * p.heads + bh) * n + qi) * 2;
      pml[0] = m_i;
      pml[1] = l_i;
    }
  } else if (qi < n) {
    const float inv = 1.f / l_i;
#pragma unroll
    for (int dt = 0; dt < DP / 16; ++dt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int d = dt * 16 + 4 * g + r;
        if (d < D) O[(int64_t)qi * p.stride_seq + d] = from_f32<T>(acc[dt][r] * inv);
      }
    if (p.lse && g == 0) p.lse[(int64_t)bh * p.stride_lse + qi] = m_i + log2f(l_i);
  }
}

/* The forward's key-range partials combined (TmAttnFwdArgs.part): for each
 * row, m = max_s m_s, l = sum_s 2^(m_s - m) l_s, O = sum_s 2^(m_s - m) O_s / l,
 * L = m + log2(l) -- the online softmax's own rescaling, applied across the
 * ranges.  Ranges with l_s = 0 (every key masked for the row) add nothing.
 * 64 threads per row (head_dim up to 128), 4 rows per workgroup. */
template <typename T>
TM_DEV void attn_fwd_combine(const TmAttnFwdArgs &p) {
  constexpr int SMAX = 16; /* the planner's largest split */
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int n = p.n_ctx, D = p.head_dim, S = p.splits;
  if (row >= (int64_t)p.heads * n) return;
  const int bh = (int)(row / n), q = (int)(row - (int64_t)bh * n);
  const int lane = threadIdx.x & 63;
  const int64_t range = (int64_t)p.heads * n; /* rows per range */
  const float *pml = p.part + (int64_t)S * range * D;
  /* every range's (m, l), then every range's two O values, each as one batch
   * of independent loads */
  float m_s[SMAX], l_s[SMAX];
#pragma unroll
  for (int s = 0; s < SMAX; ++s) {
    const bool in = s < S;
    m_s[s] = in ? pml[(s * range + row) * 2] : 0.f;
    l_s[s] = in ? pml[(s * range + row) * 2 + 1] : 0.f;
  }
  float o0_s[SMAX], o1_s[SMAX];
#pragma unroll
  for (int s = 0; s < SMAX; ++s) {
    const float *po = p.part + (s * range + row) * D;
    o0_s[s] = s < S && lane < D ? po[lane] : 0.f;
    o1_s[s] = s < S && lane + 64 < D ? po[lane + 64] : 0.f;
  }
  float m = TM_NEG_INF;
#pragma unroll
  for (int s = 0; s < SMAX; ++s)
    if (l_s[s] > 0.f) m = fmaxf(m, m_s[s]);
  float l = 0.f, o0 = 0.f, o1 = 0.f;
#pragma unroll
  for (int s = 0; s < SMAX; ++s) {
    if (!(l_s[s] > 0.f)) continue;
    const float w = exp2f(m_s[s] - m);
    l += w * l_s[s];
    o0 += w * o0_s[s];
    o1 += w * o1_s[s];
  }
  const float inv = 1.f / l;
  T *O = (T *)p.o + (int64_t)bh * p.stride_head + (int64_t)q * p.stride_seq;
  if (lane < D) O[lane] = from_f32<T>(o0 * inv);
  if (lane + 64 < D) O[lane + 64] = from_f32<T>(o1 * inv);
  if (p.lse && lane == 0) p.lse[(int64_t)bh * p.stride_lse + q] = m + log2f(l);
}

/* ---------------------------------------------------------------------------
 * attn_bwd_preprocess: Delta_i = sum_d dO_id * O_id in f32
 * (AttentionBackwardKernel.swift:53-136).  64 rows per workgroup, 16 per
 * wave: 16 lanes share a row (lane l sums d = l % 16 + 16 j), four rows at a
 * time with all their loads issued together, then a 16-lane reduction.
 * ------------------------------------------------------------------------- */
template <typename T>
TM_DEV void attn_pre_generic(const TmAttnPreArgs &p) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int bh = blockIdx.y;
  const int64_t base = (int64_t)bh * p.stride_head;
  const T *O = (const T *)p.o + base;
  const T *dO = (const T *)p.dout + base;
  const int sub = lane & 15, grp = lane >> 4;
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    const int row = blockIdx.x * 64 + wave * 16 + it * 4 + grp;
    float acc = 0.f;
    if (row < p.n_ctx) {
#pragma unroll
      for (int j = 0; j < 8; ++j) { /* head_dim <= 128 */
        const int d = sub + 16 * j;
        if (d < p.head_dim) {
          const int64_t off = (int64_t)row * p.stride_seq + d;
          acc += to_f32(O[off]) * to_f32(dO[off]);
        }
      }
    }
#pragma unroll
    for (int off = 8; off >= 1; off >>= 1) acc += __shfl_xor(acc, off, 64);
    if (sub == 0 && row < p.n_ctx) p.delta[(int64_t)bh * p.stride_lse + row] = acc;
  }
}

/* ---------------------------------------------------------------------------
 * attn_bwd_dq: per key block, P = exp2(qk_scale Q K^T - L), dP = dO V^T,
 * dS = P (dP - Delta), dQ += dS K; dQ * sm_scale on the way out
 * (AttentionBackwardKernel.swift:151-344).  64 queries per workgroup.
 * S^T / dP^T are formed per wave so a lane owns one query, as in attn_fwd.
 * ------------------------------------------------------------------------- */
template <typename T, int DP, bool CAUSAL>
TM_DEV void attn_dq_generic(const TmAttnDqArgs &p) {
  constexpr int BM = 64, BN = 32, LD = DP + 1;
  __shared__ float Ks[BN * LD];
  __shared__ float Vs[BN * LD];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, c = lane & 15;
  const int bh = blockIdx.y;
  const int q0 = blockIdx.x * BM;
  const int n = p.n_ctx, D = p.head_dim;
  const int64_t base = (int64_t)bh * p.stride_head;
  const T *Q = (const T *)p.q + base;
  const T *K = (const T *)p.k + base;
  const T *V = (const T *)p.v + base;
  const T *dO = (const T *)p.dout + base;
  T *dQ = (T *)p.dq + base;

  const int qi = q0 + wave * 16 + c;
  float q[DP / 4], dov[DP / 4];
#pragma unroll
  for (int s = 0; s < DP / 4; ++s) {
    const int d = 4 * s + g;
    const bool ok = qi < n && d < D;
    const int64_t off = (int64_t)qi * p.stride_seq + d;
    q[s] = ok ? to_f32(Q[off]) : 0.f;
    dov[s] = ok ? to_f32(dO[off]) : 0.f;
  }
  const int64_t srow = (int64_t)bh * p.stride_lse + qi;
  const float lse = qi < n ? p.lse[srow] : 0.f;
  const float delta = qi < n ? p.delta[srow] : 0.f;
  const float qk_scale = p.sm_scale * TM_LOG2E;

  f32x4 acc[DP / 16];
#pragma unroll
  for (int i = 0; i < DP / 16; ++i) acc[i] = (f32x4){0.f, 0.f, 0.f, 0.f};

  const int kend_all = CAUSAL ? min(n, q0 + BM) : n;
  const int nkb = (kend_all + BN - 1) / BN;
  const int split = blockIdx.z;
  const int kbeg = p.splits > 1 ? (int)((int64_t)split * nkb / p.splits) * BN : 0;
  const int kend = p.splits > 1 ? min(kend_all, (int)((int64_t)(split + 1) * nkb / p.splits) * BN) : kend_all;
  TileStager<T, BN, DP> kv;
  if (kbeg < kend) kv.load(K, V, kbeg, n, D, p.stride_seq, tid);
  for (int k0 = kbeg; k0 < kend; k0 += BN) {
    __syncthreads();
    kv.store(Ks, Vs, tid);
    __syncthreads();
    if (k0 + BN < kend) kv.load(K, V, k0 + BN, n, D, p.stride_seq, tid);

    float ds[2][4];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      f32x4 s = {0.f, 0.f, 0.f, 0.f}, dp = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int st = 0; st < DP / 4; ++st) {
        s = mfma_f32_16x16x4(Ks[(t * 16 + c) * LD + 4 * st + g], q[st], s);
        dp = mfma_f32_16x16x4(Vs[(t * 16 + c) * LD + 4 * st + g], dov[st], dp);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int kj = k0 + t * 16 + 4 * g + r;
        float v = s[r] * qk_scale;
        if (kj >= n || (CAUSAL && kj > qi)) v = TM_NEG_INF;
        const float pr = exp2f(v - lse);
        ds[t][r] = round_through<T>(pr * (dp[r] - delta));
      }
    }
#pragma unroll
    for (int dt = 0; dt < DP / 16; ++dt)
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          acc[dt] = mfma_f32_16x16x4(Ks[(t * 16 + 4 * g + r) * LD + dt * 16 + c], ds[t][r],
                                     acc[dt]);
  }

  if (qi < n) {
    float *po = p.splits > 1 ? p.part + (((int64_t)split * p.heads + bh) * n + qi) * D : nullptr;
#pragma unroll
    for (int dt = 0; dt < DP / 16; ++dt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int d = dt * 16 + 4 * g + r;
        if (d >= D) continue;
        if (po) po[d] = acc[dt][r];
        else dQ[(int64_t)qi * p.stride_seq + d] = from_f32<T>(acc[dt][r] * p.sm_scale);
      }
  }
}

/* ---------------------------------------------------------------------------
 * attn_bwd_dkdv: per query block, P^T = exp2(qk_scale K Q^T - L),
 * dV += P^T dO, dP^T = V dO^T, dS^T = P^T (dP^T - Delta), dK += dS^T Q;
 * dK * sm_scale and dV on the way out (AttentionBackwardKernel.swift:354-575).
 * 64 keys per workgroup (16 per wave); a lane owns one key.
 * ------------------------------------------------------------------------- */
template <typename T, int DP, bool CAUSAL>
TM_DEV void attn_dkdv_generic(const TmAttnDkdvArgs &p) {
  constexpr int BN = 64, BM = 32, LD = DP + 1;
  __shared__ float Qs[BM * LD];
  __shared__ float dOs[BM * LD];
  __shared__ float Ls[BM];
  __shared__ float Ds[BM];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, c = lane & 15;
  const int bh = blockIdx.y;
  const int k0 = blockIdx.x * BN;
  const int n = p.n_ctx, D = p.head_dim;
  const int64_t base = (int64_t)bh * p.stride_head;
  const T *Q = (const T *)p.q + base;
  const T *K = (const T *)p.k + base;
  const T *V = (const T *)p.v + base;
  const T *dO = (const T *)p.dout + base;
  T *dK = (T *)p.dk + base;
  T *dV = (T *)p.dv + base;
  const float *Lrow = p.lse + (int64_t)bh * p.stride_lse;
  const float *Drow = p.delta + (int64_t)bh * p.stride_lse;

  const int kj = k0 + wave * 16 + c;
  float kt[DP / 4], vt[DP / 4];
#pragma unroll
  for (int s = 0; s < DP / 4; ++s) {
    const int d = 4 * s + g;
    const bool ok = kj < n && d < D;
    const int64_t off = (int64_t)kj * p.stride_seq + d;
    kt[s] = ok ? to_f32(K[off]) : 0.f;
    vt[s] = ok ? to_f32(V[off]) : 0.f;
  }
  const float qk_scale = p.sm_scale * TM_LOG2E;
  f32x4 dk[DP / 16], dv[DP / 16];
#pragma unroll
  for (int i = 0; i < DP / 16; ++i) {
    dk[i] = (f32x4){0.f, 0.f, 0.f, 0.f};
    dv[i] = (f32x4){0.f, 0.f, 0.f, 0.f};
  }

  const int qfirst = CAUSAL ? (k0 / BM) * BM : 0;
  const int nqb = (n - qfirst + BM - 1) / BM;
  const int split = blockIdx.z;
  const int qstart = p.splits > 1 ? qfirst + (int)((int64_t)split * nqb / p.splits) * BM : qfirst;
  const int qstop = p.splits > 1 ? min(n, qfirst + (int)((int64_t)(split + 1) * nqb / p.splits) * BM) : n;
  TileStager<T, BM, DP> qdo;
  float l_next = 0.f, d_next = 0.f; /* thread tid < BM: L and Delta of row tid */
  auto load_stats = [&](int q0) {
    const int qi = q0 + tid;
    l_next = tid < BM && qi < n ? Lrow[qi] : 0.f;
    d_next = tid < BM && qi < n ? Drow[qi] : 0.f;
  };
  if (qstart < qstop) {
    qdo.load(Q, dO, qstart, n, D, p.stride_seq, tid);
    load_stats(qstart);
  }
  for (int q0 = qstart; q0 < qstop; q0 += BM) {
    __syncthreads();
    qdo.store(Qs, dOs, tid);
    if (tid < BM) {
      Ls[tid] = l_next;
      Ds[tid] = d_next;
    }
    __syncthreads();
    if (q0 + BM < qstop) {
      qdo.load(Q, dO, q0 + BM, n, D, p.stride_seq, tid);
      load_stats(q0 + BM);
    }

    float pt[2][4], dst[2][4];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      f32x4 s = {0.f, 0.f, 0.f, 0.f}, dp = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int st = 0; st < DP / 4; ++st) {
        s = mfma_f32_16x16x4(Qs[(t * 16 + c) * LD + 4 * st + g], kt[st], s);
        dp = mfma_f32_16x16x4(dOs[(t * 16 + c) * LD + 4 * st + g], vt[st], dp);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = t * 16 + 4 * g + r;
        const int qi = q0 + row;
        float v = s[r] * qk_scale;
        if (qi >= n || (CAUSAL && qi < kj)) v = TM_NEG_INF;
        const float pr = exp2f(v - Ls[row]);
        pt[t][r] = round_through<T>(pr);
        dst[t][r] = round_through<T>(pr * (dp[r] - Ds[row]));
      }
    }
#pragma unroll
    for (int dt = 0; dt < DP / 16; ++dt)
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = (t * 16 + 4 * g + r) * LD + dt * 16 + c;
          dv[dt] = mfma_f32_16x16x4(dOs[row], pt[t][r], dv[dt]);
          dk[dt] = mfma_f32_16x16x4(Qs[row], dst[t][r], dk[dt]);
        }
  }

  if (kj < n) {
    const int64_t plane = (int64_t)p.heads * n * D;
    float *pk = p.splits > 1 ? p.part + 2 * split * plane + ((int64_t)bh * n + kj) * D : nullptr;
#pragma unroll
    for (int dt = 0; dt < DP / 16; ++dt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int d = dt * 16 + 4 * g + r;
        if (d >= D) continue;
        if (pk) {
          pk[d] = dk[dt][r];
          pk[plane + d] = dv[dt][r];
        } else {
          const int64_t off = (int64_t)kj * p.stride_seq + d;
          dK[off] = from_f32<T>(dk[dt][r] * p.sm_scale);
          dV[off] = from_f32<T>(dv[dt][r]);
        }
      }
  }
}

/* The backward's range partials summed (TmAttnSplitReduceArgs): one row of
 * each output per 64 lanes (head_dim up to 128), 4 rows per workgroup, every
 * range's values loaded as one batch. */
template <typename T>
TM_DEV void attn_split_reduce(const TmAttnSplitReduceArgs &p) {
  constexpr int SMAX = 16; /* the planner's largest split */
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int n = p.n_ctx, D = p.head_dim, S = p.splits;
  if (row >= (int64_t)p.heads * n) return;
  const int bh = (int)(row / n), q = (int)(row - (int64_t)bh * n);
  const int lane = threadIdx.x & 63;
  const int64_t plane = (int64_t)p.heads * n * D;
  for (int w = 0; w < p.outputs; ++w) {
    float v0[SMAX], v1[SMAX];
#pragma unroll
    for (int s = 0; s < SMAX; ++s) {
      const float *src = p.part + (int64_t)(s * p.outputs + w) * plane + row * D;
      v0[s] = s < S && lane < D ? src[lane] : 0.f;
      v1[s] = s < S && lane + 64 < D ? src[lane + 64] : 0.f;
    }
    float a0 = 0.f, a1 = 0.f;
#pragma unroll
    for (int s = 0; s < SMAX; ++s) {
      a0 += v0[s];
      a1 += v1[s];
    }
    const float scale = w ? p.scale1 : p.scale0;
    T *out = (T *)(w ? p.out1 : p.out0) + (int64_t)bh * p.stride_head + (int64_t)q * p.stride_seq;
    if (lane < D) out[lane] = from_f32<T>(a0 * scale);
    if (lane + 64 < D) out[lane + 64] = from_f32<T>(a1 * scale);
  }
}

/* ---------------------------------------------------------------------------
 * tm_probe: one MFMA against the identity plus a plain store; out[i] == i for
 * i < 256 on a working device (the reference's probe idea, Runtime.swift:125-178).
 * ------------------------------------------------------------------------- */
extern "C" __global__ __launch_bounds__(64) void tm_probe(float *out) {
  const int l = threadIdx.x, g = l >> 4, c = l & 15;
  bf16x8 a, b;
#pragma unroll
  for (int s = 0; s < 8; ++s) {
    const int k = 8 * g + s;
    a[s] = (bf16_t)(c == k ? 1.f : 0.f);
    b[s] = (bf16_t)(k < 16 ? (float)(k * 16 + c) : 0.f);
  }
  f32x4 d = mfma_16x16x32(a, b, (f32x4){0.f, 0.f, 0.f, 0.f});
#pragma unroll
  for (int r = 0; r < 4; ++r) out[(4 * g + r) * 16 + c] = d[r];
}

/* ---- named instantiations (the symbols the runtime looks up) -------------- */

#define TM_GEMM(T, NAME, SAE_NAME) \
  extern "C" __global__ __launch_bounds__(256) void NAME(TmGemmArgs p) { gemm_generic<T, EPI_NONE>(p); } \
  extern "C" __global__ __launch_bounds__(256) void SAE_NAME(TmGemmArgs p) {                 \
    gemm_generic<T, EPI_BIAS_RELU>(p);                                                        \
  }
TM_GEMM(float, tm_gemm_generic_f32, tm_sae_generic_f32)
TM_GEMM(f16_t, tm_gemm_generic_f16, tm_sae_generic_f16)
TM_GEMM(bf16_t, tm_gemm_generic_bf16, tm_sae_generic_bf16)

#define TM_FWD_COMBINE(T, TN)                                                                  \
  extern "C" __global__ __launch_bounds__(256) void tm_attn_fwd_combine_##TN(TmAttnFwdArgs p) {  \
    attn_fwd_combine<T>(p);                                                                    \
  }
TM_FWD_COMBINE(float, f32)
TM_FWD_COMBINE(f16_t, f16)
TM_FWD_COMBINE(bf16_t, bf16)

#define TM_SPLIT_REDUCE(T, TN)                                                                  \
  extern "C" __global__ __launch_bounds__(256) void tm_attn_split_reduce_##TN(                   \
      TmAttnSplitReduceArgs p) {                                                                \
    attn_split_reduce<T>(p);                                                                    \
  }
TM_SPLIT_REDUCE(float, f32)
TM_SPLIT_REDUCE(f16_t, f16)
TM_SPLIT_REDUCE(bf16_t, bf16)

#define TM_PRE(T, NAME) \
  extern "C" __global__ __launch_bounds__(256) void NAME(TmAttnPreArgs p) { attn_pre_generic<T>(p); }
TM_PRE(float, tm_attn_pre_generic_f32)
TM_PRE(f16_t, tm_attn_pre_generic_f16)
TM_PRE(bf16_t, tm_attn_pre_generic_bf16)

#define TM_ATTN_ONE(T, TN, DP, CAUSAL, CN)                                                    \
  extern "C" __global__ __launch_bounds__(256) void tm_attn_fwd_generic_##TN##_d##DP##CN(     \
      TmAttnFwdArgs p) {                                                                      \
    attn_fwd_generic<T, DP, CAUSAL>(p);                                                       \
  }                                                                                           \
  extern "C" __global__ __launch_bounds__(256) void tm_attn_dq_generic_##TN##_d##DP##CN(      \
      TmAttnDqArgs p) {                                                                       \
    attn_dq_generic<T, DP, CAUSAL>(p);                                                        \
  }                                                                                           \
  extern "C" __global__ __launch_bounds__(256) void tm_attn_dkdv_generic_##TN##_d##DP##CN(    \
      TmAttnDkdvArgs p) {                                                                     \
    attn_dkdv_generic<T, DP, CAUSAL>(p);                                                      \
  }
#define TM_ATTN_DT(T, TN, DP)        \
  TM_ATTN_ONE(T, TN, DP, false, )    \
  TM_ATTN_ONE(T, TN, DP, true, _causal)
#define TM_ATTN_ALL_DP(T, TN) \
  TM_ATTN_DT(T, TN, 32)       \
  TM_ATTN_DT(T, TN, 64)       \
  TM_ATTN_DT(T, TN, 96)       \
  TM_ATTN_DT(T, TN, 128)
TM_ATTN_ALL_DP(float, f32)
TM_ATTN_ALL_DP(f16_t, f16)
TM_ATTN_ALL_DP(bf16_t, bf16)
