/*
 * Kernel argument blocks of the built-in gfx950 kernels.
 *
 * The host side of tm_launch (runtime.cpp) fills one of these from the
 * reference-ordered (kinds, values) arrays and passes it to the device function
 * as its single by-value kernel argument.  The field order follows the
 * reference's argument lists:
 *   matmul_kernel        Sources/TritonMetalBench/GEMMKernel.swift:42-45
 *   attn_fwd             Sources/TritonMetalBench/AttentionKernel.swift:75-78
 *   attn_bwd_preprocess  Sources/TritonMetalBench/AttentionBackwardKernel.swift:53-64
 *   attn_bwd_dq          Sources/TritonMetalBench/AttentionBackwardKernel.swift:170-174
 *   attn_bwd_dkdv        Sources/TritonMetalBench/AttentionBackwardKernel.swift:384-388
 * followed by what the reference bakes into its IR as compile-time constants
 * (head_dim) or carries in the grid (heads).
 */
#ifndef TM_ARGS_H
#define TM_ARGS_H

#include <stdint.h>

struct TmGemmArgs {
  const void *a;
  const void *b;
  void *c;
  int32_t m, n, k;
  int32_t sam, sak, sbk, sbn, scm, scn;
  const void *bias; /* [n] elements; read only by the bias + ReLU epilogue kernels */
  /* K split across workgroups (splits > 1, grid y): fp32 partial products
   * [splits][m][round4(n)], summed into c by the reduce dispatch */
  float *part;
  int32_t splits;
};

struct TmAttnFwdArgs {
  const void *q;
  const void *k;
  const void *v;
  void *o;
  float *lse; /* may be NULL: the 8-argument form writes no statistics */
  float sm_scale;
  int32_t stride_head, stride_seq, n_ctx, stride_lse;
  int32_t head_dim, heads;
  /* key-range split (small grids): with splits > 1, workgroup z takes the
   * z-th of `splits` ranges of its key blocks and writes fp32 partials to
   * `part` -- [splits][heads][n_ctx][head_dim] unnormalised O, then
   * [splits][heads][n_ctx][2] (row offset m, row sum l) -- which
   * tm_attn_fwd_combine_* turns into O and L */
  float *part;
  int32_t splits;
};

/* out_w[bh, q, :] = scale_w * sum_s part[s][w][bh][q][:] in the element type
 * at the caller's strides, w < outputs (the split dQ, or dK and dV) */
struct TmAttnSplitReduceArgs {
  const float *part;
  void *out0;
  void *out1;
  float scale0, scale1;
  int32_t stride_head, stride_seq, n_ctx, head_dim, heads, splits, outputs;
};

struct TmAttnPreArgs {
  const void *o;
  const void *dout;
  float *delta;
  int32_t stride_head, stride_seq, stride_lse, n_ctx;
  int32_t head_dim, heads;
};

struct TmAttnDqArgs {
  const void *q;
  const void *k;
  const void *v;
  const void *dout;
  void *dq;
  const float *lse;
  const float *delta;
  float sm_scale;
  int32_t stride_head, stride_seq, stride_lse, n_ctx;
  int32_t head_dim, heads;
  /* key-range split (small grids, generic kernels): workgroup z walks the
   * z-th of `splits` ranges of its key blocks and writes its unscaled fp32 dQ
   * to part [splits][heads][n_ctx][head_dim], summed by tm_attn_split_reduce_* */
  float *part;
  int32_t splits;
};

struct TmAttnDkdvArgs {
  const void *q;
  const void *k;
  const void *v;
  const void *dout;
  void *dk;
  void *dv;
  const float *lse;
  const float *delta;
  float sm_scale;
  int32_t stride_head, stride_seq, stride_lse, n_ctx;
  int32_t head_dim, heads;
  /* query-range split (small grids, generic kernels): workgroup z walks the
   * z-th of `splits` ranges of its query blocks and writes its unscaled fp32
   * dK then dV to part [splits][2][heads][n_ctx][head_dim] */
  float *part;
  int32_t splits;
};

/* attn_bwd_fused (built-in libraries with bwd=atomic; no reference kernel —
 * the single-pass variant the reference names at
 * AttentionBackwardKernel.swift:27-41 and docs/COMPARISON.md:151-154): the
 * dK/dV kernel's arguments plus dQ's fp32 accumulator ([heads][n_ctx][head_dim]
 * dense, zeroed before the launch). */
struct TmAttnFusedArgs {
  TmAttnDkdvArgs kv;
  float *dq_acc;
};

/* The passes around attn_bwd_fused: clear dq_acc (count floats), then write
 * dq = sm_scale * dq_acc in the element type at the caller's strides. */
struct TmAttnDqAccArgs {
  float *acc;
  void *dq;
  int64_t count;
  float sm_scale;
  int32_t stride_head, stride_seq, n_ctx, heads;
};

#endif
