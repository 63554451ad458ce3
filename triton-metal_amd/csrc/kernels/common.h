/*
 * Device helpers shared by the gfx950 kernels: element types, conversions, MFMA
 * wrappers and wavefront reductions.  CDNA4 only: 64-lane wavefronts, MFMA
 * matrix cores, 160 KB LDS per CU.
 *
 * MFMA operand layouts used throughout (lane l in [0, 64), g = l / 16):
 *   v_mfma_f32_16x16x4_f32    A: row l%16, k = g          B: col l%16, k = g
 *   v_mfma_f32_16x16x32_bf16  A: row l%16, k = 8g .. 8g+7 B: col l%16, k = 8g .. 8g+7
 *   (and _f16)                D: col l%16, rows 4g .. 4g+3 (4 floats)
 *   v_mfma_f32_32x32x16_bf16  A: row l%32, k = 8h .. 8h+7 B: col l%32, k = 8h .. 8h+7
 *   (and _f16, h = l / 32)    D: col l%32, rows 8j + 4h .. 8j + 4h + 3 in
 *                                floats 4j .. 4j+3 (j = 0..3; 16 floats)
 * On gfx950 both forms reach the dense peak when enough independent
 * accumulators are in flight (two waves per SIMD, or eight chains in one
 * wave: about 17 cycles per 16x16x32, 34 per 32x32x16); with four chains in a
 * single wave the 16x16x32 form is latency-bound at about 19 cycles.
 * The contraction index k may be permuted freely as long as A and B use the
 * same permutation; the attention kernels rely on that to feed the softmax
 * output (rows 4g..4g+3 of a 16-row tile) straight back in as a B operand.
 */
#ifndef TM_KERNELS_COMMON_H
#define TM_KERNELS_COMMON_H

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../tm_args.h"

#define TM_DEV __device__ __forceinline__

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

typedef __bf16 bf16_t;
typedef _Float16 f16_t;

/* ---- conversions ---------------------------------------------------------- */

template <typename T> TM_DEV float to_f32(T x) { return (float)x; }

/* Round-to-nearest-even narrowing (clang lowers (__bf16)f and (_Float16)f to
 * the gfx950 RNE conversions). */
template <typename T> TM_DEV T from_f32(float x) { return (T)x; }
template <> TM_DEV float from_f32<float>(float x) { return x; }

/* The value a float takes after a round trip through T: how the reference's
 * truncf of P and dS before the second dot is reproduced in an fp32 dot. */
template <typename T> TM_DEV float round_through(float x) { return (float)(T)x; }
template <> TM_DEV float round_through<float>(float x) { return x; }

/* ---- MFMA ----------------------------------------------------------------- */

TM_DEV f32x4 mfma_f32_16x16x4(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

TM_DEV f32x4 mfma_16x16x32(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
TM_DEV f32x4 mfma_16x16x32(f16x8 a, f16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

TM_DEV f32x16 mfma_32x32x16(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
TM_DEV f32x16 mfma_32x32x16(f16x8 a, f16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

/* Epilogues of the GEMM kernels: the plain product (matmul_kernel) or
 * relu(acc + bias[col]) on the fp32 accumulator before the single store
 * (sae_encode_kernel, Sources/TritonMetalMLX/SAEEncoder.swift:1-20). */
enum GemmEpilogue { EPI_NONE = 0, EPI_BIAS_RELU = 1 };

/* ---- wavefront reductions over the four 16-lane groups --------------------- */

/* IEEE maximum (NaN-propagating); gfx950 has v_maximum3_f32 for it, so a
 * chain of two needs one instruction and no canonicalising moves. */
TM_DEV float vmax(float a, float b) { return __builtin_elementwise_maximum(a, b); }

/* x and x[lane ^ 32] (resp. 16) through the gfx950 row-swap moves
 * v_permlane32_swap / v_permlane16_swap: no LDS round trip.  Swapping x with
 * itself leaves lane i holding {x[i], x[i ^ 32]} in some order. */
TM_DEV void swap32(float x, float &a, float &b) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  a = __uint_as_float(r[0]);
  b = __uint_as_float(r[1]);
}
TM_DEV void swap16(float x, float &a, float &b) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  a = __uint_as_float(r[0]);
  b = __uint_as_float(r[1]);
}

TM_DEV float group4_max(float x) {
  float a, b;
  swap32(x, a, b);
  swap16(vmax(a, b), a, b);
  return vmax(a, b);
}
TM_DEV float group4_sum(float x) {
  float a, b;
  swap32(x, a, b);
  swap16(a + b, a, b);
  return a + b;
}

TM_DEV float wave_sum(float x) {
  for (int off = 32; off >= 1; off >>= 1) x += __shfl_xor(x, off, 64);
  return x;
}

/* ---- HBM -> LDS copies ------------------------------------------------------
 * buffer_load ... lds / global_load_lds write each lane's bytes to LDS at
 * M0 + 4-byte or 16-byte lane slots, without passing through registers.  They
 * are issued from inline assembly on purpose: the compiler models an
 * in-flight LDS copy as an unordered LGKM event and then waits lgkmcnt(0) for
 * every LDS read issued while a copy is outstanding, which serialises the
 * operand reads of the whole step.  On gfx950 the copy is counted by vmcnt
 * only (a probe reads LDS 108 cycles after issuing a copy that lands 1800
 * cycles later), so the reads can be pipelined.  The compiler does not see
 * these writes: every caller waits for its copies itself (s_waitcnt
 * vmcnt(0)) and then barriers before any wave reads the tile.  The "memory"
 * clobber keeps the compiler's own LDS accesses on their side of the copy.
 * M0 (the LDS base) is an operand bound to the register itself, so the
 * compiler knows it is set.  The compiler's hazard recognizer does not look
 * inside the asm, so the asm opens with the wait states its operands may
 * need: 5 after a VALU write of an SGPR the copy reads (the resource words
 * come from v_readfirstlane), which also covers the 1 after a write of M0. */

/* lane slot = 16 bytes at M0 + 16 * lane, from the raw buffer described by
 * the (wave-uniform) resource `rsrc` at byte offset `voffset` */
TM_DEV void lds_copy16_buffer(u32x4 rsrc, int voffset, uint32_t lds_base) {
  asm volatile("s_nop 4\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               :: "{m0}"(lds_base), "v"(voffset), "s"(rsrc) : "memory");
}
/* lane slot = 16 bytes at M0 + 16 * lane, from `src` */
TM_DEV void lds_copy16_global(const void *src, uint32_t lds_base) {
  asm volatile("s_nop 4\n\tglobal_load_lds_dwordx4 %1, off"
               :: "{m0}"(lds_base), "v"(src) : "memory");
}
/* lane slot = 4 bytes at M0 + 4 * lane, from `src` */
TM_DEV void lds_copy4_global(const void *src, uint32_t lds_base) {
  asm volatile("s_nop 4\n\tglobal_load_lds_dword %1, off"
               :: "{m0}"(lds_base), "v"(src) : "memory");
}
/* LDS byte address of a shared-memory pointer (address-space cast, not the
 * flat aperture address), made wave-uniform: the M0 operand of the copies */
TM_DEV uint32_t lds_addr(const void *p) {
  typedef __attribute__((address_space(3))) const char lds_char;
  return __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_char *)p);
}
/* A raw buffer resource (gfx9 family: 48-bit base, stride 0, `bytes` records,
 * 32-bit data format) for the wave-uniform base `p`. */
TM_DEV u32x4 raw_buffer_rsrc(const void *p, int64_t bytes) {
  const uint64_t a = (uint64_t)p;
  const int32_t n = (int32_t)(bytes < (int64_t)INT32_MAX ? bytes : (int64_t)INT32_MAX);
  return (u32x4){(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)a),
                 (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(a >> 32)) & 0xffffu,
                 (uint32_t)__builtin_amdgcn_readfirstlane(n), 0x00020000u};
}

/* log2(e), written out: the reference folds sm_scale into the exp2 domain with
 * this constant (Sources/TritonMetalBench/AttentionKernel.swift:79-80). */
#define TM_LOG2E 1.44269504088896340736f

#endif
