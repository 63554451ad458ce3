/*
 * tritonmetal.h — the tm_* C ABI of libtritonmetal.so, built for AMD gfx950 (MI355X).
 *
 * Every export keeps the signature, sentinel convention and error text of the
 * reference's Swift core, so a ctypes / Swift / C caller written against the
 * reference binds this library unchanged.  Reference interface cited per entry
 * as /root/reference/<file>:<line>.
 *
 * Conventions (reference Sources/TritonMetalCore/Compiler.swift:172-177):
 *   - char* results are malloc'd; the caller frees them with tm_free.
 *   - handle-returning calls return 0 on failure; int32 calls return -1.
 *   - on failure the reason is in tm_last_error(), which clears it and reads
 *     "no error" when empty.
 *   - handles are opaque int64 values from one locked table, starting at 1.
 *
 * MI355X meaning of the objects:
 *   - a "library" is a HIP code object (hipModule_t).  It is created from
 *       * a gfx950 code object image (tm_load_metallib),
 *       * HIP C++ source compiled at run time by hiprtc (tm_compile_msl), or
 *       * a built-in library spec "builtin [element=f32|f16|bf16]
 *         [head_dim=N] [causal=0|1] [bwd=split|atomic]" (tm_compile_msl),
 *         which names the library's hand-written gfx950 kernels for the dense
 *         hot path: matmul_kernel, attn_fwd, attn_bwd_preprocess, attn_bwd_dq,
 *         attn_bwd_dkdv, sae_encode_kernel (relu(x @ W + b),
 *         Sources/TritonMetalMLX/SAEEncoder.swift:29-40), tm_probe, and with
 *         bwd=atomic attn_bwd_fused (the backward in one call
 *         that AttentionBackwardKernel.swift:27-41 names: Q, K, V, dO, dQ, dK,
 *         dV, L, Delta, sm_scale, stride_head, stride_seq, stride_lse, n_ctx;
 *         dQ summed with fp32 atomics).
 *   - a "buffer" is device memory in HBM (hipMalloc).  tm_buffer_contents
 *     gives it a host-addressable mirror (pinned host memory) that stands in
 *     for the reference's unified memory: while the mirror exists, host
 *     writes through it reach the kernels of later launches and the results
 *     of a launch are in it when the launch returns (a launch that binds such
 *     a buffer copies it to HBM before the dispatch and back afterwards, and
 *     waits: the full buffer both ways, and tm_launch_async waits too).
 *     Buffers never mapped this way, or unmapped by tm_buffer_unmap, are not
 *     copied.
 *   - launches run on one library-owned HIP stream.
 */
#ifndef TRITONMETAL_H
#define TRITONMETAL_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Launch argument kinds (reference Compiler.swift:390-401). */
#define TM_ARG_BUFFER 0 /* values[i] is a buffer handle                   */
#define TM_ARG_I32 1    /* values[i] low 32 bits are an int32             */
#define TM_ARG_F32 2    /* values[i] low 32 bits are an f32 bit pattern   */
#define TM_ARG_I64 3    /* values[i] is an int64                          */

/* ---- process / device ---------------------------------------------------- */

/* "0.0.1".  Replaces Compiler.swift:180 tm_version. */
char *tm_version(void);
/* free() of a string this library returned.  Replaces Compiler.swift:185. */
void tm_free(void *ptr);
/* Last error message, cleared by the call; "no error" when none.
 * Replaces Compiler.swift:456 tm_last_error. */
char *tm_last_error(void);
/* 1 when a HIP device is present.  Replaces Runtime.swift:295 tm_is_active. */
int32_t tm_is_active(void);
/* 1 when the device ran the MFMA probe kernel correctly.
 * Replaces Runtime.swift:305 tm_is_usable. */
int32_t tm_is_usable(void);
/* Why tm_is_usable is 0, or NULL when usable.  Replaces Runtime.swift:312. */
char *tm_unusable_reason(void);
/* "<marketing name> (<gcnArchName>)" or NULL.  Replaces Runtime.swift:318. */
char *tm_device_name(void);

/* ---- libraries ----------------------------------------------------------- */

/* ttir lowering is not part of this library: for a built-in spec it returns the
 * normalised spec text, for anything else NULL with the reason.
 * Replaces Compiler.swift:192 tm_emit_msl. */
char *tm_emit_msl(const char *module, int32_t num_simdgroups);
/* Launch metadata JSON {"kernels":[{name, block_size, block_shape,
 * threads_per_threadgroup, args:[{index, kind, dtype}]}]} for a built-in spec.
 * Replaces Compiler.swift:214 tm_kernel_info. */
char *tm_kernel_info(const char *module, int32_t num_simdgroups);
/* Built-in spec or HIP source (hiprtc, gfx950) -> library handle, 0 on failure.
 * Replaces Compiler.swift:235 tm_compile_msl. */
int64_t tm_compile_msl(const char *source);
/* gfx950 code object image -> library handle, 0 on failure.
 * Replaces Compiler.swift:250 tm_load_metallib. */
int64_t tm_load_metallib(const void *image, int64_t length);
/* Replaces Compiler.swift:383 tm_release_library. */
int32_t tm_release_library(int64_t library);

/* ---- kernels ------------------------------------------------------------- */

/* Kernel by name -> kernel handle, 0 on failure.  Replaces Compiler.swift:266. */
int64_t tm_load_kernel(int64_t library, const char *name);
/* Largest workgroup the kernel accepts, -1 on failure.  Replaces Compiler.swift:284. */
int64_t tm_kernel_max_threads(int64_t kernel);
/* Replaces Compiler.swift:378 tm_release_kernel. */
int32_t tm_release_kernel(int64_t kernel);

/* ---- buffers ------------------------------------------------------------- */

/* length > 0 bytes of HBM -> buffer handle, 0 on failure.  Replaces Compiler.swift:296. */
int64_t tm_alloc_buffer(int64_t length);
/* Host address of the buffer's contents (its host mirror, created and filled
 * from HBM on the first call), NULL on failure.  Replaces Compiler.swift:307. */
void *tm_buffer_contents(int64_t buffer);
/* Replaces Compiler.swift:317 tm_buffer_length. */
int64_t tm_buffer_length(int64_t buffer);
/* Host -> device copy, bounds-checked; 0 / -1.  Replaces Compiler.swift:328. */
int32_t tm_buffer_write(int64_t buffer, int64_t offset, const void *source, int64_t length);
/* Device -> host copy (from the mirror when the buffer has one), bounds-checked;
 * 0 / -1.  Replaces Compiler.swift:338. */
int32_t tm_buffer_read(int64_t buffer, int64_t offset, void *destination, int64_t length);
/* Replaces Compiler.swift:373 tm_free_buffer. */
int32_t tm_free_buffer(int64_t buffer);

/* ---- launch -------------------------------------------------------------- */

/* Dispatch over a gx*gy*gz grid of workgroups of `threads` threads and wait.
 * Arguments bind by position (kinds[i], values[i]).  For the built-in kernels
 * the grid is a request in the reference's own terms: the library validates
 * it, takes the head count from gy*gz for the attention kernels, and covers
 * the whole problem with its own gfx950 tile shape (tm_kernel_info publishes
 * it).  0 / -1.  Replaces Compiler.swift:403 tm_launch. */
int32_t tm_launch(int64_t kernel, int64_t gx, int64_t gy, int64_t gz, int64_t threads,
                  const int32_t *kinds, const int64_t *values, int32_t argc);
/* Live handles (a leak check).  Replaces Compiler.swift:451. */
int64_t tm_live_handle_count(void);

/* ---- extensions with no reference counterpart ---------------------------- */

/* tm_launch without the wait: the dispatch is queued on the library stream.
 * For callers that chain dispatches (a training step) and synchronise once. */
int32_t tm_launch_async(int64_t kernel, int64_t gx, int64_t gy, int64_t gz, int64_t threads,
                        const int32_t *kinds, const int64_t *values, int32_t argc);
/* Wait for everything queued on the library stream.  0 / -1. */
int32_t tm_synchronize(void);
/* The reference's benchmark timing (packed dispatches between two timestamps,
 * reference Sources/TritonMetalBench/GEMMBenchmark.swift:250-277) as one call:
 * queues `repeats` back-to-back dispatches between two HIP events on the
 * library stream, waits, and stores the elapsed milliseconds in *elapsed_ms. */
int32_t tm_launch_timed(int64_t kernel, int64_t gx, int64_t gy, int64_t gz, int64_t threads,
                        const int32_t *kinds, const int64_t *values, int32_t argc,
                        int32_t repeats, float *elapsed_ms);
/* tm_launch that allocates nothing.  No reference counterpart: for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  A dispatch that needs a work buffer
 * (attn_bwd_fused's fp32 dQ accumulator under bwd=atomic, heads * n_ctx *
 * head_dim * 4 bytes, or the partial sums of a split GEMM or generic attention
 * kernel) takes it from a static device array of 64 MiB per device, held from the
 * first such call until the process ends; larger requests are refused with an
 * error (use tm_launch).  The caller passes inputs and outputs as for
 * tm_launch; this call waits.  Calls in one process are serialised on a lock;
 * the array keeps the last call's contents, and every dispatch clears what it
 * needs zeroed.  0 / -1. */
int32_t tm_launch_noalloc(int64_t kernel, int64_t gx, int64_t gy, int64_t gz, int64_t threads,
                          const int32_t *kinds, const int64_t *values, int32_t argc);
/* Drop the host mirror that tm_buffer_contents made: host writes made through
 * it are copied to HBM, the pinned memory is freed, and the address it gave
 * is no longer valid.  Launches that bind the buffer stop copying it and no
 * longer wait (tm_launch_async is asynchronous again).  A later
 * tm_buffer_contents makes a new mirror.  No-op without a mirror.  0 / -1.
 * No reference counterpart (the reference's buffers are unified memory). */
int32_t tm_buffer_unmap(int64_t buffer);
/* Name of the device function the last planned dispatch of `kernel` ran (the
 * symbol rocprof reports), NULL on failure.  For tests and profiling. */
char *tm_kernel_variant(int64_t kernel);

#ifdef __cplusplus
}
#endif

#endif /* TRITONMETAL_H */
