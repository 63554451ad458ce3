/* Static device scratch for tm_launch_noalloc (scratch.hip). */
#ifndef TM_SCRATCH_H
#define TM_SCRATCH_H

#include <hip/hip_runtime.h>

/* 64 MiB per device: the fp32 dQ accumulator of attn_bwd_fused for up to
 * heads * n_ctx * head_dim = 16 Mi elements (e.g. B8 H16 S1024 D128). */
#define TM_SCRATCH_BYTES ((size_t)64 << 20)

/* The current device's copy of the scratch array (resolved once per device,
 * with that device current); hipSuccess or the error hipGetSymbolAddress gave. */
hipError_t tm_scratch_address(void **ptr);

#endif
