/* Diagnostic entry points of the timing build (libg9gemm_timing.so, the same
 * kernels compiled with -DG9_TIMING).  They have no counterpart in the
 * reference, which measures loop efficiency from ATT thread traces
 * (scripts/process_json.py); this build records per-workgroup phase stamps
 * instead (gfx950_gluon_tutorials_amd/profiling.py reads them).  The regular
 * library does not export them. */
#ifndef GFX950_GEMM_TIMING_H
#define GFX950_GEMM_TIMING_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Copies the first `bytes` of the stamp buffer to host memory, as left by the
 * last launch, 8 uint64 per workgroup (by block index).  Data-parallel:
 * (shader clock, 100 MHz clock) at kernel entry, main-loop start, main-loop
 * end and kernel end.  Stream-K: (shader clock, 100 MHz clock) at entry and
 * exit, then shader cycles spent waiting for predecessor flags, loading
 * partial tiles and storing them, and (partial loads << 32) | partial stores.
 * Synchronous.  Returns G9_OK, G9_ERR_SHAPE when `bytes` exceeds the buffer,
 * or G9_ERR_HIP. */
int g9_timing_read(void* host, size_t bytes);

/* Number of workgroups the buffer holds stamps for. */
int g9_timing_capacity(void);

/* Same for the flash-attention kernel (its own buffer, the same capacity):
 * (shader clock, 100 MHz clock) at kernel entry, loop start, loop end and
 * kernel end per workgroup, as left by the last g9_fmha_fwd launch. */
int g9_fmha_timing_read(void* host, size_t bytes);

#ifdef __cplusplus
}
#endif

#endif
