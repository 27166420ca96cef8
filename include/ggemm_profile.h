/* ggemm_profile.h -- in-process stage timing of the grouped pipeline.
 *
 * No counterpart in the reference's C ABI: it replaces the reference's NVTX stage ranges
 * (src/internal.h:13-34, src/ggemm.cu:622-689) for callers that need per-kernel durations
 * without an external profiler (bench.py's roofline figure).  Disabled by default; when enabled
 * every EMU_GROUPED / AUTO call records HIP events around prep, INT8 GEMM, reconstruct and the
 * native FP64 GEMM on the handle's stream (a ring of event sets, so enabling it adds no host
 * synchronisation to the calls).  Process-wide, not thread-safe.
 */
#ifndef GGEMM_PROFILE_H
#define GGEMM_PROFILE_H

#ifdef __cplusplus
extern "C" {
#endif

/* on = 1 enables, 0 disables.  Returns 0, or nonzero if the events cannot be created. */
int ggemm_profile_enable(int on);
/* Synchronises on the recorded calls, then reports the summed stage times in milliseconds
 * ms[0] prep, ms[1] INT8 GEMM, ms[2] reconstruct, ms[3] native FP64 GEMM, and the number of
 * calls measured.  reset = 1 clears the sums.  Returns 0 on success. */
int ggemm_profile_read(double* ms, long long* calls, int reset);
/* Kernel symbol name of the INT8 GEMM the last grouped call launched ("i8_grouped_kernel" or
 * "i8_large_kernel", as profilers list it), "" before any.  Recorded whether or not timing is on. */
const char* ggemm_profile_i8_kernel(void);

#ifdef __cplusplus
}
#endif
#endif
