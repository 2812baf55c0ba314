/* nnops_amd_diag.h -- measurement probes, not part of the product ABI.
 *
 * Built into a separate library, libnnops_amd_diag.so, which only the
 * benchmark loads to put the workloads beside what this part sustains outside
 * the product kernels. No counterpart in nnops.
 */
#ifndef NNOPS_AMD_DIAG_H
#define NNOPS_AMD_DIAG_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Machine ceilings for the bench's roofline context.
 * nnops_hip_diag_mfma_i8: `blocks` x 4 waves, each `iters` x 8 independent
 *   v_mfma_i32_32x32x32_i8 from register operands (src: blocks*256*24 random
 *   ints, ignored when `constant`; out: blocks*256 ints); 65536 ops per MFMA.
 * nnops_hip_diag_stream_read: non-temporal 16-byte streaming read of `bytes`
 *   (16-byte aligned, a multiple of 16); out: 256 ints.
 * nnops_hip_diag_empty: an empty launch (the per-launch fixed cost). */
int nnops_hip_diag_mfma_i8(const int* src, int* out, int blocks, int iters, int constant, void* stream);
int nnops_hip_diag_stream_read(const void* buf, int64_t bytes, int* out, int blocks, void* stream);
int nnops_hip_diag_empty(int* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* NNOPS_AMD_DIAG_H */
