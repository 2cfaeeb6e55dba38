/* C-ABI of libsolvedelta_noalloc.so: the forward without any allocation.
 *
 * No counterpart in the reference.  For callers that cannot call hipMalloc:
 * code under HIP graph capture, tight serving loops, harnesses that forbid
 * allocation.  sd_fwd_noalloc runs sd_fwd's kernels (libsolvedelta_hip.so, which
 * this library links) with the workspace in a device-resident static array of
 * SD_NOALLOC_SCRATCH_BYTES per GPU instead of a caller buffer.  The array lives
 * in this library only: processes that do not load it carry no static device
 * memory; one that does holds the array on each GPU it runs on until it exits.
 *
 *   - Inference only: the next call on the device overwrites the workspace, so
 *     there is no sd_bwd after it.
 *   - Shapes whose forward workspace (sd_fwd_workspace_bytes) exceeds the array
 *     return SD_ERR_WORKSPACE before any launch (B1 T1024 H8 r=V=128 fits).
 *   - Calls that overlap on one GPU (two streams, two threads) share the array
 *     and race; serialise them.
 */
#ifndef SOLVEDELTA_NOALLOC_H
#define SOLVEDELTA_NOALLOC_H

#include "solvedelta.h"

#ifdef __cplusplus
extern "C" {
#endif

#define SD_NOALLOC_SCRATCH_BYTES ((size_t)96 << 20)
size_t sd_noalloc_scratch_bytes(void);
int sd_fwd_noalloc(const sd_inputs *in, void *out, float *C_T, float *S_T, void *stream);

#ifdef __cplusplus
}
#endif
#endif
