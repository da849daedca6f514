/* Per-wave timeline of librq's kernels: exported only by librq_tl.so, the
 * same library built with -DRQ_TIMELINE (rllm_amd/build.py), which bench.py
 * --timeline loads in a child process. No counterpart in the reference: a
 * measurement aid, not part of the drop-in ABI of include/rq.h.
 *
 * Each instrumented kernel (the dot4 matvecs rq_mvx_* and GLU rq_glu_*, the
 * int8-MFMA classes rq_mmq*_* but Q6_K's 16-column ones) keeps up to
 * RQ_TL_MARKS stamps of the GPU's 100 MHz real-time counter per wave and
 * stores them at its end into its code object's array of RQ_TL_SLOTS slots
 * (slot = workgroup * waves per workgroup + wave, RQ_TL_MARKS u64 each);
 * every launch overwrites its own slots. */
#ifndef RQ_TIMELINE_H
#define RQ_TIMELINE_H

#include "rq.h"

#ifdef __cplusplus
extern "C" {
#endif

#define RQ_TL_MARKS 8
#define RQ_TL_SLOTS 32768

/* Copies the first `bytes` of code object `which`'s stamp array (0:
 * rq_kernels, 1: rq_mmq) to host memory, after the context's stream has
 * finished. */
rq_status rq_timeline_read(rq_ctx* ctx, int which, void* host, int64_t bytes);

#ifdef __cplusplus
}
#endif

#endif
