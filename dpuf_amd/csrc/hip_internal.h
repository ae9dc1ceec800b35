// hip_internal.h -- host-side helpers shared by the HIP translation units of
// the engine (rt.hip, gemv.hip, gemm.hip, gemt.hip, attn.hip, attn_wide.hip,
// attn_dec.hip).
#ifndef DPUF_HIP_INTERNAL_H
#define DPUF_HIP_INTERNAL_H

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "hip_layer.h"

// Records e (when it is the first error of the current API call on this
// thread) with the name of what failed.
void dpuf_note(hipError_t e, const char* what);
static inline void note(hipError_t e, const char* what) { dpuf_note(e, what); }
#define CK(x) note((x), #x)
#define LAUNCHED(name) note(hipGetLastError(), name)
#define ST(s) ((hipStream_t)(s))

// Counts an attention launch of path `which` (dpuf_hip_attn_path_count).
void attn_path_note(int which);

extern "C" {
// Compute units of the current device (cached; 1 when the query fails).
int dpuf_hip_cu_count(void);
// Cap of the GEMV / K-split GEMM workgroups (dpuf_hip_set_gemv_max_wg; 0: none).
int dpuf_hip_mv_max_wg(void);
// Device error word bound to the current API call on this thread (NULL: none).
int32_t* dpuf_hip_error_word(void);
// The M > 1 GEMM of n_jobs matrices of one mode; rows [z0, z1) of zo (row
// stride zld) are set to 0 by the same launch.
void dpuf_hip_gm_launch(void* s, int32_t M, int32_t n_jobs, const DpufGemvJob* jobs, float* zo, int32_t zld,
                        int32_t z0, int32_t z1);
// The few-token GEMM (mode 12, 2 <= M <= 16, K a multiple of 128 up to
// 4096, more 16-row fragments than CUs); -1 without launching otherwise.
int32_t dpuf_hip_mvt_launch(void* s, int32_t M, int32_t n_jobs, const DpufGemvJob* jobs);
}

#endif
