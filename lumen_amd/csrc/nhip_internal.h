// Declarations shared by runtime.cpp and kernels.hip (not part of the C ABI).
#pragma once

#include <hip/hip_runtime.h>

#include <string>

#include "../../include/nhip.h"

namespace nhip {

// Records `msg` as this thread's last error and returns 1.
int fail(const std::string &msg);
// 0 if `e` is hipSuccess, else fail("<what>: <hip message>").
int check(hipError_t e, const char *what);
// The current device's stream (created on first use), or nullptr.
hipStream_t stream_of_current();

// Built-in kernels queued on stream `s` (kernels.hip).
int gemm_on(hipStream_t s, const nhip_gemm_desc *d, const void *a, const void *b, void *out);
int gemm_splitk_on(hipStream_t s, const nhip_gemm_desc *d, const void *a, const void *b, void *out, void *ws);
int flash_fwd_on(hipStream_t s, const nhip_attn_desc *d, const void *q, const void *k, const void *v, void *o,
                 float *lse);
int flash_bwd_on(hipStream_t s, const nhip_attn_desc *d, const void *q, const void *k, const void *v,
                 const void *o, const void *d_o, const float *lse, void *dq, void *dk, void *dv, void *ws);
int fill_on(hipStream_t s, void *dst, size_t bytes, unsigned char value);
int lce_on(hipStream_t s, const nhip_lce_desc *d, const void *h, const void *w, const void *target, float *out,
           void *ws);

}  // namespace nhip
