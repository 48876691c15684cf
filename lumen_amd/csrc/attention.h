// Flash attention kernels for gfx950 (placeholder entry points; the kernels follow).
#pragma once

#include "device_common.h"
#include "nhip_internal.h"

namespace nhip {

inline size_t flash_bwd_workspace_bytes(const nhip_attn_desc *d) {
    return size_t(d->batch) * d->heads * d->sq * sizeof(float);
}

int flash_fwd_on(hipStream_t, const nhip_attn_desc *, const void *, const void *, const void *, void *, float *) {
    return fail("flash attention: the hip backend has no kernel for it yet");
}

int flash_bwd_on(hipStream_t, const nhip_attn_desc *, const void *, const void *, const void *, const void *,
                        const void *, const float *, void *, void *, void *, void *) {
    return fail("flash attention backward: the hip backend has no kernel for it yet");
}

}  // namespace nhip
