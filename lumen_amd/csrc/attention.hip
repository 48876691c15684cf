// C entry points of the flash attention kernels (attention.h): nhip_flash_fwd, nhip_flash_bwd.
#include "attention.h"
#include "nhip_internal.h"

using namespace nhip;

extern "C" {

int nhip_flash_fwd(const nhip_attn_desc *desc, const void *q, const void *k, const void *v, void *o, float *lse) {
    hipStream_t s = stream_of_current();
    if (!s) return fail("no HIP stream: call nhip_set_device first");
    return flash_fwd_on(s, desc, q, k, v, o, lse);
}

int nhip_flash_bwd(const nhip_attn_desc *desc, const void *q, const void *k, const void *v, const void *o,
                   const void *d_o, const float *lse, void *dq, void *dk, void *dv, void *workspace) {
    hipStream_t s = stream_of_current();
    if (!s) return fail("no HIP stream: call nhip_set_device first");
    return flash_bwd_on(s, desc, q, k, v, o, d_o, lse, dq, dk, dv, workspace);
}

int nhip_flash_bwd_workspace(const nhip_attn_desc *desc, size_t *bytes) {
    *bytes = flash_bwd_workspace_bytes(desc);
    return 0;
}

}  // extern "C"
