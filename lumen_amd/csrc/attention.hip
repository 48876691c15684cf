// C entry points of the flash attention kernels (attention.h): nhip_flash_fwd, nhip_flash_bwd and the
// allocation-free nhip_flash_bwd_noalloc.
#include <map>
#include <mutex>
#include <string>

#include "attention.h"
#include "nhip_internal.h"

using namespace nhip;

namespace {

// Scratch of nhip_flash_bwd_noalloc: the backward's workspace (delta and base-2 LSE, 2 floats a query row, then
// the mode's dS tiles or dQ accumulator), for callers that cannot allocate. One copy per GPU, held until the
// process ends; 16 MiB covers 2^21 query rows (batch x heads x sq) in mode 2, e.g. [4, 4096, 16, 128] uses
// 2 MiB there.
constexpr size_t kFlashScratchBytes = size_t(16) << 20;
__device__ __align__(256) unsigned char scratch[kFlashScratchBytes];

std::mutex scratch_mutex;
std::map<int, void *> scratch_address;  // device -> its copy of `scratch` (device address)

// The device address of the current device's `scratch`, looked up once per device. The array's name is a
// host-side stand-in, never passed to a kernel or a copy itself.
int scratch_of_current(void **out) {
    int dev = -1;
    if (check(hipGetDevice(&dev), "hipGetDevice")) return 1;
    std::lock_guard<std::mutex> lock(scratch_mutex);
    auto it = scratch_address.find(dev);
    if (it == scratch_address.end()) {
        void *ptr = nullptr;
        if (check(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)")) return 1;
        it = scratch_address.emplace(dev, ptr).first;
    }
    *out = it->second;
    return 0;
}

}  // namespace

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

int nhip_attn_config_count(int *count) {
    *count = kNumAttnConfigs;
    return 0;
}

int nhip_flash_bwd_workspace(const nhip_attn_desc *desc, size_t *bytes) {
    *bytes = flash_bwd_workspace_bytes(desc);
    return 0;
}

int nhip_flash_bwd_noalloc(const nhip_attn_desc *desc, const void *q, const void *k, const void *v, const void *o,
                           const void *d_o, const float *lse, void *dq, void *dk, void *dv) {
    hipStream_t s = stream_of_current();
    if (!s) return fail("no HIP stream: call nhip_set_device first");
    const size_t need = flash_bwd_workspace_bytes(desc);
    if (need > kFlashScratchBytes)
        return fail("nhip_flash_bwd_noalloc: " + std::to_string(desc->batch * desc->heads * desc->sq) +
                    " query rows need " + std::to_string(need) + " bytes of scratch, above its " +
                    std::to_string(kFlashScratchBytes) + " (mode 2 takes " + std::to_string(kFlashScratchBytes / 8) +
                    " rows); use nhip_flash_bwd with a workspace, or deterministic = 2");
    void *ws = nullptr;
    if (scratch_of_current(&ws)) return 1;
    // every scratch word the kernels read is written first in the same call (delta and LSE by the prep
    // kernel), so nothing needs clearing between calls
    return flash_bwd_on(s, desc, q, k, v, o, d_o, lse, dq, dk, dv, ws);
}

}  // extern "C"
