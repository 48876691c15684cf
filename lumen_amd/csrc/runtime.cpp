// Host runtime of libnhip: device selection, the static region allocator, copies, events, code objects,
// launches and the plan executor. Kernel entry points (nhip_gemm, nhip_flash_*) live in kernels.hip.
//
// Reference behaviour followed:
//   device:    lumen/device/cuda.rs:24-85 (device_count, set_device)
//   allocator: lumen/allocator/region.rs:15-242 (first-fit over one lazily reserved range, 256 B blocks,
//              synchronize-and-retry once, then an error naming static_allocator_bytes)
//   stream:    lumen/runtime/stream/mod.rs:31-78 (one stream per device; launches never wait)
//   launch:    lumen/runtime/kernel/cuda/mod.rs:88-169 (zero-size grids are no-ops)
//   plan:      lumen/plan/run.rs:356-427 (steps run in order on one host thread)
#include "nhip_internal.h"

#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

namespace nhip {

static thread_local std::string g_error;

int fail(const std::string &msg) {
    g_error = msg;
    return 1;
}

int check(hipError_t e, const char *what) {
    if (e == hipSuccess) return 0;
    return fail(std::string(what) + ": " + hipGetErrorString(e));
}

namespace {

constexpr size_t kAlignment = 256;
constexpr size_t kDefaultRegion = size_t(1) << 30;

struct Region {
    char *base = nullptr;
    size_t capacity = 0;
    std::map<size_t, size_t> free_blocks;  // offset -> length, coalesced
    std::map<size_t, size_t> live;         // offset -> length taken
    std::map<void *, size_t> own;          // blocks with their own hipMalloc -> bytes
    size_t live_bytes = 0;
};

struct Device {
    hipStream_t stream = nullptr;
    Region region;
};

std::mutex g_mutex;
std::map<int, std::unique_ptr<Device>> g_devices;

int current_device(int *dev) { return check(hipGetDevice(dev), "hipGetDevice"); }

// The device record, creating its stream on first use. Called with g_mutex held.
int device_locked(int dev, Device **out) {
    auto it = g_devices.find(dev);
    if (it == g_devices.end()) {
        int prev = 0;
        if (check(hipGetDevice(&prev), "hipGetDevice")) return 1;
        if (check(hipSetDevice(dev), "hipSetDevice")) return 1;
        auto d = std::make_unique<Device>();
        // Default priority: streams of other priorities have hung on these boxes.
        if (check(hipStreamCreateWithFlags(&d->stream, hipStreamNonBlocking), "hipStreamCreate")) return 1;
        if (prev != dev) hipSetDevice(prev);
        it = g_devices.emplace(dev, std::move(d)).first;
    }
    *out = it->second.get();
    return 0;
}

size_t round_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

int reserve_locked(int dev, Region &r, size_t bytes) {
    if (r.base) return 0;
    bytes = round_up(bytes ? bytes : kDefaultRegion, kAlignment);
    void *p = nullptr;
    int prev = 0;
    hipGetDevice(&prev);
    hipSetDevice(dev);
    hipError_t e = hipMalloc(&p, bytes);
    hipSetDevice(prev);
    if (e != hipSuccess)
        return fail("hip:" + std::to_string(dev) + " cannot reserve its static region of " + std::to_string(bytes) +
                    " bytes: " + hipGetErrorString(e));
    r.base = static_cast<char *>(p);
    r.capacity = bytes;
    r.free_blocks.clear();
    r.free_blocks[0] = bytes;
    return 0;
}

// First fit of `bytes` at `align` in the free list; returns the offset or SIZE_MAX.
size_t take_locked(Region &r, size_t bytes, size_t align) {
    for (auto it = r.free_blocks.begin(); it != r.free_blocks.end(); ++it) {
        size_t off = it->first, len = it->second;
        size_t start = round_up(off, align);
        if (start + bytes > off + len) continue;
        r.free_blocks.erase(it);
        if (start > off) r.free_blocks[off] = start - off;
        if (off + len > start + bytes) r.free_blocks[start + bytes] = off + len - (start + bytes);
        r.live[start] = bytes;
        r.live_bytes += bytes;
        return start;
    }
    return SIZE_MAX;
}

void release_locked(Region &r, size_t off) {
    auto it = r.live.find(off);
    size_t len = it->second;
    r.live_bytes -= len;
    r.live.erase(it);
    auto next = r.free_blocks.lower_bound(off);
    if (next != r.free_blocks.end() && next->first == off + len) {
        len += next->second;
        r.free_blocks.erase(next);
    }
    auto prev = r.free_blocks.lower_bound(off);
    if (prev != r.free_blocks.begin()) {
        --prev;
        if (prev->first + prev->second == off) {
            prev->second += len;
            return;
        }
    }
    r.free_blocks[off] = len;
}

struct Module {
    hipModule_t module;
};
std::map<std::string, Module> g_modules;

}  // namespace

hipStream_t stream_of_current() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return nullptr;
    std::lock_guard<std::mutex> lock(g_mutex);
    Device *d = nullptr;
    if (device_locked(dev, &d)) return nullptr;
    return d->stream;
}

}  // namespace nhip

using namespace nhip;

extern "C" {

const char *nhip_last_error(void) { return g_error.c_str(); }

int nhip_device_count(int *count) {
    *count = 0;
    hipError_t e = hipGetDeviceCount(count);
    if (e == hipErrorNoDevice) {
        *count = 0;
        return 0;
    }
    return check(e, "hipGetDeviceCount");
}

int nhip_set_device(int device) {
    int n = 0;
    if (nhip_device_count(&n)) return 1;
    if (device < 0 || device >= n)
        return fail("hip:" + std::to_string(device) + " is not available: " + std::to_string(n) + " HIP device(s)");
    if (check(hipSetDevice(device), "hipSetDevice")) return 1;
    std::lock_guard<std::mutex> lock(g_mutex);
    Device *d = nullptr;
    return device_locked(device, &d);
}

int nhip_device_props(int device, nhip_props *props) {
    hipDeviceProp_t p;
    if (check(hipGetDeviceProperties(&p, device), "hipGetDeviceProperties")) return 1;
    std::memset(props, 0, sizeof(*props));
    std::snprintf(props->name, sizeof(props->name), "%s", p.name);
    std::snprintf(props->arch, sizeof(props->arch), "%s", p.gcnArchName);
    props->compute_units = p.multiProcessorCount;
    props->lds_bytes = static_cast<int32_t>(p.sharedMemPerBlock);
    props->clock_khz = p.clockRate;
    props->memory_clock_khz = p.memoryClockRate;
    props->memory_bus_bits = p.memoryBusWidth;
    props->l2_bytes = p.l2CacheSize;
    props->hbm_bytes = p.totalGlobalMem;
    // gfx950 and gfx942 parts are built of 8 XCDs (32 CUs each on MI355X).
    props->xcds = (std::strncmp(p.gcnArchName, "gfx95", 5) == 0 || std::strncmp(p.gcnArchName, "gfx94", 5) == 0) ? 8 : 0;
    return 0;
}

int nhip_region_reserve(int device, size_t bytes) {
    std::lock_guard<std::mutex> lock(g_mutex);
    Device *d = nullptr;
    if (device_locked(device, &d)) return 1;
    if (d->region.base) {
        if (d->region.capacity >= bytes) return 0;
        if (!d->region.live.empty())
            return fail("hip:" + std::to_string(device) + " static region is in use: cannot grow it to " +
                        std::to_string(bytes) + " bytes");
        hipFree(d->region.base);
        d->region.base = nullptr;
    }
    return reserve_locked(device, d->region, bytes);
}

int nhip_alloc(int device, size_t bytes, size_t alignment, void **ptr) {
    *ptr = nullptr;
    if (alignment == 0) alignment = kAlignment;
    if (alignment & (alignment - 1)) return fail("nhip_alloc: alignment must be a power of two");
    if (alignment < kAlignment) alignment = kAlignment;
    size_t n = round_up(bytes ? bytes : 1, kAlignment);
    std::lock_guard<std::mutex> lock(g_mutex);
    Device *d = nullptr;
    if (device_locked(device, &d)) return 1;
    Region &r = d->region;
    if (!r.base && reserve_locked(device, r, 0)) return 1;
    if (n > r.capacity / 4) {
        // A large block (a plan workspace, a weight matrix): an allocation of its own, freed with it, so
        // large blocks never fragment the region the small ones share.
        int prev = 0;
        hipGetDevice(&prev);
        hipSetDevice(device);
        void *p = nullptr;
        hipError_t e = hipMalloc(&p, n);
        hipSetDevice(prev);
        if (e != hipSuccess)
            return fail("hip:" + std::to_string(device) + " out of memory: " + std::to_string(bytes) +
                        " bytes requested: " + hipGetErrorString(e));
        r.own[p] = n;
        *ptr = p;
        return 0;
    }
    size_t off = take_locked(r, n, alignment);
    if (off == SIZE_MAX) {
        // Blocks freed by queued work come back once the stream drains; retry once after it.
        hipStreamSynchronize(d->stream);
        off = take_locked(r, n, alignment);
    }
    if (off == SIZE_MAX) {
        size_t free_total = 0, largest = 0;
        for (auto &kv : r.free_blocks) {
            free_total += kv.second;
            largest = std::max(largest, kv.second);
        }
        return fail("hip:" + std::to_string(device) + " static allocator out of memory: " + std::to_string(bytes) +
                    " bytes requested, " + std::to_string(free_total) + " of " + std::to_string(r.capacity) +
                    " bytes free (largest block " + std::to_string(largest) +
                    "); raise lumen_amd.config.static_allocator_bytes");
    }
    *ptr = r.base + off;
    return 0;
}

int nhip_free(int device, void *ptr, size_t bytes) {
    (void)bytes;
    if (!ptr) return 0;
    std::lock_guard<std::mutex> lock(g_mutex);
    Device *d = nullptr;
    if (device_locked(device, &d)) return 1;
    Region &r = d->region;
    auto own = r.own.find(ptr);
    if (own != r.own.end()) {
        hipStreamSynchronize(d->stream);
        hipError_t e = hipFree(ptr);
        r.own.erase(own);
        return check(e, "hipFree");
    }
    char *p = static_cast<char *>(ptr);
    if (!r.base || p < r.base || p >= r.base + r.capacity || !r.live.count(size_t(p - r.base)))
        return fail("nhip_free: the pointer was not allocated by nhip_alloc on this device");
    release_locked(r, size_t(p - r.base));
    return 0;
}

int nhip_region_stats(int device, size_t *live_bytes, size_t *capacity) {
    std::lock_guard<std::mutex> lock(g_mutex);
    Device *d = nullptr;
    if (device_locked(device, &d)) return 1;
    size_t own = 0;
    for (auto &kv : d->region.own) own += kv.second;
    *live_bytes = d->region.live_bytes + own;
    *capacity = d->region.capacity;
    return 0;
}

int nhip_memcpy_h2d(void *dst, const void *src, size_t bytes) {
    if (!bytes) return 0;
    hipStream_t s = stream_of_current();
    if (!s) return fail("no HIP stream: call nhip_set_device first");
    // A pageable source is staged by the runtime; the host may reuse it when this returns.
    if (check(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, s), "hipMemcpyAsync(H2D)")) return 1;
    return check(hipStreamSynchronize(s), "hipStreamSynchronize");
}

int nhip_memcpy_d2h(void *dst, const void *src, size_t bytes) {
    if (!bytes) return 0;
    hipStream_t s = stream_of_current();
    if (!s) return fail("no HIP stream: call nhip_set_device first");
    if (check(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, s), "hipMemcpyAsync(D2H)")) return 1;
    return check(hipStreamSynchronize(s), "hipStreamSynchronize");
}

int nhip_memcpy_d2d(void *dst, const void *src, size_t bytes) {
    if (!bytes) return 0;
    hipStream_t s = stream_of_current();
    if (!s) return fail("no HIP stream: call nhip_set_device first");
    return check(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, s), "hipMemcpyAsync(D2D)");
}

int nhip_memset(void *dst, int value, size_t bytes) {
    if (!bytes) return 0;
    hipStream_t s = stream_of_current();
    if (!s) return fail("no HIP stream: call nhip_set_device first");
    return check(hipMemsetAsync(dst, value, bytes, s), "hipMemsetAsync");
}

int nhip_stream_sync(int device) {
    hipStream_t s;
    {
        std::lock_guard<std::mutex> lock(g_mutex);
        Device *d = nullptr;
        if (device_locked(device, &d)) return 1;
        s = d->stream;
    }
    return check(hipStreamSynchronize(s), "hipStreamSynchronize");
}

int nhip_event_create(void **event) {
    hipEvent_t e;
    if (check(hipEventCreate(&e), "hipEventCreate")) return 1;
    *event = e;
    return 0;
}

int nhip_event_record(void *event) {
    hipStream_t s = stream_of_current();
    if (!s) return fail("no HIP stream: call nhip_set_device first");
    return check(hipEventRecord(static_cast<hipEvent_t>(event), s), "hipEventRecord");
}

int nhip_event_elapsed_ms(void *start, void *end, float *ms) {
    if (check(hipEventSynchronize(static_cast<hipEvent_t>(end)), "hipEventSynchronize")) return 1;
    return check(hipEventElapsedTime(ms, static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(end)),
                 "hipEventElapsedTime");
}

int nhip_event_destroy(void *event) { return check(hipEventDestroy(static_cast<hipEvent_t>(event)), "hipEventDestroy"); }

int nhip_module_load(const char *path, void **module) {
    std::lock_guard<std::mutex> lock(g_mutex);
    auto it = g_modules.find(path);
    if (it == g_modules.end()) {
        hipModule_t m;
        if (check(hipModuleLoad(&m, path), (std::string("hipModuleLoad(") + path + ")").c_str())) return 1;
        it = g_modules.emplace(path, Module{m}).first;
    }
    *module = it->second.module;
    return 0;
}

int nhip_module_function(void *module, const char *name, void **function) {
    hipFunction_t f;
    if (check(hipModuleGetFunction(&f, static_cast<hipModule_t>(module), name),
              (std::string("hipModuleGetFunction(") + name + ")").c_str()))
        return 1;
    *function = f;
    return 0;
}

static int launch_on(hipStream_t s, void *function, const uint32_t grid[3], const uint32_t block[3],
                     uint32_t lds_bytes, const void *args, size_t args_bytes) {
    if (!grid[0] || !grid[1] || !grid[2]) return 0;
    size_t size = args_bytes;
    void *config[] = {HIP_LAUNCH_PARAM_BUFFER_POINTER, const_cast<void *>(args), HIP_LAUNCH_PARAM_BUFFER_SIZE, &size,
                      HIP_LAUNCH_PARAM_END};
    return check(hipModuleLaunchKernel(static_cast<hipFunction_t>(function), grid[0], grid[1], grid[2], block[0],
                                       block[1], block[2], lds_bytes, s, nullptr, config),
                 "hipModuleLaunchKernel");
}

int nhip_launch(void *function, const uint32_t grid[3], const uint32_t block[3], uint32_t lds_bytes, const void *args,
                size_t args_bytes) {
    hipStream_t s = stream_of_current();
    if (!s) return fail("no HIP stream: call nhip_set_device first");
    return launch_on(s, function, grid, block, lds_bytes, args, args_bytes);
}

// ---- plans ----------------------------------------------------------------------------------------------

namespace {

struct Step {
    int kind = 0;  // 0: launch, else NHIP_STEP_*
    void *function = nullptr;
    uint32_t grid[3] = {1, 1, 1}, block[3] = {1, 1, 1}, lds = 0;
    std::vector<unsigned char> args;  // launch arguments, or the built-in's descriptor
    std::vector<nhip_reloc> relocs;
};

struct Plan {
    std::vector<Step> steps;
    std::vector<unsigned char> scratch;
    bool profile = false;
    std::vector<hipEvent_t> events;  // one before each step and one after the last, when profiling
};

}  // namespace

int nhip_plan_create(void **plan) {
    *plan = new Plan();
    return 0;
}

int nhip_plan_destroy(void *plan) {
    Plan *p = static_cast<Plan *>(plan);
    for (hipEvent_t e : p->events) (void)hipEventDestroy(e);
    delete p;
    return 0;
}

int nhip_plan_profile(void *plan, int enable) {
    Plan *p = static_cast<Plan *>(plan);
    p->profile = enable != 0;
    while (p->profile && p->events.size() < p->steps.size() + 1) {
        hipEvent_t e;
        if (check(hipEventCreate(&e), "hipEventCreate")) return 1;
        p->events.push_back(e);
    }
    return 0;
}

int nhip_plan_step_ms(void *plan, float *ms, size_t n) {
    Plan *p = static_cast<Plan *>(plan);
    if (!p->profile || p->events.size() < p->steps.size() + 1) return fail("nhip_plan_step_ms: profiling is off");
    if (check(hipEventSynchronize(p->events[p->steps.size()]), "hipEventSynchronize")) return 1;
    for (size_t i = 0; i < n && i < p->steps.size(); ++i)
        if (check(hipEventElapsedTime(&ms[i], p->events[i], p->events[i + 1]), "hipEventElapsedTime")) return 1;
    return 0;
}

static int check_relocs(const nhip_reloc *relocs, size_t n, size_t limit, bool bytes) {
    for (size_t i = 0; i < n; ++i) {
        size_t end = bytes ? size_t(relocs[i].slot) + sizeof(void *) : size_t(relocs[i].slot) + 1;
        if (end > limit) return fail("nhip_plan: a relocation slot is outside the step's arguments");
        if (relocs[i].base > NHIP_BASE_INPUT) return fail("nhip_plan: unknown relocation base");
    }
    return 0;
}

int nhip_plan_add_launch(void *plan, void *function, const uint32_t grid[3], const uint32_t block[3],
                         uint32_t lds_bytes, const void *args, size_t args_bytes, const nhip_reloc *relocs,
                         size_t nrelocs) {
    if (check_relocs(relocs, nrelocs, args_bytes, true)) return 1;
    Step s;
    s.kind = 0;
    s.function = function;
    for (int i = 0; i < 3; ++i) s.grid[i] = grid[i], s.block[i] = block[i];
    s.lds = lds_bytes;
    s.args.assign(static_cast<const unsigned char *>(args), static_cast<const unsigned char *>(args) + args_bytes);
    s.relocs.assign(relocs, relocs + nrelocs);
    static_cast<Plan *>(plan)->steps.push_back(std::move(s));
    return 0;
}

int nhip_plan_add_builtin(void *plan, int kind, const void *desc, size_t desc_bytes, const nhip_reloc *relocs,
                          size_t nrelocs) {
    if (kind < NHIP_STEP_GEMM || kind > NHIP_STEP_LCE) return fail("nhip_plan_add_builtin: unknown step kind");
    // the descriptor must hold what run_steps reads for the kind
    size_t need = 0;
    switch (kind) {
        case NHIP_STEP_GEMM: need = sizeof(nhip_gemm_desc); break;
        case NHIP_STEP_FLASH_FWD:
        case NHIP_STEP_FLASH_BWD: need = sizeof(nhip_attn_desc); break;
        case NHIP_STEP_COPY: need = 8; break;
        case NHIP_STEP_FILL: need = 12; break;
        case NHIP_STEP_LCE: need = sizeof(nhip_lce_desc); break;
    }
    if (!desc || desc_bytes < need)
        return fail("nhip_plan_add_builtin: a descriptor of " + std::to_string(desc_bytes) + " bytes for a step kind " +
                    "that reads " + std::to_string(need));
    if (check_relocs(relocs, nrelocs, 16, false)) return 1;
    Step s;
    s.kind = kind;
    s.args.assign(static_cast<const unsigned char *>(desc), static_cast<const unsigned char *>(desc) + desc_bytes);
    s.relocs.assign(relocs, relocs + nrelocs);
    static_cast<Plan *>(plan)->steps.push_back(std::move(s));
    return 0;
}

int nhip_plan_steps(void *plan, size_t *count) {
    *count = static_cast<Plan *>(plan)->steps.size();
    return 0;
}

int nhip_plan_run(void *plan_, void *workspace, void *const *inputs, size_t ninputs) {
    Plan *plan = static_cast<Plan *>(plan_);
    return nhip_plan_run_steps(plan_, workspace, inputs, ninputs, 0, plan->steps.size());
}

static int run_steps(Plan *plan, void *workspace, void *const *inputs, size_t ninputs, size_t begin, size_t end,
                     bool events);

int nhip_plan_run_steps(void *plan_, void *workspace, void *const *inputs, size_t ninputs, size_t begin, size_t end) {
    return run_steps(static_cast<Plan *>(plan_), workspace, inputs, ninputs, begin, end, true);
}

struct Graph {
    hipGraphExec_t exec = nullptr;
    int device = 0;
};

int nhip_plan_capture(void *plan_, void *workspace, void *const *inputs, size_t ninputs, void **graph) {
    Plan *plan = static_cast<Plan *>(plan_);
    hipStream_t s = stream_of_current();
    if (!s) return fail("no HIP stream: call nhip_set_device first");
    int dev = 0;
    if (check(hipGetDevice(&dev), "hipGetDevice")) return 1;
    if (check(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture")) return 1;
    const int rc = run_steps(plan, workspace, inputs, ninputs, 0, plan->steps.size(), false);
    const std::string err = rc ? g_error : std::string();
    hipGraph_t g = nullptr;
    const hipError_t end = hipStreamEndCapture(s, &g);  // ends the capture even when a step failed
    if (rc) {
        if (g) (void)hipGraphDestroy(g);
        return fail("nhip_plan_capture: " + err);
    }
    if (check(end, "hipStreamEndCapture")) return 1;
    hipGraphExec_t exec = nullptr;
    const hipError_t inst = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (check(inst, "hipGraphInstantiate")) return 1;
    Graph *out = new Graph;
    out->exec = exec;
    out->device = dev;
    *graph = out;
    return 0;
}

int nhip_graph_launch(void *graph_) {
    Graph *graph = static_cast<Graph *>(graph_);
    hipStream_t s = stream_of_current();
    if (!s) return fail("no HIP stream: call nhip_set_device first");
    int dev = 0;
    if (check(hipGetDevice(&dev), "hipGetDevice")) return 1;
    if (dev != graph->device) return fail("nhip_graph_launch: the graph was captured on another device");
    return check(hipGraphLaunch(graph->exec, s), "hipGraphLaunch");
}

int nhip_graph_destroy(void *graph_) {
    Graph *graph = static_cast<Graph *>(graph_);
    if (!graph) return 0;
    const int rc = graph->exec ? check(hipGraphExecDestroy(graph->exec), "hipGraphExecDestroy") : 0;
    delete graph;
    return rc;
}

static int run_steps(Plan *plan, void *workspace, void *const *inputs, size_t ninputs, size_t begin, size_t end,
                     bool events) {
    hipStream_t s = stream_of_current();
    if (!s) return fail("no HIP stream: call nhip_set_device first");
    if (begin > end || end > plan->steps.size())
        return fail("nhip_plan_run_steps: steps [" + std::to_string(begin) + ", " + std::to_string(end) + ") of " +
                    std::to_string(plan->steps.size()));
    // per-step events only when profiling has created one for every step boundary (steps added after
    // nhip_plan_profile(1) run untimed until it is called again)
    const bool whole = events && begin == 0 && end == plan->steps.size() && plan->profile &&
                       plan->events.size() >= plan->steps.size() + 1;
    char *ws = static_cast<char *>(workspace);
    for (size_t i = begin; i < end; ++i) {
        Step &st = plan->steps[i];
        if (whole && check(hipEventRecord(plan->events[i], s), "hipEventRecord")) return 1;
        auto resolve = [&](const nhip_reloc &r, void **out) -> int {
            char *base;
            if (r.base == NHIP_BASE_WORKSPACE) {
                base = ws;
            } else {
                if (r.index >= ninputs) return fail("nhip_plan_run: a step reads input " + std::to_string(r.index) +
                                                    " of " + std::to_string(ninputs));
                base = static_cast<char *>(inputs[r.index]);
            }
            *out = base + r.offset;
            return 0;
        };
        if (st.kind == 0) {
            plan->scratch.assign(st.args.begin(), st.args.end());
            for (auto &r : st.relocs) {
                void *p;
                if (resolve(r, &p)) return 1;
                std::memcpy(plan->scratch.data() + r.slot, &p, sizeof(p));
            }
            if (launch_on(s, st.function, st.grid, st.block, st.lds, plan->scratch.data(), plan->scratch.size()))
                return fail("plan step " + std::to_string(i) + ": " + g_error);
            continue;
        }
        void *ptrs[16] = {nullptr};
        for (auto &r : st.relocs)
            if (resolve(r, &ptrs[r.slot])) return 1;
        int rc = 0;
        switch (st.kind) {
            case NHIP_STEP_GEMM:
                rc = gemm_splitk_on(s, reinterpret_cast<const nhip_gemm_desc *>(st.args.data()), ptrs[0], ptrs[1],
                                    ptrs[2], ptrs[3]);
                break;
            case NHIP_STEP_FLASH_FWD:
                rc = flash_fwd_on(s, reinterpret_cast<const nhip_attn_desc *>(st.args.data()), ptrs[0], ptrs[1],
                                  ptrs[2], ptrs[3], static_cast<float *>(ptrs[4]));
                break;
            case NHIP_STEP_FLASH_BWD:
                rc = flash_bwd_on(s, reinterpret_cast<const nhip_attn_desc *>(st.args.data()), ptrs[0], ptrs[1],
                                  ptrs[2], ptrs[3], ptrs[4], static_cast<const float *>(ptrs[5]), ptrs[6], ptrs[7],
                                  ptrs[8], ptrs[9]);
                break;
            case NHIP_STEP_COPY: {
                uint64_t n;
                std::memcpy(&n, st.args.data(), 8);
                if (n) rc = check(hipMemcpyAsync(ptrs[0], ptrs[1], n, hipMemcpyDeviceToDevice, s), "hipMemcpyAsync");
                break;
            }
            case NHIP_STEP_LCE:
                rc = lce_on(s, reinterpret_cast<const nhip_lce_desc *>(st.args.data()), ptrs[0], ptrs[1], ptrs[2],
                            static_cast<float *>(ptrs[3]), ptrs[4]);
                break;
            case NHIP_STEP_FILL: {
                uint64_t n;
                uint32_t v;
                std::memcpy(&n, st.args.data(), 8);
                std::memcpy(&v, st.args.data() + 8, 4);
                rc = fill_on(s, ptrs[0], n, static_cast<unsigned char>(v));
                break;
            }
        }
        if (rc) return fail("plan step " + std::to_string(i) + ": " + g_error);
    }
    if (whole && check(hipEventRecord(plan->events[plan->steps.size()], s), "hipEventRecord"))
        return 1;
    return 0;
}

}  // extern "C"
