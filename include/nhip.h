/*
 * nhip.h: the C ABI of libnhip, lumen's MI355X (gfx950) execution backend.
 *
 * Every function returns an int status: 0 on success, nonzero on failure, with a message for the calling
 * thread in nhip_last_error(). This mirrors the Result<_, String> contracts of the reference's Rust
 * backends. No torch or HIP types appear in these signatures: pointers are device addresses as void*,
 * sizes are bytes or elements as stated.
 *
 * Ordering: every device operation is queued on the device's one stream (lumen/runtime/stream/README.md,
 * "one stream per device"); launches never wait. nhip_memcpy_d2h and nhip_stream_sync block the host.
 */
#ifndef NHIP_H
#define NHIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- errors ---------------------------------------------------------------------------------------- */

/* The last failure's message on this thread ("" if none). Replaces Result::Err strings
 * (lumen/device/mod.rs:24-35, lumen/runtime/kernel/cuda/mod.rs:94-168). */
const char *nhip_last_error(void);

/* ---- device (lumen/device/mod.rs:14-39 DeviceBackend; lumen/device/cuda.rs:28-84) ----------------- */

typedef struct {
    char name[64];          /* marketing name */
    char arch[32];          /* gcnArchName, e.g. "gfx950:sramecc+:xnack-" */
    int32_t compute_units;  /* CUs (256 on MI355X) */
    int32_t xcds;           /* accelerator complex dies, 8 on MI355X (0 when unknown) */
    int32_t lds_bytes;      /* LDS per workgroup limit */
    int32_t clock_khz;      /* peak shader clock */
    int32_t memory_clock_khz;
    int32_t memory_bus_bits;
    int32_t l2_bytes;
    size_t hbm_bytes;       /* total device memory */
} nhip_props;

/* Number of HIP devices visible to the process (device_count). */
int nhip_device_count(int *count);
/* Makes `device` current for this thread and creates its stream on first use (set_device). */
int nhip_set_device(int device);
/* Properties the roofline needs: CU count, LDS, clocks, HBM size. */
int nhip_device_props(int device, nhip_props *props);

/* ---- memory (lumen/allocator/cuda.rs:34-116, lumen/allocator/region.rs:15-242) --------------------- */

/* Reserves `bytes` of device memory as `device`'s static region (one hipMalloc), carved first-fit in
 * 256-byte blocks by nhip_alloc. Without a reservation nhip_alloc reserves 1 GiB on first use. */
int nhip_region_reserve(int device, size_t bytes);
/* Takes `bytes` at a multiple of `alignment` (a power of two; 256 when 0) from the region, or with its own
 * hipMalloc when the block is larger than a quarter of the region (a plan workspace of tens of GB). */
int nhip_alloc(int device, size_t bytes, size_t alignment, void **ptr);
/* Returns a block nhip_alloc gave (bytes as requested). Waits for the device's queued work first, since a
 * kernel may still read it. */
int nhip_free(int device, void *ptr, size_t bytes);
/* Live bytes and the region's capacity (allocator statistics for tests). */
int nhip_region_stats(int device, size_t *live_bytes, size_t *capacity);

/* ---- copies (lumen/runtime/device_transfer/cuda.rs:14-104) ---------------------------------------- */

int nhip_memcpy_h2d(void *dst, const void *src, size_t bytes);  /* stream-ordered; host may reuse src */
int nhip_memcpy_d2h(void *dst, const void *src, size_t bytes);  /* waits for the stream, then copies */
int nhip_memcpy_d2d(void *dst, const void *src, size_t bytes);  /* stream-ordered */
int nhip_memset(void *dst, int value, size_t bytes);            /* stream-ordered byte fill */

/* ---- stream / events (lumen/runtime/stream/mod.rs:31-52, lumen/runtime/event/cuda.rs:46-128) ------- */

int nhip_stream_sync(int device);
int nhip_event_create(void **event);
int nhip_event_record(void *event);                        /* on the current device's stream */
int nhip_event_elapsed_ms(void *start, void *end, float *ms); /* waits for `end` */
int nhip_event_destroy(void *event);

/* ---- code objects and launches (lumen/runtime/kernel/cuda/mod.rs:88-169, driver.rs:148-179) -------- */

/* Loads a gfx950 code object (.hsaco) from `path`; cached by path for the process. */
int nhip_module_load(const char *path, void **module);
int nhip_module_function(void *module, const char *name, void **function);
/* Launches `function` on the stream with a packed argument buffer. A grid with a zero dimension is a
 * no-op (lumen/runtime/kernel/cuda/mod.rs:130-132). */
int nhip_launch(void *function, const uint32_t grid[3], const uint32_t block[3], uint32_t lds_bytes,
                const void *args, size_t args_bytes);

/* ---- dtypes of the kernel descriptors --------------------------------------------------------------- */

enum {
    NHIP_F32 = 0,
    NHIP_BF16 = 1,
    NHIP_F16 = 2,
};

/* ---- dot_general as a GEMM (lumen/codegen/dot_general/cuda/mod.rs:656-758; contract of cuda_gemm,
 * lumen/graph_compiler/python.rs:847-1015) ------------------------------------------------------------ *
 *
 * D[b, i, j] = sum_k A[b, i, k] * B[b, k, j], with element strides for every axis (a transposed operand
 * is a strided view, lumen/codegen/dot_general/cuda/mod.rs:724-732). Up to three batch axes, each with its
 * own strides. bf16/f16 operands run on MFMA (v_mfma_f32_32x32x16_{bf16,f16}) with float32 accumulation;
 * float32 operands run the exact kernel: each output a sequential k-order fold, every product and sum
 * rounded to float32 (lumen/reference/mod.rs:981-993), bit-identical to the reference interpreter. */
typedef struct {
    int64_t m, n, k;
    int32_t nbatch;               /* 0..3 batch axes */
    int32_t a_dtype, b_dtype, d_dtype;
    int64_t batch[3];             /* sizes of the batch axes */
    int64_t a_batch[3], b_batch[3], d_batch[3];  /* element strides per batch axis */
    int64_t a_m, a_k;             /* element strides of A along m and k */
    int64_t b_k, b_n;             /* element strides of B along k and n */
    int64_t d_m, d_n;             /* element strides of D along m and n */
    int32_t config;               /* tile config index; -1 picks the default for the shape */
    int32_t splits;               /* split-k factor for nhip_gemm_splitk (0 or 1: none) */
} nhip_gemm_desc;

/* Queues D = A.B on the stream. A and B must be float dtypes of one kind (bf16/f16 together, or f32). */
int nhip_gemm(const nhip_gemm_desc *desc, const void *a, const void *b, void *d);
/* Number of tile configs nhip_gemm accepts in desc->config for bf16/f16 (autotuning, autotune/mod.rs). */
int nhip_gemm_config_count(int *count);
/* Split-k: D = A.B with k cut into desc->splits equal parts computed by separate workgroups (for shapes with
 * too few output tiles to fill the GPU, such as weight gradients), their float32 partial products summed in
 * split order by a second kernel. Needs 16-bit operands in the MFMA layouts, k a multiple of 64 * splits,
 * and `workspace` of nhip_gemm_workspace bytes (the scratch of a plan step,
 * lumen/plan/step/mod.rs:65-66). */
int nhip_gemm_splitk(const nhip_gemm_desc *desc, const void *a, const void *b, void *d, void *workspace);
int nhip_gemm_workspace(const nhip_gemm_desc *desc, size_t *bytes);

/* ---- flash attention (lumen/codegen/attention/cuda/mod.rs:33-59 Forward/Operand; Triton algorithm
 * lumen/codegen/attention/triton/kernel.py:34-256) ------------------------------------------------------ *
 *
 * Q [B, Sq, N, H], K [B, Sk, Nkv, H], V [B, Sk, Nkv, H], O [B, Sq, N, H] as element strides per axis
 * (batch, sequence, head; the head-dim axis is contiguous; every stride a multiple of 8 elements). N must be a
 * multiple of Nkv (grouped-query). H is a multiple of 8, at most 256 for the forward and 128 for the backward
 * (lumen/graph_compiler/passes/attention/forward.rs:100 MAX_HEAD, backward.rs:86); the kernels run at 64, 128 or
 * 256 with the columns past H read as zeros, which needs each (batch, head) of an operand within 2 GiB.
 * LSE and delta are float32 [B, N, Sq] (contiguous). Causal masks key j for query i where
 * j > i + Sk - Sq (bottom-right aligned, lumen/functional/attention/flash.py:95-97). */
typedef struct {
    int64_t batch, heads, kv_heads, sq, sk, head_dim;
    int32_t dtype;      /* NHIP_BF16 or NHIP_F16 */
    int32_t causal;
    float scale;
    int32_t config;     /* -1: default */
    int64_t q_b, q_s, q_n;
    int64_t k_b, k_s, k_n;
    int64_t v_b, v_s, v_n;
    int64_t o_b, o_s, o_n;
    int64_t do_b, do_s, do_n;    /* backward only */
    int64_t dq_b, dq_s, dq_n;    /* backward only */
    int64_t dk_b, dk_s, dk_n;    /* backward only */
    int64_t dv_b, dv_s, dv_n;    /* backward only */
    int32_t deterministic;       /* backward only, dQ's mode: 0 = added atomically by the dK/dV kernel into a
                                    float32 buffer (the reference's default, lumen/graph_compiler/config/mod.rs:117);
                                    1 = dQ = dS K from the 16-bit dS tiles the dK/dV kernel stores in the workspace
                                    (same bits every run); 2 = by a kernel recomputing S and dP (same bits every
                                    run, no dS workspace) */
    int64_t value_head_dim;      /* V's, O's and dO's head dim Hv (0: H), a multiple of 8 like H; the forward.rs
                                    `hv` (passes/attention/forward.rs:721) */
} nhip_attn_desc;

/* O = softmax(scale Q K^T [causal]) V, P rounded to the inputs' dtype before P V; writes LSE = m + log l
 * (kernel.py:99-102). */
int nhip_flash_fwd(const nhip_attn_desc *desc, const void *q, const void *k, const void *v, void *o, float *lse);
/* Number of forward tile configs nhip_attn_desc.config accepts (0: 128 queries a workgroup, the default for -1;
 * 1: 256; 2: 64) for autotuning and forced configs (the CUDA attention `Config`,
 * lumen/codegen/attention/cuda/mod.rs:312-420). */
int nhip_attn_config_count(int *count);
/* FlashAttention-2 backward (kernel.py:107-256): delta = rowsum(dO * O) (float32 [B, N, Sq]), then dK, dV
 * per key block, and dQ by desc->deterministic's mode: from the dS tiles the dK/dV kernel stored (1), per query
 * block by a kernel recomputing S and dP (2), or added atomically by the dK/dV kernel into a float32
 * [B, N, Sq, D] buffer in the workspace (D = H padded to 64 or 128), then rounded into dq (0). `workspace` needs nhip_flash_bwd_workspace
 * bytes (mode 1: 2 B N Sk Sq bytes of dS tiles, rounded up to 128 keys x 64 queries). */
int nhip_flash_bwd(const nhip_attn_desc *desc, const void *q, const void *k, const void *v, const void *o,
                   const void *d_o, const float *lse, void *dq, void *dk, void *dv, void *workspace);
int nhip_flash_bwd_workspace(const nhip_attn_desc *desc, size_t *bytes);
/* nhip_flash_bwd without a workspace argument and without allocating: its scratch (what
 * nhip_flash_bwd_workspace reports for the same desc) is a 16 MiB array in the library's device memory, one
 * per GPU, held until the process ends. No counterpart in the reference: for callers that cannot allocate
 * (code under HIP graph capture, serving loops, harnesses that forbid hipMalloc). Fails when the workspace
 * exceeds 16 MiB: mode 2 (8 bytes a query row) takes up to batch * heads * sq = 2^21 rows; modes 1 and 0 much
 * fewer (dS tiles, the float32 dQ accumulator). Calls that overlap on one GPU (several host threads or
 * streams) share the array and race. */
int nhip_flash_bwd_noalloc(const nhip_attn_desc *desc, const void *q, const void *k, const void *v, const void *o,
                           const void *d_o, const float *lse, void *dq, void *dk, void *dv);

/* ---- linear cross entropy (Primitive::LinearCrossEntropy, lumen/reference/mod.rs:1092-1120; the Triton kernel
 * lumen/codegen/dot_general/triton/linear_cross_entropy_kernel.py; the pass that emits it,
 * lumen/graph_compiler/passes/linear_cross_entropy.rs) ---------------------------------------------------- *
 *
 * h [b, d] and w [v, d] row-major (both bf16, both f16, or both float32), target [b] int32 or int64 (as
 * target_dtype NHIP_LCE_I32 / NHIP_LCE_I64). out is float32 [2, b]: row 0 the loss lse - logit[class], row 1
 * lse = max + log(sum_j exp(logit_j - max)), class = target clamped into [0, v). The [b, v] logits never
 * exist whole. With 16-bit operands, d % 64 == 0 and v % 64 == 0 (and h, w 16-byte aligned) the GEMM's store
 * reduces each row's 64-class blocks to a (maximum, float32 sum of exponentials) pair and picks the class's
 * logit, and a second kernel combines a row's pairs in float64 (workspace: b * v / 64 pairs of floats, rounded
 * up to 256 bytes, plus b floats; at least one row of logits). Otherwise the float32 logits of chunk_rows rows
 * at a time go through `workspace` (chunk_rows * v float32) by nhip_gemm, then one workgroup a row reduces them
 * (maximum, float32 exponentials summed in float64, picked logit). nhip_linear_cross_entropy_workspace gives
 * the bytes for either form. */
enum {
    NHIP_LCE_I32 = 0,
    NHIP_LCE_I64 = 1,
};
typedef struct {
    int64_t b, v, d;
    int64_t chunk_rows;  /* rows a pass; <= 0: all b */
    int32_t dtype;       /* NHIP_BF16, NHIP_F16 or NHIP_F32 */
    int32_t target_dtype;
} nhip_lce_desc;

int nhip_linear_cross_entropy(const nhip_lce_desc *desc, const void *h, const void *w, const void *target, float *out,
                              void *workspace);
int nhip_linear_cross_entropy_workspace(const nhip_lce_desc *desc, size_t *bytes);

/* ---- static plans (lumen/plan/run.rs:356-427 execute; lumen/plan/step/cuda.rs:17-63) ----------------- *
 *
 * A plan is a list of steps run in order on the stream: generated kernels (a function of a loaded module)
 * and built-in kernels (nhip_gemm, nhip_flash_fwd, nhip_flash_bwd, copies). Every pointer a step reads is
 * a relocation resolved at run time against the workspace base or one of the run's inputs, so a step list
 * is built once and run with any workspace and inputs, with no host work but the launches. */

enum {
    NHIP_BASE_WORKSPACE = 0,  /* index ignored: the workspace pointer */
    NHIP_BASE_INPUT = 1,      /* inputs[index] */
};

typedef struct {
    uint32_t slot;    /* byte offset in the launch's argument buffer (launch steps) or pointer index
                         (built-in steps) */
    uint32_t base;    /* NHIP_BASE_* */
    uint32_t index;   /* input index for NHIP_BASE_INPUT */
    uint32_t pad;
    uint64_t offset;  /* byte offset added to the base */
} nhip_reloc;

enum {
    NHIP_STEP_GEMM = 1,       /* desc: nhip_gemm_desc; pointers: a, b, d (and the workspace when splits > 1) */
    NHIP_STEP_FLASH_FWD = 2,  /* desc: nhip_attn_desc; pointers: q, k, v, o, lse */
    NHIP_STEP_FLASH_BWD = 3,  /* desc: nhip_attn_desc; pointers: q, k, v, o, do, lse, dq, dk, dv, ws */
    NHIP_STEP_COPY = 4,       /* desc: uint64 bytes; pointers: dst, src */
    NHIP_STEP_FILL = 5,       /* desc: uint64 bytes, uint32 byte value; pointers: dst */
    NHIP_STEP_LCE = 6,        /* desc: nhip_lce_desc; pointers: h, w, target, out, workspace */
};

int nhip_plan_create(void **plan);
int nhip_plan_destroy(void *plan);
/* Appends a launch of a generated kernel: its packed arguments with `nrelocs` pointer slots patched. */
int nhip_plan_add_launch(void *plan, void *function, const uint32_t grid[3], const uint32_t block[3],
                         uint32_t lds_bytes, const void *args, size_t args_bytes, const nhip_reloc *relocs,
                         size_t nrelocs);
/* Appends a built-in step of `kind` with its descriptor and pointer relocations. */
int nhip_plan_add_builtin(void *plan, int kind, const void *desc, size_t desc_bytes, const nhip_reloc *relocs,
                          size_t nrelocs);
/* Queues every step on the stream, in order (never waits). */
int nhip_plan_run(void *plan, void *workspace, void *const *inputs, size_t ninputs);
/* Queues steps [begin, end) only (profiling one step's kernels in isolation; the caller keeps their inputs
 * valid, e.g. by a whole run first). Per-step profiling events are recorded by whole runs only. */
int nhip_plan_run_steps(void *plan, void *workspace, void *const *inputs, size_t ninputs, size_t begin, size_t end);
/* Number of steps (for tests). */
int nhip_plan_steps(void *plan, size_t *count);
/* Profiling: with `enable`, each run records a HIP event before every step and after the last, on the
 * stream the steps launch on (lumen/plan/run.rs:418-422 times each step for the profiler). */
int nhip_plan_profile(void *plan, int enable);
/* Milliseconds of each of the first `n` steps of the last profiled run (waits for it to finish). */
int nhip_plan_step_ms(void *plan, float *ms, size_t n);

/* HIP graphs of a plan (the analogue of the reference's CUDA graphs: lumen/graph/tracer.py:958-1049,
 * lumen/runtime/stream/cuda.rs:119-294). nhip_plan_capture records every step of one run, bound to
 * `workspace` and `inputs` (whose addresses the graph keeps; the caller stages new argument values into
 * the same memory before each launch), into an executable graph; profiling events are not recorded.
 * nhip_graph_launch queues it on the current device's stream; nhip_graph_destroy frees it. */
int nhip_plan_capture(void *plan, void *workspace, void *const *inputs, size_t ninputs, void **graph);
int nhip_graph_launch(void *graph);
int nhip_graph_destroy(void *graph);

#ifdef __cplusplus
}
#endif

#endif /* NHIP_H */
