// Built-in kernels of libnhip and their C entry points: nhip_gemm (dot_general) and the fill used by plans
// (a kernel, not hipMemsetAsync, so a captured plan replays it correctly).
#include <cstring>

#include "gemm.h"
#include "nhip_internal.h"

using namespace nhipk;

namespace nhip {
namespace {

struct TileConfig {
    int bm, bn, bk, wm, wn;
};

// Candidates for bf16/f16 GEMMs, largest first (lumen/codegen/dot_general/cuda/mod.rs:430-633 keeps a
// similar list for SM80; these are sized for 160 KiB of LDS and wave64).
constexpr TileConfig kConfigs[] = {
    {256, 256, 64, 2, 4},
    {256, 128, 64, 2, 2},
    {128, 256, 64, 2, 2},
    {128, 128, 64, 2, 2},
    {128, 64, 64, 2, 2},
    {64, 64, 64, 2, 2},
};
constexpr int kNumTiled = sizeof(kConfigs) / sizeof(kConfigs[0]);
// Configs past the tiled ones: gemm_stream (256 x 256, operands streamed into LDS): k tile 64 with 4 waves of
// 128 x 128 (2 stages) and with 8 waves of 128 x 64 (2 stages); k tile 32 with 8 waves (4 stages); and
// gemm_stream128 (128 x 128 tiles, 4 waves of 64 x 64, 2 stages, two workgroups a CU); and
// gemm_stream_persist (the 8-wave 256 x 256 kernel, one persistent workgroup a CU walking the tiles); and the
// k tile 32, 8-wave kernel with its MFMA fragments read ahead across k tiles (gemm_stream_tile's XPF); and the
// k tile 32, 8-wave kernel whose two waves a SIMD alternate memory and MFMA phases (ping-pong); and the k tile
// 32, 4-wave (128 x 128 a wave) kernel with the cross-tile fragment prefetch.
constexpr int kStream4w = kNumTiled, kStream8w = kNumTiled + 1, kStream8w32 = kNumTiled + 2,
              kStream128 = kNumTiled + 3, kStreamPersist = kNumTiled + 4, kStream8wX = kNumTiled + 5,
              kStream8wP = kNumTiled + 6, kStream4wX = kNumTiled + 7, kStream4w64X = kNumTiled + 8,
              kStream8w64X = kNumTiled + 9;
constexpr int kNumConfigs = kNumTiled + 10;

GemmShape shape_of(const nhip_gemm_desc *d) {
    GemmShape s;
    std::memset(&s, 0, sizeof(s));
    s.m = d->m;
    s.n = d->n;
    s.k = d->k;
    s.nbatch = d->nbatch;
    for (int i = 0; i < 3; ++i) {
        s.batch[i] = d->batch[i];
        s.a_batch[i] = d->a_batch[i];
        s.b_batch[i] = d->b_batch[i];
        s.d_batch[i] = d->d_batch[i];
    }
    s.a_m = d->a_m;
    s.a_k = d->a_k;
    s.b_k = d->b_k;
    s.b_n = d->b_n;
    s.d_m = d->d_m;
    s.d_n = d->d_n;
    return s;
}

int64_t batch_count(const nhip_gemm_desc *d) {
    int64_t z = 1;
    for (int i = 0; i < d->nbatch; ++i) z *= d->batch[i];
    return z;
}

// The default tile for a shape: the streamed 256 x 256 kernel when k allows it and its tiles fill the 256 CUs,
// else the streamed 128 x 128 kernel (two workgroups a CU) when its tiles fill half of them, else the largest
// tiled config whose tile count fills them at least once.
int default_config(const nhip_gemm_desc *d) {
    int64_t z = batch_count(d);
    if (d->k % 64 == 0 && ((d->m + 255) / 256) * ((d->n + 255) / 256) * z >= 256) return kStream8w;
    if (d->k % 64 == 0 && ((d->m + 127) / 128) * ((d->n + 127) / 128) * z >= 128) return kStream128;
    for (int c = 0; c < kNumTiled; ++c) {
        int64_t tiles = ((d->m + kConfigs[c].bm - 1) / kConfigs[c].bm) * ((d->n + kConfigs[c].bn - 1) / kConfigs[c].bn) * z;
        if (tiles >= 256) return c;
    }
    return kNumTiled - 1;
}

template <typename TD>
int launch_exact(hipStream_t st, GemmShape s, const nhip_gemm_desc *d, const void *a, const void *b, void *out) {
    s.tiles_m = int((s.m + 63) / 64);
    s.tiles_n = int((s.n + 63) / 64);
    dim3 grid(s.tiles_m * s.tiles_n, unsigned(batch_count(d)));
    StoreEpilogue<TD> epi{static_cast<TD *>(out)};
    if (d->a_dtype == NHIP_F32)
        hipLaunchKernelGGL((gemm_exact<float, float, StoreEpilogue<TD>>), grid, dim3(256), 0, st,
                           s, static_cast<const float *>(a), static_cast<const float *>(b), epi);
    else if (d->a_dtype == NHIP_BF16)
        hipLaunchKernelGGL((gemm_exact<bf16_t, bf16_t, StoreEpilogue<TD>>), grid, dim3(256), 0, st,
                           s, static_cast<const bf16_t *>(a), static_cast<const bf16_t *>(b), epi);
    else
        hipLaunchKernelGGL((gemm_exact<f16_t, f16_t, StoreEpilogue<TD>>), grid, dim3(256), 0, st,
                           s, static_cast<const f16_t *>(a), static_cast<const f16_t *>(b), epi);
    return check(hipGetLastError(), "gemm_exact launch");
}

template <bool F16, int BM, int BN, int BK, int WM, int WN, bool AT, bool BT>
int launch_mfma_cfg(hipStream_t st, GemmShape s, int64_t z, const void *a, const void *b, void *out, int dtype) {
    s.tiles_m = int((s.m + BM - 1) / BM);
    s.tiles_n = int((s.n + BN - 1) / BN);
    constexpr int lds = gemm_mfma_lds_bytes<BM, BN, BK, AT, BT>();
    auto kern = gemm_mfma<F16, BM, BN, BK, WM, WN, AT, BT, AnyStore>;
    static bool attr = false;
    if (!attr) {
        if (check(hipFuncSetAttribute(reinterpret_cast<const void *>(kern), hipFuncAttributeMaxDynamicSharedMemorySize, lds),
                  "hipFuncSetAttribute"))
            return 1;
        attr = true;
    }
    dim3 grid(s.tiles_m * s.tiles_n, unsigned(z));
    hipLaunchKernelGGL(kern, grid, dim3(WM * WN * 64), lds, st, s, static_cast<const uint16_t *>(a),
                       static_cast<const uint16_t *>(b), AnyStore{out, dtype});
    return check(hipGetLastError(), "gemm_mfma launch");
}

template <bool F16, int BK, int WN, bool AT, bool BT, bool BUF, int KL = 0>
int launch_stream_kernel(hipStream_t st, const GemmShape &s, int64_t z, const void *a, const void *b, void *out,
                         int dtype, int splits) {
    constexpr int lds = gemm_stream_lds_bytes<BK, WN>();
    auto kern = gemm_stream<F16, BK, WN, AT, BT, BUF, KL>;
    static bool attr = false;
    if (!attr) {
        if (check(hipFuncSetAttribute(reinterpret_cast<const void *>(kern), hipFuncAttributeMaxDynamicSharedMemorySize, lds),
                  "hipFuncSetAttribute"))
            return 1;
        attr = true;
    }
    dim3 grid(s.tiles_m * s.tiles_n, unsigned(z), unsigned(splits));
    hipLaunchKernelGGL(kern, grid, dim3(128 * WN), lds, st, s, static_cast<const uint16_t *>(a),
                       static_cast<const uint16_t *>(b), AnyStore{out, dtype});
    return check(hipGetLastError(), "gemm_stream launch");
}

template <bool F16, bool AT, bool BT, bool BUF>
int launch_stream128_kernel(hipStream_t st, const GemmShape &s, int64_t z, const void *a, const void *b, void *out,
                            int dtype, int splits) {
    constexpr int lds = gemm_stream_lds_bytes<64, 2, 128>();
    auto kern = gemm_stream128<F16, AT, BT, BUF>;
    static bool attr = false;
    if (!attr) {
        if (check(hipFuncSetAttribute(reinterpret_cast<const void *>(kern), hipFuncAttributeMaxDynamicSharedMemorySize, lds),
                  "hipFuncSetAttribute"))
            return 1;
        attr = true;
    }
    dim3 grid(s.tiles_m * s.tiles_n, unsigned(z), unsigned(splits));
    hipLaunchKernelGGL(kern, grid, dim3(256), lds, st, s, static_cast<const uint16_t *>(a),
                       static_cast<const uint16_t *>(b), AnyStore{out, dtype});
    return check(hipGetLastError(), "gemm_stream128 launch");
}

template <bool F16, bool AT, bool BT>
int launch_stream128(hipStream_t st, GemmShape s, int64_t z, const void *a, const void *b, void *out, int dtype,
                     int splits = 1) {
    s.tiles_m = int((s.m + 127) / 128);
    s.tiles_n = int((s.n + 127) / 128);
    if (stream_buffer_ok(s.m, s.n, s.k, AT, BT, s.a_m, s.a_k, s.b_k, s.b_n))
        return launch_stream128_kernel<F16, AT, BT, true>(st, s, z, a, b, out, dtype, splits);
    return launch_stream128_kernel<F16, AT, BT, false>(st, s, z, a, b, out, dtype, splits);
}

// KL 1, the cross-tile fragment prefetch (buffer-load path only; the 64-bit-address path runs without it), 2,
// the ping-pong k loop, or 3, the two-stage k-64 loop placed by hand
template <bool F16, int BK, int WN, bool AT, bool BT, int KL = 0>
int launch_stream(hipStream_t st, GemmShape s, int64_t z, const void *a, const void *b, void *out, int dtype,
                  int splits = 1) {
    s.tiles_m = int((s.m + 255) / 256);
    s.tiles_n = int((s.n + 255) / 256);
    if constexpr (KL == 2 || KL == 3) {
        if (stream_buffer_ok(s.m, s.n, s.k, AT, BT, s.a_m, s.a_k, s.b_k, s.b_n))
            return launch_stream_kernel<F16, BK, WN, AT, BT, true, KL>(st, s, z, a, b, out, dtype, splits);
        return launch_stream_kernel<F16, BK, WN, AT, BT, false, KL>(st, s, z, a, b, out, dtype, splits);
    }
    if constexpr (KL == 1)
        if (stream_buffer_ok(s.m, s.n, s.k, AT, BT, s.a_m, s.a_k, s.b_k, s.b_n))
            return launch_stream_kernel<F16, BK, WN, AT, BT, true, 1>(st, s, z, a, b, out, dtype, splits);
    if (stream_buffer_ok(s.m, s.n, s.k, AT, BT, s.a_m, s.a_k, s.b_k, s.b_n))
        return launch_stream_kernel<F16, BK, WN, AT, BT, true>(st, s, z, a, b, out, dtype, splits);
    return launch_stream_kernel<F16, BK, WN, AT, BT, false>(st, s, z, a, b, out, dtype, splits);
}

// CUs of the current device (the persistent kernel's grid), asked once per device
int device_cus() {
    static int cus[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (!cus[dev]) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cus[dev] = n;
    }
    return cus[dev];
}

template <bool F16, bool AT, bool BT, bool BUF>
int launch_stream_persist_kernel(hipStream_t st, const GemmShape &s, const void *a, const void *b, void *out,
                                 int dtype) {
    constexpr int lds = gemm_stream_persist_lds_bytes();
    auto kern = gemm_stream_persist<F16, 64, 4, AT, BT, BUF>;
    static bool attr = false;
    if (!attr) {
        if (check(hipFuncSetAttribute(reinterpret_cast<const void *>(kern), hipFuncAttributeMaxDynamicSharedMemorySize, lds),
                  "hipFuncSetAttribute"))
            return 1;
        attr = true;
    }
    const int tiles = s.tiles_m * s.tiles_n;
    const int cus = device_cus();
    dim3 grid(tiles < cus ? tiles : cus, 1, 1);
    hipLaunchKernelGGL(kern, grid, dim3(512), lds, st, s, static_cast<const uint16_t *>(a),
                       static_cast<const uint16_t *>(b), AnyStore{out, dtype});
    return check(hipGetLastError(), "gemm_stream_persist launch");
}

// One batch: the persistent kernel; batched dots take the one-workgroup-a-tile kernel
template <bool F16, bool AT, bool BT>
int launch_stream_persist(hipStream_t st, GemmShape s, int64_t z, const void *a, const void *b, void *out, int dtype) {
    if (z != 1) return launch_stream<F16, 64, 4, AT, BT>(st, s, z, a, b, out, dtype);
    s.tiles_m = int((s.m + 255) / 256);
    s.tiles_n = int((s.n + 255) / 256);
    if (stream_buffer_ok(s.m, s.n, s.k, AT, BT, s.a_m, s.a_k, s.b_k, s.b_n))
        return launch_stream_persist_kernel<F16, AT, BT, true>(st, s, a, b, out, dtype);
    return launch_stream_persist_kernel<F16, AT, BT, false>(st, s, a, b, out, dtype);
}


template <bool F16, bool AT, bool BT>
int launch_mfma_layout(hipStream_t st, int cfg, GemmShape s, int64_t z, const void *a, const void *b, void *out, int dtype) {
    switch (cfg) {
        case kStream4w: return launch_stream<F16, 64, 2, AT, BT>(st, s, z, a, b, out, dtype);
        case kStream8w: return launch_stream<F16, 64, 4, AT, BT>(st, s, z, a, b, out, dtype);
        case kStream8w32: return launch_stream<F16, 32, 4, AT, BT>(st, s, z, a, b, out, dtype);
        case kStream8wX: return launch_stream<F16, 32, 4, AT, BT, 1>(st, s, z, a, b, out, dtype);
        case kStream8wP: return launch_stream<F16, 32, 4, AT, BT, 2>(st, s, z, a, b, out, dtype);
        case kStream4wX: return launch_stream<F16, 32, 2, AT, BT, 1>(st, s, z, a, b, out, dtype);
        case kStream4w64X: return launch_stream<F16, 64, 2, AT, BT, 3>(st, s, z, a, b, out, dtype);
        case kStream8w64X: return launch_stream<F16, 64, 4, AT, BT, 3>(st, s, z, a, b, out, dtype);
        case kStream128: return launch_stream128<F16, AT, BT>(st, s, z, a, b, out, dtype);
        case kStreamPersist: return launch_stream_persist<F16, AT, BT>(st, s, z, a, b, out, dtype);
        case 0: return launch_mfma_cfg<F16, 256, 256, 64, 2, 4, AT, BT>(st, s, z, a, b, out, dtype);
        case 1: return launch_mfma_cfg<F16, 256, 128, 64, 2, 2, AT, BT>(st, s, z, a, b, out, dtype);
        case 2: return launch_mfma_cfg<F16, 128, 256, 64, 2, 2, AT, BT>(st, s, z, a, b, out, dtype);
        case 3: return launch_mfma_cfg<F16, 128, 128, 64, 2, 2, AT, BT>(st, s, z, a, b, out, dtype);
        case 4: return launch_mfma_cfg<F16, 128, 64, 64, 2, 2, AT, BT>(st, s, z, a, b, out, dtype);
        default: return launch_mfma_cfg<F16, 64, 64, 64, 2, 2, AT, BT>(st, s, z, a, b, out, dtype);
    }
}

template <bool F16>
int launch_mfma(hipStream_t st, int cfg, GemmShape s, int64_t z, const void *a, const void *b, void *out, int dtype,
                bool at, bool bt) {
    if (at) return bt ? launch_mfma_layout<F16, true, true>(st, cfg, s, z, a, b, out, dtype)
                      : launch_mfma_layout<F16, true, false>(st, cfg, s, z, a, b, out, dtype);
    return bt ? launch_mfma_layout<F16, false, true>(st, cfg, s, z, a, b, out, dtype)
              : launch_mfma_layout<F16, false, false>(st, cfg, s, z, a, b, out, dtype);
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// Whether the MFMA kernel reads these operands: each k-contiguous or mn-contiguous, with 16-byte aligned
// rows along its contiguous dimension. `at` / `bt` say an operand is mn-contiguous.
bool mfma_ready(const nhip_gemm_desc *d, const void *a, const void *b, bool &at, bool &bt) {
    if (d->a_dtype != d->b_dtype || d->a_dtype == NHIP_F32) return false;
    if (!aligned16(a) || !aligned16(b)) return false;
    if (d->a_k == 1 && d->k % 8 == 0 && (d->a_m % 8 == 0 || d->m == 1)) at = false;
    else if (d->a_m == 1 && d->m % 8 == 0 && d->a_k % 8 == 0) at = true;
    else return false;
    if (d->b_k == 1 && d->k % 8 == 0 && (d->b_n % 8 == 0 || d->n == 1)) bt = false;
    else if (d->b_n == 1 && d->n % 8 == 0 && d->b_k % 8 == 0) bt = true;
    else return false;
    for (int i = 0; i < d->nbatch; ++i)
        if (d->a_batch[i] % 8 || d->b_batch[i] % 8) return false;
    return true;
}

}  // namespace

size_t splitk_workspace_bytes(const nhip_gemm_desc *d) {
    return d->splits > 1 ? size_t(d->splits) * size_t(batch_count(d)) * size_t(d->m) * size_t(d->n) * sizeof(float) : 0;
}

// Split-k through the streamed 8-wave kernel: partials into the workspace as [split][batch][m][n] float32, then
// the ordered sum into D.
int gemm_splitk_on(hipStream_t st, const nhip_gemm_desc *d, const void *a, const void *b, void *out, void *ws) {
    if (d->splits <= 1) return gemm_on(st, d, a, b, out);
    if (d->nbatch < 0 || d->nbatch > 3) return fail("nhip_gemm_splitk: at most 3 batch axes");
    int64_t z = batch_count(d);
    if (d->m == 0 || d->n == 0 || z == 0) return 0;
    if (z > 65535 || d->splits > 64) return fail("nhip_gemm_splitk: more than 65535 batches or 64 splits");
    bool at = false, bt = false;
    if (!mfma_ready(d, a, b, at, bt) || d->k % (64 * int64_t(d->splits)))
        return fail("nhip_gemm_splitk: needs 16-bit operands in an MFMA layout and k a multiple of 64 * splits");
    if (!ws) return fail("nhip_gemm_splitk: no workspace");
    // partial products: contiguous [split][batch...][m][n]
    GemmShape p = shape_of(d);
    p.k = d->k / d->splits;
    p.d_m = d->n;
    p.d_n = 1;
    int64_t stride = d->m * d->n;
    for (int i = d->nbatch - 1; i >= 0; --i) {
        p.d_batch[i] = stride;
        stride *= d->batch[i];
    }
    p.d_split = stride;
    int rc;
    bool f16 = d->a_dtype == NHIP_F16;
    // the partial products come from the 128 x 128 streamed kernel when the caller picked it (config 9), else
    // from the 256 x 256 one
#define NHIP_SPLIT(FF, AA, BB)                                                                      \
    rc = d->config == kStream128 ? launch_stream128<FF, AA, BB>(st, p, z, a, b, ws, NHIP_F32, d->splits) \
                                 : launch_stream<FF, 64, 4, AA, BB>(st, p, z, a, b, ws, NHIP_F32, d->splits)
    if (f16) {
        if (at) { if (bt) NHIP_SPLIT(true, true, true); else NHIP_SPLIT(true, true, false); }
        else { if (bt) NHIP_SPLIT(true, false, true); else NHIP_SPLIT(true, false, false); }
    } else {
        if (at) { if (bt) NHIP_SPLIT(false, true, true); else NHIP_SPLIT(false, true, false); }
        else { if (bt) NHIP_SPLIT(false, false, true); else NHIP_SPLIT(false, false, false); }
    }
#undef NHIP_SPLIT
    if (rc) return rc;
    GemmShape s = shape_of(d);
    const int64_t total = z * d->m * d->n;
    int64_t blocks = (total + 255) / 256;
    if (blocks > 8192) blocks = 8192;
    hipLaunchKernelGGL(gemm_splitk_reduce, dim3(unsigned(blocks)), dim3(256), 0, st, s, static_cast<const float *>(ws),
                       d->splits, total, AnyStore{out, d->d_dtype});
    return check(hipGetLastError(), "gemm split-k reduce launch");
}

int gemm_on(hipStream_t st, const nhip_gemm_desc *d, const void *a, const void *b, void *out) {
    if (d->nbatch < 0 || d->nbatch > 3) return fail("nhip_gemm: at most 3 batch axes");
    if ((d->a_dtype == NHIP_F32) != (d->b_dtype == NHIP_F32))
        return fail("nhip_gemm: operands must both be float32 or both 16-bit");
    GemmShape s = shape_of(d);
    int64_t z = batch_count(d);
    if (d->m == 0 || d->n == 0 || z == 0) return 0;
    if (z > 65535) return fail("nhip_gemm: more than 65535 batches");
    bool at = false, bt = false;
    if (d->k > 0 && mfma_ready(d, a, b, at, bt)) {  // k == 0 folds nothing: the exact kernel writes zeros
        int cfg = d->config < 0 ? default_config(d) : d->config;
        if (cfg >= kNumConfigs) return fail("nhip_gemm: no tile config " + std::to_string(cfg));
        if (((cfg == kStream4w || cfg == kStream8w || cfg == kStream128 || cfg == kStreamPersist || cfg == kStream4w64X ||
              cfg == kStream8w64X) &&
             d->k % 64) ||
            ((cfg == kStream8w32 || cfg == kStream8wX || cfg == kStream8wP || cfg == kStream4wX) && d->k % 32))
            return fail("nhip_gemm: the streamed configs need k to be a multiple of their k tile");
        if (d->a_dtype == NHIP_F16) return launch_mfma<true>(st, cfg, s, z, a, b, out, d->d_dtype, at, bt);
        return launch_mfma<false>(st, cfg, s, z, a, b, out, d->d_dtype, at, bt);
    }
    switch (d->d_dtype) {
        case NHIP_F32: return launch_exact<float>(st, s, d, a, b, out);
        case NHIP_BF16: return launch_exact<bf16_t>(st, s, d, a, b, out);
        default: return launch_exact<f16_t>(st, s, d, a, b, out);
    }
}

__global__ void fill_kernel(unsigned char *dst, size_t n, unsigned char v) {
    size_t i = (size_t(blockIdx.x) * blockDim.x + threadIdx.x) * 16;
    size_t stride = size_t(gridDim.x) * blockDim.x * 16;
    uint32_t w = v * 0x01010101u;
    for (; i < n; i += stride) {
        if (i + 16 <= n && (reinterpret_cast<uintptr_t>(dst + i) & 15) == 0) {
            *reinterpret_cast<uint4 *>(dst + i) = make_uint4(w, w, w, w);
        } else {
            for (size_t j = i; j < n && j < i + 16; ++j) dst[j] = v;
        }
    }
}

int fill_on(hipStream_t st, void *dst, size_t bytes, unsigned char value) {
    if (!bytes) return 0;
    size_t blocks = (bytes + 256 * 16 - 1) / (256 * 16);
    if (blocks > 4096) blocks = 4096;
    hipLaunchKernelGGL(fill_kernel, dim3(unsigned(blocks)), dim3(256), 0, st, static_cast<unsigned char *>(dst), bytes,
                       value);
    return check(hipGetLastError(), "fill launch");
}

// ---- linear cross entropy (lumen/reference/mod.rs:1092-1120) ---------------------------------------------

// exp(x) for x <= 0 in float32: x log2 e as a rounded product and its fma residual, the hardware exp2 of the
// product times (1 + residual ln 2); within 2 ulp, results below 2^-126 flushed to zero.
__device__ __forceinline__ float lce_exp(float x) {
    const float hi = x * 1.4426950216293335f;
    float lo = fmaf(x, 1.4426950216293335f, -hi) + x * 1.9259629890910901e-08f;
    lo = __builtin_isinf(x) ? 0.0f : lo;
    const float r = __builtin_amdgcn_exp2f(hi);
    return r * fmaf(lo, 0.6931471805599453f, 1.0f);
}

// One workgroup a row of float32 logits [rows, v], read once: each thread keeps a running maximum and the
// float64 sum of exp(logit - that maximum) (four float32 terms at a time), rescaled when the maximum grows; the
// threads' sums are rescaled to
// the row maximum and added in float64 (float32 exponentials within 2 ulp where the reference takes float64
// ones). lse = max + log(sum) rounded to float32; the loss is lse minus the logit of the clamped class,
// rounded once. out[r0 + row] = loss, out[b + r0 + row] = lse. 16-byte loads when rows are a multiple of 4.
__device__ __forceinline__ void lce_add(float x, float &m, double &sum) {
    if (x > m) {  // a new running maximum: earlier terms scale by exp(m - x) (0 when m is -inf)
        sum *= double(lce_exp(m - x));
        m = x;
    }
    sum += double(lce_exp(x - m));
}

__global__ __launch_bounds__(256) void lce_rows_kernel(const float *__restrict__ logits, int64_t v,
                                                       const void *__restrict__ target, int t64,
                                                       float *__restrict__ out, int64_t b, int64_t r0) {
    __shared__ float smax[4];
    __shared__ double ssum[4];
    const int64_t row = blockIdx.x;
    const float *x = logits + row * v;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    float m = -INFINITY;
    double sum = 0.0;
    if ((v & 3) == 0) {
        auto add4 = [&](const float4 &q) {
            const float mq = fmaxf(fmaxf(q.x, q.y), fmaxf(q.z, q.w));
            if (mq > m) {  // one rescale for four logits
                sum *= double(lce_exp(m - mq));
                m = mq;
            }
            // four float32 terms (each at most 1) summed in float32, then added in float64
            sum += double((lce_exp(q.x - m) + lce_exp(q.y - m)) + (lce_exp(q.z - m) + lce_exp(q.w - m)));
        };
        int64_t j = 4 * tid;
        for (; j + 3 * 1024 < v; j += 4 * 1024) {  // four loads in flight before any is used
            float4 q[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) q[u] = *reinterpret_cast<const float4 *>(x + j + u * 1024);
#pragma unroll
            for (int u = 0; u < 4; ++u) add4(q[u]);
        }
        for (; j < v; j += 1024) add4(*reinterpret_cast<const float4 *>(x + j));
    } else {
        for (int64_t j = tid; j < v; j += 256) lce_add(x[j], m, sum);
    }
    float rm = m;
    for (int o = 32; o > 0; o >>= 1) rm = fmaxf(rm, __shfl_xor(rm, o, 64));
    if (lane == 0) smax[wave] = rm;
    __syncthreads();
    rm = fmaxf(fmaxf(smax[0], smax[1]), fmaxf(smax[2], smax[3]));
    sum = m == -INFINITY ? 0.0 : sum * double(lce_exp(m - rm));
    for (int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o, 64);
    if (lane == 0) ssum[wave] = sum;
    __syncthreads();
    if (tid == 0) {
        sum = ((ssum[0] + ssum[1]) + ssum[2]) + ssum[3];
        const int64_t t = t64 ? static_cast<const int64_t *>(target)[r0 + row] : static_cast<const int32_t *>(target)[r0 + row];
        const int64_t cls = t < 0 ? 0 : (t >= v ? v - 1 : t);
        const float l = float(double(rm) + log(sum));
        out[r0 + row] = float(double(l) - double(x[cls]));
        out[b + r0 + row] = l;
    }
}

// The fused form: the streamed GEMM's store runs LceOut instead of writing logits. gemm_stream_tile hands a
// lane four consecutive columns of one row, and the 16 lanes of a DPP row (lanes 16 q .. 16 q + 15) hold the 64
// columns of one row of a wave's 64-column block (a row's lanes are all in or all out of range, rows by row
// and columns because v % 64 == 0): each block's maximum and float32 sum of exp(logit - maximum) combine
// across those lanes by DPP rotations, and the block's first lane stores them as part[row][block]; the lane
// holding the row's clamped class (read ahead with the chunk, Pre) stores that logit. lce_merge_kernel then
// reduces a row's v / 64 pairs: nothing of size [b, v] is written.
template <int CTRL>
__device__ __forceinline__ float lce_dpp(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, false));
}

struct LceOut {
    float2 *part;
    float *picked;
    const void *target;
    int t64;
    int64_t nblk;
    static constexpr int kPrefetch = 8;
    static constexpr bool kColSum = false;
    struct Pre {
        int64_t cls;
    };
    __device__ __forceinline__ Pre load(int64_t r, int64_t) const {
        const int64_t t = t64 ? static_cast<const int64_t *>(target)[r] : static_cast<const int32_t *>(target)[r];
        const int64_t v = nblk * 64;
        return Pre{t < 0 ? 0 : (t >= v ? v - 1 : t)};
    }
    __device__ __forceinline__ void operator()(int64_t r, int64_t c, float4 acc, const Pre &pre) const {
        // row_ror 8, row_ror 4, then the quad permutations [2,3,0,1] and [1,0,3,2]: every lane of the DPP row
        // ends with the combination of all 16
        float m = fmaxf(fmaxf(acc.x, acc.y), fmaxf(acc.z, acc.w));
        m = fmaxf(m, lce_dpp<0x128>(m));
        m = fmaxf(m, lce_dpp<0x124>(m));
        m = fmaxf(m, lce_dpp<0x4e>(m));
        m = fmaxf(m, lce_dpp<0xb1>(m));
        // exp(x - m) = 2^((x - m) log2 e): the difference is exact near the maximum, where the terms matter
        constexpr float kLog2e = 1.4426950408889634f;
        float e = 0.0f;
        if (m != -INFINITY)
            e = (__builtin_amdgcn_exp2f((acc.x - m) * kLog2e) + __builtin_amdgcn_exp2f((acc.y - m) * kLog2e)) +
                (__builtin_amdgcn_exp2f((acc.z - m) * kLog2e) + __builtin_amdgcn_exp2f((acc.w - m) * kLog2e));
        e += lce_dpp<0x128>(e);
        e += lce_dpp<0x124>(e);
        e += lce_dpp<0x4e>(e);
        e += lce_dpp<0xb1>(e);
        if ((c & 63) == 0) part[r * nblk + (c >> 6)] = make_float2(m, e);
        if (pre.cls >= c && pre.cls < c + 4) {
            const int64_t q = pre.cls - c;
            picked[r] = q == 0 ? acc.x : (q == 1 ? acc.y : (q == 2 ? acc.z : acc.w));
        }
    }
};

template <bool F16, bool BUF>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2))) void lce_gemm_kernel(
    GemmShape s, const uint16_t *__restrict__ a, const uint16_t *__restrict__ b, LceOut out) {
    extern __shared__ __align__(1024) char smem[];
    gemm_stream_tile<F16, 64, 4, false, false, BUF, LceOut, 256, false>(s, a, b, out, smem);
}

// One wavefront a row: the maximum of the row's block maxima, then the float64 sum of each block's sum scaled
// by exp(block maximum - row maximum) (float32 exponentials, as lce_rows_kernel); lse and loss rounded as there.
__global__ __launch_bounds__(256) void lce_merge_kernel(const float2 *__restrict__ part, const float *__restrict__ picked,
                                                        int64_t nblk, float *__restrict__ out, int64_t b) {
    const int64_t row = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= b) return;  // the whole wavefront
    const float2 *p = part + row * nblk;
    float m = -INFINITY;
    for (int64_t j = lane; j < nblk; j += 64) m = fmaxf(m, p[j].x);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
    double sum = 0.0;
    for (int64_t j = lane; j < nblk; j += 64) {
        const float2 q = p[j];
        if (q.x != -INFINITY) sum += double(q.y) * double(lce_exp(q.x - m));
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o, 64);
    if (lane == 0) {
        const float l = float(double(m) + log(sum));
        out[row] = float(double(l) - double(picked[row]));
        out[b + row] = l;
    }
}

// Whether `d` takes the fused form (16-bit operands, k a multiple of the GEMM's k tile, whole 64-class blocks).
bool lce_fused(const nhip_lce_desc *d) {
    return d->dtype != NHIP_F32 && d->b > 0 && d->d > 0 && d->d % 64 == 0 && d->v % 64 == 0;
}

size_t lce_part_bytes(const nhip_lce_desc *d) { return (size_t(d->b) * size_t(d->v / 64) * 8 + 255) / 256 * 256; }

size_t lce_workspace_bytes(const nhip_lce_desc *d) {
    if (d->b <= 0 || d->v <= 0) return 0;
    if (lce_fused(d)) {
        // the partials and picked logits, and at least one row of logits for the unfused form (operands that
        // are not 16-byte aligned)
        const size_t fused = lce_part_bytes(d) + size_t(d->b) * 4, row = size_t(d->v) * 4;
        return fused > row ? fused : row;
    }
    const int64_t chunk = d->chunk_rows <= 0 || d->chunk_rows > d->b ? d->b : d->chunk_rows;
    return size_t(chunk) * size_t(d->v) * 4;
}

int lce_fused_on(hipStream_t st, const nhip_lce_desc *d, const void *h, const void *w, const void *target, float *out,
                 void *ws) {
    GemmShape s;
    std::memset(&s, 0, sizeof(s));
    s.m = d->b;
    s.n = d->v;
    s.k = d->d;
    s.a_m = d->d;
    s.a_k = 1;
    s.b_k = 1;
    s.b_n = d->d;
    s.d_m = d->v;
    s.d_n = 1;
    s.tiles_m = int((d->b + 255) / 256);
    s.tiles_n = int((d->v + 255) / 256);
    LceOut o;
    o.part = static_cast<float2 *>(ws);
    o.picked = reinterpret_cast<float *>(static_cast<char *>(ws) + lce_part_bytes(d));
    o.target = target;
    o.t64 = d->target_dtype == NHIP_LCE_I64;
    o.nblk = d->v / 64;
    constexpr int lds = gemm_stream_lds_bytes<64, 4>();
    const bool buf = stream_buffer_ok(s.m, s.n, s.k, false, false, s.a_m, s.a_k, s.b_k, s.b_n);
    const bool f16 = d->dtype == NHIP_F16;
    auto kern = f16 ? (buf ? lce_gemm_kernel<true, true> : lce_gemm_kernel<true, false>)
                    : (buf ? lce_gemm_kernel<false, true> : lce_gemm_kernel<false, false>);
    if (int rc = check(hipFuncSetAttribute(reinterpret_cast<const void *>(kern),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, lds),
                       "hipFuncSetAttribute"))
        return rc;
    if (int64_t(s.tiles_m) * s.tiles_n > 0x7fffffff) return fail("nhip_linear_cross_entropy: too many tiles");
    hipLaunchKernelGGL(kern, dim3(unsigned(s.tiles_m * s.tiles_n)), dim3(512), lds, st, s,
                       static_cast<const uint16_t *>(h), static_cast<const uint16_t *>(w), o);
    if (int rc = check(hipGetLastError(), "lce_gemm_kernel launch")) return rc;
    hipLaunchKernelGGL(lce_merge_kernel, dim3(unsigned((d->b + 3) / 4)), dim3(256), 0, st,
                       static_cast<const float2 *>(o.part), static_cast<const float *>(o.picked), o.nblk, out, d->b);
    return check(hipGetLastError(), "lce_merge_kernel launch");
}

int64_t lce_chunk(const nhip_lce_desc *d) {
    return d->chunk_rows <= 0 || d->chunk_rows > d->b ? d->b : d->chunk_rows;
}

int lce_on(hipStream_t st, const nhip_lce_desc *d, const void *h, const void *w, const void *target, float *out,
           void *ws) {
    if (d->b < 0 || d->v < 1 || d->d < 0) return fail("nhip_linear_cross_entropy: needs b >= 0, v >= 1, d >= 0");
    if (d->dtype != NHIP_F32 && d->dtype != NHIP_BF16 && d->dtype != NHIP_F16)
        return fail("nhip_linear_cross_entropy: h and w must be float32, bf16 or f16");
    if (d->target_dtype != NHIP_LCE_I32 && d->target_dtype != NHIP_LCE_I64)
        return fail("nhip_linear_cross_entropy: targets must be int32 or int64");
    if (d->b == 0) return 0;
    if (!ws) return fail("nhip_linear_cross_entropy: no workspace");
    int64_t chunk = lce_chunk(d);
    if (lce_fused(d)) {
        if (aligned16(h) && aligned16(w)) return lce_fused_on(st, d, h, w, target, out, ws);
        // unaligned operands: the unfused form, as many rows a pass as the fused form's workspace holds
        const int64_t fit = int64_t(lce_workspace_bytes(d) / (size_t(d->v) * 4));
        chunk = chunk < fit ? chunk : fit;
    }
    const int64_t esize = d->dtype == NHIP_F32 ? 4 : 2;
    for (int64_t r0 = 0; r0 < d->b; r0 += chunk) {
        const int64_t rows = d->b - r0 < chunk ? d->b - r0 : chunk;
        nhip_gemm_desc g;
        std::memset(&g, 0, sizeof(g));
        g.m = rows;
        g.n = d->v;
        g.k = d->d;
        g.a_dtype = g.b_dtype = d->dtype;
        g.d_dtype = NHIP_F32;
        g.a_m = d->d;  // h rows
        g.a_k = 1;
        g.b_k = 1;     // w [v, d]: B[k][n] = w[n * d + k]
        g.b_n = d->d;
        g.d_m = d->v;
        g.d_n = 1;
        g.config = -1;
        g.splits = 1;
        if (int rc = gemm_on(st, &g, static_cast<const char *>(h) + r0 * d->d * esize, w, ws)) return rc;
        if (rows > 0x7fffffff) return fail("nhip_linear_cross_entropy: more than 2^31 rows a chunk");
        hipLaunchKernelGGL(lce_rows_kernel, dim3(unsigned(rows)), dim3(256), 0, st, static_cast<const float *>(ws),
                           d->v, target, int(d->target_dtype == NHIP_LCE_I64), out, d->b, r0);
        if (int rc = check(hipGetLastError(), "lce_rows_kernel launch")) return rc;
    }
    return 0;
}

}  // namespace nhip

using namespace nhip;

extern "C" {

int nhip_gemm(const nhip_gemm_desc *desc, const void *a, const void *b, void *d) {
    hipStream_t s = stream_of_current();
    if (!s) return fail("no HIP stream: call nhip_set_device first");
    return gemm_on(s, desc, a, b, d);
}

int nhip_gemm_config_count(int *count) {
    *count = kNumConfigs;
    return 0;
}

int nhip_gemm_splitk(const nhip_gemm_desc *desc, const void *a, const void *b, void *d, void *workspace) {
    hipStream_t s = stream_of_current();
    if (!s) return fail("no HIP stream: call nhip_set_device first");
    return gemm_splitk_on(s, desc, a, b, d, workspace);
}

int nhip_gemm_workspace(const nhip_gemm_desc *desc, size_t *bytes) {
    *bytes = splitk_workspace_bytes(desc);
    return 0;
}

int nhip_linear_cross_entropy(const nhip_lce_desc *desc, const void *h, const void *w, const void *target, float *out,
                              void *workspace) {
    hipStream_t s = stream_of_current();
    if (!s) return fail("no HIP stream: call nhip_set_device first");
    return lce_on(s, desc, h, w, target, out, workspace);
}

int nhip_linear_cross_entropy_workspace(const nhip_lce_desc *desc, size_t *bytes) {
    *bytes = lce_workspace_bytes(desc);
    return 0;
}

}  // extern "C"
