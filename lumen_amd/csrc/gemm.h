// dot_general kernels for gfx950.
//
//  * gemm_mfma: bf16/f16 operands on the matrix cores (v_mfma_f32_32x32x16_{bf16,f16}), float32
//    accumulation, LDS-staged double-buffered tiles. Each operand may be k-contiguous or mn-contiguous in
//    memory: an mn-contiguous tile is kept [k][mn] in LDS and its MFMA fragments are read transposed with
//    ds_read_tr16_b64, so transposed operands (the weight and input gradients) need no layout pass.
//  * gemm_exact: any strides and dtypes; each output is the reference's sequential k-order fold with the
//    product and every partial sum rounded to float32 (lumen/reference/mod.rs:981-993), so float32 dots are
//    bit-identical to the reference interpreter.
//
// Both take an Epilogue functor (row, col, batch offset, float32 value) so generated plans can fuse
// elementwise work after a dot into its stores.
#pragma once

#include "device_common.h"

namespace nhipk {

struct GemmShape {
    int64_t m, n, k;
    int32_t nbatch;
    int64_t batch[3];
    int64_t a_batch[3], b_batch[3], d_batch[3];
    int64_t a_m, a_k, b_k, b_n, d_m, d_n;
    int32_t tiles_m, tiles_n;
};

// Element offsets of batch `z` in A, B and D.
__device__ __forceinline__ void batch_offsets(const GemmShape &s, int64_t z, int64_t &oa, int64_t &ob, int64_t &od) {
    oa = ob = od = 0;
    for (int i = s.nbatch - 1; i >= 0; --i) {
        int64_t idx = z % s.batch[i];
        z /= s.batch[i];
        oa += idx * s.a_batch[i];
        ob += idx * s.b_batch[i];
        od += idx * s.d_batch[i];
    }
}

// Plain store of the accumulator into D (strided), rounded once to D's dtype.
template <typename TD>
struct StoreEpilogue {
    TD *d;
    __device__ __forceinline__ void operator()(const GemmShape &s, int64_t od, int64_t row, int64_t col, float v) const {
        store_f32_as(d + od + row * s.d_m + col * s.d_n, v);
    }
};

// Maps a linear workgroup id to a (tile_m, tile_n) pair: workgroups are dealt round-robin to the 8 XCDs,
// so consecutive ids are first regrouped per XCD (each XCD gets a contiguous run of tiles and its own L2
// sees neighbouring tiles), then walked in column groups of 8 tile-rows that share B tiles.
__device__ __forceinline__ void tile_of(int pid, int tiles_m, int tiles_n, int &tm, int &tn) {
    int total = tiles_m * tiles_n;
    if (total % 8 == 0) {
        int per = total / 8;
        pid = (pid % 8) * per + pid / 8;
    }
    const int group = 8;
    int width = group * tiles_n;
    int g = pid / width;
    int first_m = g * group;
    int rows = min(tiles_m - first_m, group);
    int in = pid % width;
    tm = first_m + in % rows;
    tn = in / rows;
}

// ---- exact fold --------------------------------------------------------------------------------------

template <typename TA, typename TB, class Epi>
__global__ __launch_bounds__(256) void gemm_exact(GemmShape s, const TA *__restrict__ a, const TB *__restrict__ b, Epi epi) {
    constexpr int BM = 64, BN = 64, BK = 16;
    __shared__ float As[BK][BM + 1];
    __shared__ float Bs[BK][BN + 1];
    int tm, tn;
    tile_of(blockIdx.x, s.tiles_m, s.tiles_n, tm, tn);
    int64_t oa, ob, od;
    batch_offsets(s, blockIdx.y, oa, ob, od);
    const int64_t m0 = int64_t(tm) * BM, n0 = int64_t(tn) * BN;
    const int tx = threadIdx.x % 16, ty = threadIdx.x / 16;
    float acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = 0.0f;
    for (int64_t k0 = 0; k0 < s.k; k0 += BK) {
        for (int e = threadIdx.x; e < BK * BM; e += 256) {
            int kk = e / BM, mm = e % BM;
            int64_t gm = m0 + mm, gk = k0 + kk;
            As[kk][mm] = (gm < s.m && gk < s.k) ? load_as_f32(a + oa + gm * s.a_m + gk * s.a_k) : 0.0f;
        }
        for (int e = threadIdx.x; e < BK * BN; e += 256) {
            int kk = e / BN, nn = e % BN;
            int64_t gn = n0 + nn, gk = k0 + kk;
            Bs[kk][nn] = (gn < s.n && gk < s.k) ? load_as_f32(b + ob + gk * s.b_k + gn * s.b_n) : 0.0f;
        }
        __syncthreads();
        int kmax = int(min<int64_t>(BK, s.k - k0));
        for (int kk = 0; kk < kmax; ++kk) {
            float av[4], bv[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) av[i] = As[kk][ty + 16 * i];
#pragma unroll
            for (int j = 0; j < 4; ++j) bv[j] = Bs[kk][tx + 16 * j];
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = __fadd_rn(acc[i][j], __fmul_rn(av[i], bv[j]));
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            int64_t r = m0 + ty + 16 * i, c = n0 + tx + 16 * j;
            if (r < s.m && c < s.n) epi(s, od, r, c, acc[i][j]);
        }
}

// ---- MFMA -----------------------------------------------------------------------------------------------

template <bool F16>
struct Mfma;
template <>
struct Mfma<false> {
    __device__ __forceinline__ static f32x16_t run(uint4 a, uint4 b, f32x16_t c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                        c, 0, 0, 0);
    }
};
template <>
struct Mfma<true> {
    __device__ __forceinline__ static f32x16_t run(uint4 a, uint4 b, f32x16_t c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), c,
                                                       0, 0, 0);
    }
};

// LDS row pitch in 16-bit elements: BK plus 8 so that 8 lanes reading 16 B at one k offset from 8
// consecutive rows hit disjoint banks.
template <int BK>
struct Pitch {
    static constexpr int value = BK + 8;
};

// Output of any float dtype chosen at run time (one kernel instantiation serves all three).
// The dtype branch is taken once, outside the unrolled store loops (a branch per element keeps the
// compiler from unrolling them, which sends the accumulators to scratch memory).
struct AnyStore {
    void *d;
    int32_t dtype;  // 0 f32, 1 bf16, 2 f16
    template <class F>
    __device__ __forceinline__ void visit(F &&f) const {
        if (dtype == 0) f(StoreEpilogue<float>{static_cast<float *>(d)});
        else if (dtype == 1) f(StoreEpilogue<bf16_t>{static_cast<bf16_t *>(d)});
        else f(StoreEpilogue<f16_t>{static_cast<f16_t *>(d)});
    }
};

typedef short gv4i16_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) gv4i16_t glds_v4i16_t;

// Two transposed 64-bit LDS reads, 4 rows apart, of a [k][mn] tile: 8 consecutive k at one mn column.
__device__ __forceinline__ uint4 gemm_read_tr(const uint16_t *p0, const uint16_t *p1) {
    gv4i16_t a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((glds_v4i16_t *)(p0));
    gv4i16_t b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((glds_v4i16_t *)(p1));
    uint2 x = __builtin_bit_cast(uint2, a), y = __builtin_bit_cast(uint2, b);
    return make_uint4(x.x, x.y, y.x, y.y);
}

// A tile of one operand in LDS: k-major rows ([rows][BK], read with ds_read_b128) when the operand is
// k-contiguous in memory, else mn-major rows ([BK][rows], read transposed with ds_read_tr16_b64). Either way
// global loads are 16-byte chunks along the contiguous dimension, so every load is coalesced.
template <int ROWS, int BK, bool T>
struct TileLayout {
    static constexpr int pitch = T ? ROWS + 16 : BK + 8;
    static constexpr int elems = T ? BK * pitch : ROWS * pitch;
    static constexpr int chunks_per_line = T ? ROWS / 8 : BK / 8;
};

template <bool T, int P>
struct FragLayout {
    static constexpr bool transposed = T;
    static constexpr int pitch = P;
};

template <bool F16, int BM, int BN, int BK, int WM, int WN, bool AT, bool BT, class Epi>
__global__ __launch_bounds__(WM *WN * 64) void gemm_mfma(GemmShape s, const uint16_t *__restrict__ a,
                                                           const uint16_t *__restrict__ b, Epi epi) {
    constexpr int T = WM * WN * 64;
    using LA = TileLayout<BM, BK, AT>;
    using LB = TileLayout<BN, BK, BT>;
    constexpr int TM = BM / WM, TN = BN / WN;
    constexpr int FM = TM / 32, FN = TN / 32;
    constexpr int VA = BM * BK / 8 / T, VB = BN * BK / 8 / T;
    static_assert(BM * BK / 8 % T == 0 && BN * BK / 8 % T == 0, "tile loads must divide evenly");
    extern __shared__ __align__(16) uint16_t lds[];
    uint16_t *As = lds;                 // [2][LA::elems]
    uint16_t *Bs = lds + 2 * LA::elems; // [2][LB::elems]

    int tm, tn;
    tile_of(blockIdx.x, s.tiles_m, s.tiles_n, tm, tn);
    int64_t oa, ob, od;
    batch_offsets(s, blockIdx.y, oa, ob, od);
    const int64_t m0 = int64_t(tm) * BM, n0 = int64_t(tn) * BN;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int wm = wave / WN, wn = wave % WN;
    const int h = lane >> 5, l32 = lane & 31, g = lane >> 4, s16 = lane & 15;

    const uint16_t *pa = a + oa;
    const uint16_t *pb = b + ob;

    uint4 ra[VA], rb[VB];
    auto load = [&](int64_t k0) {
#pragma unroll
        for (int v = 0; v < VA; ++v) {
            int idx = t + v * T, line = idx / LA::chunks_per_line, ch = idx % LA::chunks_per_line;
            int64_t gm, gk;
            if (AT) gk = k0 + line, gm = m0 + ch * 8;
            else gm = m0 + line, gk = k0 + ch * 8;
            bool ok = gm < s.m && gk < s.k;
            const uint16_t *src = AT ? pa + gk * s.a_k + gm : pa + gm * s.a_m + gk;
            ra[v] = ok ? *reinterpret_cast<const uint4 *>(src) : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int v = 0; v < VB; ++v) {
            int idx = t + v * T, line = idx / LB::chunks_per_line, ch = idx % LB::chunks_per_line;
            int64_t gn, gk;
            if (BT) gk = k0 + line, gn = n0 + ch * 8;
            else gn = n0 + line, gk = k0 + ch * 8;
            bool ok = gn < s.n && gk < s.k;
            const uint16_t *src = BT ? pb + gk * s.b_k + gn : pb + gn * s.b_n + gk;
            rb[v] = ok ? *reinterpret_cast<const uint4 *>(src) : make_uint4(0, 0, 0, 0);
        }
    };
    auto store = [&](int buf) {
#pragma unroll
        for (int v = 0; v < VA; ++v) {
            int idx = t + v * T, line = idx / LA::chunks_per_line, ch = idx % LA::chunks_per_line;
            *reinterpret_cast<uint4 *>(As + buf * LA::elems + line * LA::pitch + ch * 8) = ra[v];
        }
#pragma unroll
        for (int v = 0; v < VB; ++v) {
            int idx = t + v * T, line = idx / LB::chunks_per_line, ch = idx % LB::chunks_per_line;
            *reinterpret_cast<uint4 *>(Bs + buf * LB::elems + line * LB::pitch + ch * 8) = rb[v];
        }
    };
    // Fragment reads: 8 consecutive k at this lane's row (m or n), k offset 8 * half-wave.
    auto frag = [&](const uint16_t *base, int row0, int kk, auto layout) -> uint4 {
        using L = decltype(layout);
        if constexpr (L::transposed) {
            const uint16_t *p0 = base + (kk + 8 * h + s16 / 4) * L::pitch + row0 + 16 * (g & 1) + 4 * (s16 & 3);
            return gemm_read_tr(p0, p0 + 4 * L::pitch);
        } else {
            return *reinterpret_cast<const uint4 *>(base + (row0 + l32) * L::pitch + kk + 8 * h);
        }
    };
    using LAT = FragLayout<AT, LA::pitch>;
    using LBT = FragLayout<BT, LB::pitch>;

    f32x16_t acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

    const int ktiles = int((s.k + BK - 1) / BK);
    load(0);
    store(0);
    __syncthreads();
    for (int kt = 0; kt < ktiles; ++kt) {
        const int buf = kt & 1;
        if (kt + 1 < ktiles) load(int64_t(kt + 1) * BK);
        const uint16_t *as = As + buf * LA::elems;
        const uint16_t *bs = Bs + buf * LB::elems;
#pragma unroll
        for (int kk = 0; kk < BK; kk += 16) {
            uint4 fa[FM], fb[FN];
#pragma unroll
            for (int i = 0; i < FM; ++i) fa[i] = frag(as, wm * TM + i * 32, kk, LAT{});
#pragma unroll
            for (int j = 0; j < FN; ++j) fb[j] = frag(bs, wn * TN + j * 32, kk, LBT{});
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j) acc[i][j] = Mfma<F16>::run(fa[i], fb[j], acc[i][j]);
        }
        if (kt + 1 < ktiles) store(buf ^ 1);
        __syncthreads();
    }

    // C layout of a 32x32 block: lane holds column lane % 32, rows 8 * (e / 4) + 4 * (lane / 32) + e % 4.
    epi.visit([&](auto st) {
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j)
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    int64_t r = m0 + wm * TM + i * 32 + 8 * (e / 4) + 4 * h + (e % 4);
                    int64_t c = n0 + wn * TN + j * 32 + l32;
                    if (r < s.m && c < s.n) st(s, od, r, c, acc[i][j][e]);
                }
    });
}

template <int BM, int BN, int BK, bool AT, bool BT>
constexpr int gemm_mfma_lds_bytes() {
    return 2 * (TileLayout<BM, BK, AT>::elems + TileLayout<BN, BK, BT>::elems) * 2;
}


}  // namespace nhipk
