// dot_general kernels for gfx950.
//
//  * gemm_mfma: bf16/f16 operands on the matrix cores (v_mfma_f32_32x32x16_{bf16,f16}), float32
//    accumulation, LDS-staged double-buffered tiles. Both operands are read k-contiguous (A as [m][k],
//    B as [n][k]); the plan gives a transposed operand a layout pass first.
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

template <bool F16, int BM, int BN, int BK, int WM, int WN, class Epi>
__global__ __launch_bounds__(WM *WN * 64) void gemm_mfma(GemmShape s, const uint16_t *__restrict__ a,
                                                           const uint16_t *__restrict__ b, Epi epi) {
    constexpr int T = WM * WN * 64;
    constexpr int P = Pitch<BK>::value;
    constexpr int TM = BM / WM, TN = BN / WN;
    constexpr int FM = TM / 32, FN = TN / 32;
    constexpr int CH = BK / 8;                 // 16-byte chunks per tile row
    constexpr int VA = BM * CH / T, VB = BN * CH / T;
    static_assert(BM * CH % T == 0 && BN * CH % T == 0, "tile loads must divide evenly");
    extern __shared__ __align__(16) uint16_t lds[];
    uint16_t *As = lds;                        // [2][BM][P]
    uint16_t *Bs = lds + 2 * BM * P;           // [2][BN][P]

    int tm, tn;
    tile_of(blockIdx.x, s.tiles_m, s.tiles_n, tm, tn);
    int64_t oa, ob, od;
    batch_offsets(s, blockIdx.y, oa, ob, od);
    const int64_t m0 = int64_t(tm) * BM, n0 = int64_t(tn) * BN;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int wm = wave / WN, wn = wave % WN;

    const uint16_t *pa = a + oa;
    const uint16_t *pb = b + ob;

    uint4 ra[VA], rb[VB];
    auto load = [&](int64_t k0) {
#pragma unroll
        for (int v = 0; v < VA; ++v) {
            int idx = t + v * T, row = idx / CH, ch = idx % CH;
            int64_t gm = m0 + row, gk = k0 + ch * 8;
            ra[v] = (gm < s.m && gk < s.k) ? *reinterpret_cast<const uint4 *>(pa + gm * s.a_m + gk) : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int v = 0; v < VB; ++v) {
            int idx = t + v * T, row = idx / CH, ch = idx % CH;
            int64_t gn = n0 + row, gk = k0 + ch * 8;
            rb[v] = (gn < s.n && gk < s.k) ? *reinterpret_cast<const uint4 *>(pb + gn * s.b_n + gk) : make_uint4(0, 0, 0, 0);
        }
    };
    auto store = [&](int buf) {
#pragma unroll
        for (int v = 0; v < VA; ++v) {
            int idx = t + v * T, row = idx / CH, ch = idx % CH;
            *reinterpret_cast<uint4 *>(As + (buf * BM + row) * P + ch * 8) = ra[v];
        }
#pragma unroll
        for (int v = 0; v < VB; ++v) {
            int idx = t + v * T, row = idx / CH, ch = idx % CH;
            *reinterpret_cast<uint4 *>(Bs + (buf * BN + row) * P + ch * 8) = rb[v];
        }
    };

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
    const int lrow = lane & 31, lk = (lane >> 5) * 8;
    for (int kt = 0; kt < ktiles; ++kt) {
        const int buf = kt & 1;
        if (kt + 1 < ktiles) load(int64_t(kt + 1) * BK);
        const uint16_t *as = As + (buf * BM + wm * TM + lrow) * P + lk;
        const uint16_t *bs = Bs + (buf * BN + wn * TN + lrow) * P + lk;
#pragma unroll
        for (int kk = 0; kk < BK; kk += 16) {
            uint4 fa[FM], fb[FN];
#pragma unroll
            for (int i = 0; i < FM; ++i) fa[i] = *reinterpret_cast<const uint4 *>(as + i * 32 * P + kk);
#pragma unroll
            for (int j = 0; j < FN; ++j) fb[j] = *reinterpret_cast<const uint4 *>(bs + j * 32 * P + kk);
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j) acc[i][j] = Mfma<F16>::run(fa[i], fb[j], acc[i][j]);
        }
        if (kt + 1 < ktiles) store(buf ^ 1);
        __syncthreads();
    }

    // C layout of a 32x32 block: lane holds column lane % 32, rows 8 * (e / 4) + 4 * (lane / 32) + e % 4.
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                int64_t r = m0 + wm * TM + i * 32 + 8 * (e / 4) + 4 * (lane >> 5) + (e % 4);
                int64_t c = n0 + wn * TN + j * 32 + (lane & 31);
                if (r < s.m && c < s.n) epi(s, od, r, c, acc[i][j][e]);
            }
}

template <int BM, int BN, int BK>
constexpr int gemm_mfma_lds_bytes() {
    return 2 * (BM + BN) * Pitch<BK>::value * 2;
}

}  // namespace nhipk
