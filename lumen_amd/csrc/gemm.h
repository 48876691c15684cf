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

#include <type_traits>

#include "device_common.h"

namespace nhipk {

struct GemmShape {
    int64_t m, n, k;
    int32_t nbatch;
    int64_t batch[3];
    int64_t a_batch[3], b_batch[3], d_batch[3];
    int64_t a_m, a_k, b_k, b_n, d_m, d_n;
    int32_t tiles_m, tiles_n;
    int64_t d_split;  // split-k: element offset of split blockIdx.z's partial product in D (k is one split's)
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

// ---- MFMA, operands streamed HBM -> LDS (256 x 256 tiles) ------------------------------------------------
//
// gemm_stream: 2 x WN wavefronts, each a 128 x (256 / WN) block of D as 4 x FN MFMA 32x32x16 tiles (WN = 2:
// 4 waves of 128 x 128, one a SIMD, 0.5 KiB of LDS reads per MFMA; WN = 4: 8 waves of 128 x 64). Operand
// tiles go straight from HBM into LDS with global_load_lds_dwordx4 (no VGPR staging), STAGES deep, so loads of
// later k tiles run under the MFMAs of the current one. A wave's 16-byte LDS writes are contiguous (lane i
// at byte 16 i of a 1 KiB segment): lines are unpadded and the 16-byte chunks of each line are XOR-swizzled
// so that the fragment reads (16 rows at one chunk for a k-contiguous tile; 4 k-lines of 64 bytes for an
// mn-contiguous one read with ds_read_tr16_b64) fall on distinct banks. Fragments of k step kk + 16 are
// read while the MFMAs of step kk run (their issue order pinned with sched_group_barrier).
// The MFMA computes D^T blocks (B fragment as the A operand), so each lane ends with 4 consecutive columns
// of one row; the epilogue stages the tile through LDS and writes rows with 16-byte stores.
// Requires k % BK == 0 (a clamped k tail would add products of repeated columns).

template <int BK>
__device__ __forceinline__ int kmaj_swz(int r) {
    if constexpr (BK == 64) return ((r >> 1) & 7) ^ ((r & 1) << 2);
    else return (r >> 2) & 3;
}
__device__ __forceinline__ int mnmaj_swz(int k) { return (k & 3) << 2; }

typedef __attribute__((address_space(3))) void glds_void_t;

template <int BK, bool T, int TM = 256>
struct StreamTile {
    static constexpr int line_bytes = T ? TM * 2 : BK * 2;  // a k-line of TM mn, or a row of BK k
    static constexpr int chunks = line_bytes / 16;
    static constexpr int lines_per_seg = 1024 / line_bytes;
    static constexpr int bytes = TM * BK * 2;
    static constexpr int segs = bytes / 1024;
};

// The persistent kernel's LDS: two operand stages plus one wave's 32 staging rows (the other waves stage in the
// stage the tile's last k step has read).
constexpr int gemm_stream_persist_lds_bytes() { return 2 * 2 * 256 * 64 * 2 + 32 * (64 * 4 + 16); }

// Stages: 128 KiB of operand tiles for the 256 x 256 tile (one workgroup a CU); two stages (64 KiB, two
// workgroups a CU) for the 128 x 128 tile.
template <int BK, int TM = 256>
constexpr int gemm_stream_stages() { return TM == 256 ? (128 * 1024) / (2 * 256 * BK * 2) : 2; }
// Epilogue staging: a wave's 64 rows at a time, 16 bytes of padding a row.
template <int WN, int TM = 256>
constexpr int gemm_stream_stage_pitch() { return (TM / WN) * 4 + 16; }
// LDS: the operand stages, or the epilogue's staging (float32 rows), whichever is larger.
template <int BK, int WN, int TM = 256>
constexpr int gemm_stream_lds_bytes() {
    constexpr int ops = gemm_stream_stages<BK, TM>() * 2 * TM * BK * 2;
    constexpr int epi = 2 * WN * 64 * gemm_stream_stage_pitch<WN, TM>();
    return ops > epi ? ops : epi;
}

// Writes rows [rbase, rbase + ROWS) x columns [cbase, cbase + WCOLS) of D from a wave's float32 staging rows
// (`PITCH` bytes apart): 16-byte stores when D is row-contiguous and aligned, else element by element through
// the strided store.
template <int WCOLS, int PITCH, int ROWS = 64>
__device__ __forceinline__ void stream_store_rows(const GemmShape &s, const AnyStore &out, int64_t od, const char *stage,
                                                  int64_t rbase, int64_t cbase, int lane) {
    const int esize = out.dtype == 0 ? 4 : 2;
    const bool vec = s.d_n == 1 && s.n % 8 == 0 && s.d_m % 8 == 0 &&
                     ((reinterpret_cast<uintptr_t>(out.d) + od * esize) & 15) == 0;
    char *dbase = static_cast<char *>(out.d) + od * esize;
    if (vec) {
        const int epc = 16 / esize;            // output elements a 16-byte chunk
        const int cpr = WCOLS / epc;           // chunks a row
        for (int idx = lane; idx < ROWS * cpr; idx += 64) {
            const int r = idx / cpr, ch = idx % cpr;
            const int64_t gr = rbase + r, gc = cbase + ch * epc;
            if (gr >= s.m || gc >= s.n) continue;
            const float *src = reinterpret_cast<const float *>(stage + r * PITCH) + ch * epc;
            uint4 v;
            if (out.dtype == 0) {
                v = *reinterpret_cast<const uint4 *>(src);
            } else {
                const float4 x = *reinterpret_cast<const float4 *>(src);
                const float4 y = *reinterpret_cast<const float4 *>(src + 4);
                if (out.dtype == 1)
                    v = make_uint4(uint32_t(f32_to_bf16(x.x)) | (uint32_t(f32_to_bf16(x.y)) << 16),
                                   uint32_t(f32_to_bf16(x.z)) | (uint32_t(f32_to_bf16(x.w)) << 16),
                                   uint32_t(f32_to_bf16(y.x)) | (uint32_t(f32_to_bf16(y.y)) << 16),
                                   uint32_t(f32_to_bf16(y.z)) | (uint32_t(f32_to_bf16(y.w)) << 16));
                else
                    v = make_uint4(uint32_t(f32_to_f16(x.x)) | (uint32_t(f32_to_f16(x.y)) << 16),
                                   uint32_t(f32_to_f16(x.z)) | (uint32_t(f32_to_f16(x.w)) << 16),
                                   uint32_t(f32_to_f16(y.x)) | (uint32_t(f32_to_f16(y.y)) << 16),
                                   uint32_t(f32_to_f16(y.z)) | (uint32_t(f32_to_f16(y.w)) << 16));
            }
            *reinterpret_cast<uint4 *>(dbase + (gr * s.d_m + gc) * esize) = v;
        }
    } else {
        out.visit([&](auto stf) {
            for (int idx = lane; idx < ROWS * WCOLS; idx += 64) {
                const int r = idx / WCOLS, c = idx % WCOLS;
                const int64_t gr = rbase + r, gc = cbase + c;
                if (gr < s.m && gc < s.n) stf(s, od, gr, gc, *reinterpret_cast<const float *>(stage + r * PITCH + c * 4));
            }
        });
    }
}

// Writes the float32 sums of a wave's 64-row half `half` (MFMA tiles 2 half and 2 half + 1) to its LDS stage:
// acc[i][j][e] is row 32 i + l32, column 32 j + 8 (e / 4) + 4 h + e % 4 of the wave's block.
template <int FM, int FN, int PITCH>
__device__ __forceinline__ void stage_acc(const f32x16_t (&acc)[FM][FN], int half, char *stage, int l32, int h) {
#pragma unroll
    for (int ii = 0; ii < 2; ++ii) {
        const int i = 2 * half + ii;
        const int r = 32 * ii + l32;
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int e4 = 0; e4 < 4; ++e4)
                *reinterpret_cast<float4 *>(stage + r * PITCH + (32 * j + 8 * e4 + 4 * h) * 4) =
                    make_float4(acc[i][j][4 * e4], acc[i][j][4 * e4 + 1], acc[i][j][4 * e4 + 2], acc[i][j][4 * e4 + 3]);
    }
}

// Runs tile(kt, P) for kt = 0 .. ktiles - 1 with P = kt % S as a constant (std::integral_constant), S tiles at
// a time: a k loop whose LDS stage is a constant has the stage offsets in its LDS instructions' immediates
// instead of recomputing addresses every tile.
template <int S, int P = 0, class F>
__device__ __forceinline__ void tiles_block(int kt, int n, F &tile) {
    if constexpr (P < S) {
        if (P < n) {
            tile(kt + P, std::integral_constant<int, P>{});
            tiles_block<S, P + 1>(kt, n, tile);
        }
    }
}
template <int S, class F>
__device__ __forceinline__ void for_tiles(int ktiles, F &&tile) {
    int kt = 0;
    for (; kt + S <= ktiles; kt += S) tiles_block<S>(kt, S, tile);
    tiles_block<S>(kt, ktiles - kt, tile);
}

// One workgroup's 256 x 256 output tile. `out` is AnyStore (a plain store of D), or a generated epilogue
// functor called as out(row, col, float4, pre) with the float32 sums of four consecutive columns (col a
// multiple of 4, within m x n) and pre = out.load(row, col), its other operands read ahead. `smem` holds gemm_stream_lds_bytes<BK, WN>() bytes.
// KL, the k loop: 0 fragments of the next k step read under the current step's MFMAs; 1 (XPF) that read also
// across k tiles; 2 (ping-pong) the two waves of each SIMD alternate between a memory phase and an MFMA phase;
// 3 (k tile 64, two stages, four waves) the cross-tile read placed by hand with the loads split in halves.
template <bool F16, int BK, int WN, bool AT, bool BT, bool BUF, class Out, int TM = 256, int KL = 0>
__device__ __forceinline__ void gemm_stream_tile(const GemmShape &s, const uint16_t *__restrict__ a,
                                                 const uint16_t *__restrict__ b, const Out &out, char *smem) {
    constexpr int NW = 2 * WN;       // wavefronts (2 x WN)
    constexpr int WR = TM / 2;       // rows a wave
    constexpr int FM = WR / 32;      // 32-row MFMA tiles a wave
    constexpr int WCOLS = TM / WN;   // columns a wave
    constexpr int FN = WCOLS / 32;   // 32-column MFMA tiles a wave
    constexpr int STAGES = gemm_stream_stages<BK, TM>();
    using TA = StreamTile<BK, AT, TM>;
    using TB = StreamTile<BK, BT, TM>;
    constexpr int STAGE_BYTES = TA::bytes + TB::bytes;
    constexpr int LPS = (TA::segs + TB::segs) / NW;  // load instructions a wave issues per stage
    constexpr int NRD = (AT ? 2 * FM : FM) + (BT ? 2 * FN : FN);  // LDS read instructions a k step

    int tm, tn;
    tile_of(blockIdx.x, s.tiles_m, s.tiles_n, tm, tn);
    int64_t oa, ob, od;
    batch_offsets(s, blockIdx.y, oa, ob, od);
    const int64_t m0 = int64_t(tm) * TM, n0 = int64_t(tn) * TM;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave / WN, wn = wave % WN;
    const int h = lane >> 5, l32 = lane & 31, g = lane >> 4, s16 = lane & 15;
    // one wave a SIMD (WN = 2): the wave index as a scalar, so the loads' LDS destinations are scalar arithmetic
    const int wave_u = WN == 2 ? __builtin_amdgcn_readfirstlane(wave) : wave;
    const int64_t ks = int64_t(blockIdx.z) * s.k;  // split-k: this workgroup's first k
    od += int64_t(blockIdx.z) * s.d_split;
    const uint16_t *pa = a + oa + ks * s.a_k, *pb = b + ob + ks * s.b_k;
    const int ktiles = int(s.k / BK);

    // issues this wave's loads [lo, hi) of tile kt into stage st (A segments first, then B)
    // Buffer resources over this tile's rows of A and B (columns when mn-contiguous): the loads then take a
    // per-lane 32-bit offset fixed for the whole k loop plus a uniform k offset, with no per-load address
    // arithmetic, and rows past m / n read zeros. Operands whose tile span exceeds 2^31 bytes use 64-bit
    // global addresses instead.
    const int64_t mrem = s.m - m0 < TM ? s.m - m0 : TM, nrem = s.n - n0 < TM ? s.n - n0 : TM;
    const int64_t abytes = AT ? ((s.k - 1) * s.a_k + mrem) * 2 : ((mrem - 1) * s.a_m + s.k) * 2;
    const int64_t bbytes = BT ? ((s.k - 1) * s.b_k + nrem) * 2 : ((nrem - 1) * s.b_n + s.k) * 2;
    constexpr bool buf = BUF;  // the launcher checked stream_buffer_ok()
    const __amdgpu_buffer_rsrc_t rsa = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(AT ? pa + m0 : pa + m0 * s.a_m), (short)0, int(abytes), 0x00020000);
    const __amdgpu_buffer_rsrc_t rsb = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(BT ? pb + n0 : pb + n0 * s.b_n), (short)0, int(bbytes), 0x00020000);
    auto issue = [&](int st, int kt, int lo, int hi) {
        char *base = smem + st * STAGE_BYTES;
        const int64_t k0 = int64_t(kt) * BK;
#pragma unroll
        for (int i = 0; i < TA::segs / NW; ++i) {
            if (i < lo || i >= hi) continue;
            const int seg = wave_u + NW * i;
            const int line = seg * TA::lines_per_seg + lane / TA::chunks, c = lane % TA::chunks;
            if constexpr (buf) {
                const uint32_t vo = AT ? uint32_t((line * s.a_k + ((c ^ mnmaj_swz(line)) << 3)) * 2)
                                       : uint32_t((line * s.a_m + ((c ^ kmaj_swz<BK>(line)) << 3)) * 2);
                const uint32_t so = AT ? uint32_t(k0 * s.a_k * 2) : uint32_t(k0 * 2);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rsa, (glds_void_t *)(base + seg * 1024), 16, vo, so, 0, 0);
                continue;
            }
            const uint16_t *src;
            if (AT) {
                int64_t mm = m0 + ((c ^ mnmaj_swz(line)) << 3);
                mm = mm < s.m ? mm : s.m - 8;
                src = pa + (k0 + line) * s.a_k + mm;
            } else {
                int64_t mm = m0 + line;
                mm = mm < s.m ? mm : s.m - 1;
                src = pa + mm * s.a_m + k0 + ((c ^ kmaj_swz<BK>(line)) << 3);
            }
            __builtin_amdgcn_global_load_lds(src, (glds_void_t *)(base + seg * 1024), 16, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < TB::segs / NW; ++i) {
            if (TA::segs / NW + i < lo || TA::segs / NW + i >= hi) continue;
            const int seg = wave_u + NW * i;
            const int line = seg * TB::lines_per_seg + lane / TB::chunks, c = lane % TB::chunks;
            if constexpr (buf) {
                const uint32_t vo = BT ? uint32_t((line * s.b_k + ((c ^ mnmaj_swz(line)) << 3)) * 2)
                                       : uint32_t((line * s.b_n + ((c ^ kmaj_swz<BK>(line)) << 3)) * 2);
                const uint32_t so = BT ? uint32_t(k0 * s.b_k * 2) : uint32_t(k0 * 2);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rsb, (glds_void_t *)(base + TA::bytes + seg * 1024), 16, vo, so, 0, 0);
                continue;
            }
            const uint16_t *src;
            if (BT) {
                int64_t nn = n0 + ((c ^ mnmaj_swz(line)) << 3);
                nn = nn < s.n ? nn : s.n - 8;
                src = pb + (k0 + line) * s.b_k + nn;
            } else {
                int64_t nn = n0 + line;
                nn = nn < s.n ? nn : s.n - 1;
                src = pb + nn * s.b_n + k0 + ((c ^ kmaj_swz<BK>(line)) << 3);
            }
            __builtin_amdgcn_global_load_lds(src, (glds_void_t *)(base + TA::bytes + seg * 1024), 16, 0, 0);
        }
    };
    // fragment: 8 consecutive k (from kk + 8 h) at row `r0 + l32` of the tile
    auto frag = [&](const char *tile, int r0, int kk, auto tr) -> uint4 {
        if constexpr (decltype(tr)::value) {
            const int kl = kk + 8 * h + s16 / 4;
            const int mn = r0 + 16 * (g & 1) + 4 * (s16 & 3);
            const char *p0 = tile + kl * (TM * 2) + (((mn >> 3) ^ mnmaj_swz(kl)) << 4) + ((mn & 7) << 1);
            const char *p1 = tile + (kl + 4) * (TM * 2) + (((mn >> 3) ^ mnmaj_swz(kl + 4)) << 4) + ((mn & 7) << 1);
            gv4i16_t x = __builtin_amdgcn_ds_read_tr16_b64_v4i16((glds_v4i16_t *)(p0));
            gv4i16_t y = __builtin_amdgcn_ds_read_tr16_b64_v4i16((glds_v4i16_t *)(p1));
            uint2 xa = __builtin_bit_cast(uint2, x), ya = __builtin_bit_cast(uint2, y);
            return make_uint4(xa.x, xa.y, ya.x, ya.y);
        } else {
            const int r = r0 + l32;
            return *reinterpret_cast<const uint4 *>(tile + r * (BK * 2) + ((((kk >> 3) + h) ^ kmaj_swz<BK>(r)) << 4));
        }
    };

    f32x16_t acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

    constexpr bool XPF = KL == 1;
    if constexpr (KL == 3) {
        // k tile 64 (128-byte row segments: one L2 request a 128-byte line instead of two for k tile 32), two
        // stages, one or two waves a SIMD, placed by hand one MFMA at a time. Each tile's loads go out in two halves: A
        // of tile kt + 2 in tile kt's last k step, right after the barrier that frees its stage, B in tile
        // kt + 1's first k step. Each k step reads the next one's fragments after its first FM + FN MFMAs; the
        // last waits for all of tile kt + 1, meets the barrier after BARPOS MFMAs and reads tile kt + 1's first
        // fragments under its own MFMAs. Past the last tile the loads repeat it into the free stage, so every
        // tile runs the same straight-line body.
        static_assert(STAGES == 2 && BK == 64 && (WN == 2 || WN == 4), "two stages of k 64 on four or eight waves");
        constexpr int NSTEP = BK / 16, NM = FM * FN, NL = LPS / 2;
        constexpr int BARPOS = 2, L0 = 1, S0 = 2, L3 = WN == 2 ? 4 : 3, S3 = 1;
        static_assert(NL == TA::segs / NW, "the halves are A's and B's loads");
        static_assert(L0 + S0 * (NL - 1) < NM && L3 >= BARPOS && L3 + S3 * (NL - 1) < NM, "every load is issued");
        static_assert(BARPOS + FM + FN - 1 < NM, "every fragment read is issued");
        uint4 fa[2][FM], fb[2][FN];
        auto read1 = [&](const char *ta_, int buf, int kk, int q) {  // q-th fragment: A 0, B 0 .. FN - 1, A 1 ..
            const char *tb_ = ta_ + TA::bytes;
            if (q == 0) fa[buf][0] = frag(ta_, wm * WR, kk, std::integral_constant<bool, AT>{});
            else if (q <= FN) fb[buf][q - 1] = frag(tb_, wn * WCOLS + 32 * (q - 1), kk, std::integral_constant<bool, BT>{});
            else fa[buf][q - FN] = frag(ta_, wm * WR + 32 * (q - FN), kk, std::integral_constant<bool, AT>{});
        };
        issue(0, 0, 0, LPS);
        issue(1, min(1, ktiles - 1), 0, NL);
        __builtin_amdgcn_s_waitcnt((NL & 15) | ((NL >> 4) << 14) | 0x0070);  // tile 0 landed (this thread)
        __syncthreads();
#pragma unroll
        for (int q = 0; q < FM + FN; ++q) read1(smem, 0, 0, q);
        // one k tile in stage P (a constant: the loop below runs tiles in pairs, so the stages' LDS offsets
        // fold into the fragment reads' immediates)
        auto tile = [&](int kt, auto parc) {
            constexpr int P = decltype(parc)::value;
            const char *ta = smem + P * STAGE_BYTES;
            const char *tn = smem + (P ^ 1) * STAGE_BYTES;
            const int k1 = min(kt + 1, ktiles - 1), k2 = min(kt + 2, ktiles - 1);
#pragma unroll
            for (int st = 0; st < NSTEP; ++st) {
                const int cur = st & 1;
#pragma unroll
                for (int t = 0; t < NM; ++t) {
                    __builtin_amdgcn_sched_barrier(0);
                    if (st == NSTEP - 1 && t == BARPOS) {
                        __builtin_amdgcn_s_waitcnt(0x0070);      // tile kt + 1 landed (this thread), LDS reads done
                        asm volatile("s_barrier" ::: "memory");  // ... every thread's; stage kt is free
                        __builtin_amdgcn_sched_barrier(0);
                    }
                    acc[t / FN][t % FN] = Mfma<F16>::run(fb[cur][t % FN], fa[cur][t / FN], acc[t / FN][t % FN]);
                    if (st < NSTEP - 1) {
                        if (t < FM + FN) read1(ta, cur ^ 1, 16 * (st + 1), t);
                    } else if (t >= BARPOS && t - BARPOS < FM + FN) {
                        read1(tn, cur ^ 1, 0, t - BARPOS);
                    }
                    if (st == 0 && t >= L0 && (t - L0) % S0 == 0 && (t - L0) / S0 < NL)
                        issue(P ^ 1, k1, NL + (t - L0) / S0, NL + (t - L0) / S0 + 1);
                    if (st == NSTEP - 1 && t >= L3 && (t - L3) % S3 == 0 && (t - L3) / S3 < NL)
                        issue(P, k2, (t - L3) / S3, (t - L3) / S3 + 1);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        };
        for (int kt = 0; kt + 1 < ktiles; kt += 2) {
            tile(kt, std::integral_constant<int, 0>{});
            tile(kt + 1, std::integral_constant<int, 1>{});
        }
        if (ktiles & 1) tile(ktiles - 1, std::integral_constant<int, 0>{});
        __builtin_amdgcn_s_waitcnt(0x0070);  // the repeated loads land before LDS is reused
    } else if constexpr (KL == 2) {
        // Ping-pong: waves w and w + 4 share a SIMD (wm = 0 and 1). Each wave alternates a memory phase --
        // issue its loads of tile kt + STAGES - 1 into the stage tile kt - 1 left, read all of tile kt's MFMA
        // fragments into registers, wait for them and for its own loads of tile kt + 1 -- and an MFMA phase --
        // the tile's FM x FN x BK / 16 MFMAs at raised wave priority -- with one workgroup barrier between
        // phases. The wm = 1 waves run one phase behind, so in every phase one wave of each SIMD feeds its
        // MFMA pipe while the other loads. Stage reuse: tile kt - 1 was last read in the phase before tile kt's
        // first memory phase (every read completed before that phase's closing barrier); a tile is first read
        // after a barrier that every wave reached with its own loads of it landed.
        static_assert(STAGES >= 3 && NW == 8, "ping-pong needs 8 waves and loads two tiles ahead");
        constexpr int NSTEP = BK / 16;
        uint4 fa[NSTEP][FM], fb[NSTEP][FN];
        auto wait_tiles = [&](int later) {  // at most `later` tiles of this thread's loads in flight, LDS reads done
            if (later <= 0) __builtin_amdgcn_s_waitcnt(0x0070);
            else if (later == 1) __builtin_amdgcn_s_waitcnt((LPS & 15) | ((LPS >> 4) << 14) | 0x0070);
            else __builtin_amdgcn_s_waitcnt(((2 * LPS) & 15) | (((2 * LPS) >> 4) << 14) | 0x0070);
        };
#pragma unroll
        for (int st = 0; st < STAGES - 1; ++st)
            if (st < ktiles) issue(st, st, 0, LPS);
        wait_tiles(min(STAGES - 2, ktiles - 1));
        __builtin_amdgcn_s_barrier();
        if (wm == 1) __builtin_amdgcn_s_barrier();
        for_tiles<STAGES>(ktiles, [&](int kt, auto pc) {
            constexpr int P = decltype(pc)::value;  // kt % STAGES
            __builtin_amdgcn_sched_barrier(0);
            const char *ta = smem + P * STAGE_BYTES;
            const char *tb = ta + TA::bytes;
            if (kt + STAGES - 1 < ktiles) issue((P + STAGES - 1) % STAGES, kt + STAGES - 1, 0, LPS);
#pragma unroll
            for (int i = 0; i < NSTEP; ++i) {
#pragma unroll
                for (int ii = 0; ii < FM; ++ii) fa[i][ii] = frag(ta, wm * WR + 32 * ii, 16 * i, std::integral_constant<bool, AT>{});
#pragma unroll
                for (int j = 0; j < FN; ++j) fb[i][j] = frag(tb, wn * WCOLS + 32 * j, 16 * i, std::integral_constant<bool, BT>{});
            }
            wait_tiles(min(STAGES - 2, ktiles - 2 - kt));
            __builtin_amdgcn_sched_barrier(0);
            __builtin_amdgcn_s_barrier();
            __builtin_amdgcn_sched_barrier(0);
            __builtin_amdgcn_s_setprio(1);
#pragma unroll
            for (int i = 0; i < NSTEP; ++i)
#pragma unroll
                for (int ii = 0; ii < FM; ++ii)
#pragma unroll
                    for (int j = 0; j < FN; ++j) acc[ii][j] = Mfma<F16>::run(fb[i][j], fa[i][ii], acc[ii][j]);
            __builtin_amdgcn_s_setprio(0);
            __builtin_amdgcn_sched_barrier(0);
            __builtin_amdgcn_s_barrier();
        });
        if (wm == 0) __builtin_amdgcn_s_barrier();
    } else if constexpr (XPF) {
        // Fragments run ahead across k tiles: the last k step of tile kt waits for tile kt + 1's loads (issued
        // STAGES - 1 tiles earlier), meets the other waves at the barrier (which also frees tile kt's stage:
        // every wave's reads of it have completed) and reads tile kt + 1's first fragments under its own MFMAs,
        // so the MFMA stream has no gap at tile boundaries. Tile kt + STAGES - 1's loads are issued during the
        // first k step of tile kt, into the stage the previous barrier freed.
        static_assert(STAGES >= 3, "cross-tile fragment prefetch needs a tile of loads in flight");
        constexpr int NSTEP = BK / 16;
        // UNI (one wave a SIMD): every k tile issues its loads and waits the same way -- past the last tile the
        // loads repeat the last tile into the free stage -- so the loop body is one basic block and the loads
        // can be placed among the MFMAs
        constexpr bool UNI = WN == 2;
        uint4 fa[2][FM], fb[2][FN];
        auto read = [&](const char *ta, int buf, int kk) {
            const char *tb = ta + TA::bytes;
            fa[buf][0] = frag(ta, wm * WR, kk, std::integral_constant<bool, AT>{});
#pragma unroll
            for (int j = 0; j < FN; ++j) fb[buf][j] = frag(tb, wn * WCOLS + 32 * j, kk, std::integral_constant<bool, BT>{});
#pragma unroll
            for (int i = 1; i < FM; ++i) fa[buf][i] = frag(ta, wm * WR + 32 * i, kk, std::integral_constant<bool, AT>{});
        };
        // waits until at most `later` tiles' loads of this thread are in flight (vector memory completes in order)
        auto wait_tiles = [&](int later) {
            if (later <= 0) __builtin_amdgcn_s_waitcnt(0x0070);
            else if (later == 1) __builtin_amdgcn_s_waitcnt((LPS & 15) | ((LPS >> 4) << 14) | 0x0070);
            else if (later == 2) __builtin_amdgcn_s_waitcnt(((2 * LPS) & 15) | (((2 * LPS) >> 4) << 14) | 0x0070);
            else __builtin_amdgcn_s_waitcnt(((3 * LPS) & 15) | (((3 * LPS) >> 4) << 14) | 0x0070);
        };
#pragma unroll
        for (int st = 0; st < STAGES - 1; ++st)
            if (UNI || st < ktiles) issue(st, UNI ? min(st, ktiles - 1) : st, 0, LPS);
        wait_tiles(UNI ? STAGES - 2 : min(STAGES - 2, ktiles - 1));
        __syncthreads();
        read(smem, 0, 0);
        if constexpr (UNI && NSTEP == 2) {
            // Placed by hand, one MFMA at a time: each of the two k steps runs its FM x FN MFMAs with one fragment
            // read after each of the first FM + FN (step 0: this tile's second k step; step 1: the next tile's
            // first, once it has landed) and half of tile kt + STAGES - 1's loads spread LSTRIDE MFMAs apart.
            // Step 1 waits and meets the other waves after BARPOS MFMAs rather than before its first, so the
            // barrier's skew hides under MFMAs already issued.
            constexpr int NM = FM * FN, NL = LPS / 2;
            constexpr int BARPOS = 2, LSTART = 2;
            constexpr int LSTRIDE = NL > 1 ? (NM - 1 - LSTART) / (NL - 1) < 3 ? (NM - 1 - LSTART) / (NL - 1) : 3 : 1;
            static_assert(LPS % 2 == 0 && LSTART >= BARPOS && LSTRIDE >= 1 && LSTART + LSTRIDE * (NL - 1) < NM,
                          "every load is issued, none of step 1's before its wait");
            static_assert(BARPOS + FM + FN - 1 < NM, "every fragment read is issued");
            // at step 1's wait: tiles kt + 2 .. kt + STAGES - 2 and the first half of tile kt + STAGES - 1 may fly
            constexpr int LATER = (STAGES - 3) * LPS + NL;
            static_assert(LATER < 64, "vmcnt holds 6 bits");
            auto read1 = [&](const char *ta_, int buf, int kk, int q) {  // q-th fragment in read()'s order
                const char *tb_ = ta_ + TA::bytes;
                if (q == 0) fa[buf][0] = frag(ta_, wm * WR, kk, std::integral_constant<bool, AT>{});
                else if (q <= FN) fb[buf][q - 1] = frag(tb_, wn * WCOLS + 32 * (q - 1), kk, std::integral_constant<bool, BT>{});
                else fa[buf][q - FN] = frag(ta_, wm * WR + 32 * (q - FN), kk, std::integral_constant<bool, AT>{});
            };
            for_tiles<STAGES>(ktiles, [&](int kt, auto pc) {
                constexpr int P = decltype(pc)::value;  // kt % STAGES
                const char *ta = smem + P * STAGE_BYTES;
                const char *tn = smem + ((P + 1) % STAGES) * STAGE_BYTES;
                constexpr int lst = (P + STAGES - 1) % STAGES;
                const int lkt = min(kt + STAGES - 1, ktiles - 1);
#pragma unroll
                for (int t = 0; t < NM; ++t) {
                    __builtin_amdgcn_sched_barrier(0);
                    acc[t / FN][t % FN] = Mfma<F16>::run(fb[0][t % FN], fa[0][t / FN], acc[t / FN][t % FN]);
                    if (t < FM + FN) read1(ta, 1, 16, t);
                    if (t >= LSTART && (t - LSTART) % LSTRIDE == 0 && (t - LSTART) / LSTRIDE < NL)
                        issue(lst, lkt, (t - LSTART) / LSTRIDE, (t - LSTART) / LSTRIDE + 1);
                }
#pragma unroll
                for (int t = 0; t < NM; ++t) {
                    __builtin_amdgcn_sched_barrier(0);
                    if (t == BARPOS) {
                        // tile kt + 1 landed (this thread), LDS reads done; then every thread's (stage kt is free)
                        __builtin_amdgcn_s_waitcnt((LATER & 15) | ((LATER >> 4) << 14) | 0x0070);
                        asm volatile("s_barrier" ::: "memory");
                        __builtin_amdgcn_sched_barrier(0);
                    }
                    acc[t / FN][t % FN] = Mfma<F16>::run(fb[1][t % FN], fa[1][t / FN], acc[t / FN][t % FN]);
                    if (t >= BARPOS && t - BARPOS < FM + FN) read1(tn, 0, 0, t - BARPOS);
                    if (t >= LSTART && (t - LSTART) % LSTRIDE == 0 && (t - LSTART) / LSTRIDE < NL)
                        issue(lst, lkt, NL + (t - LSTART) / LSTRIDE, NL + (t - LSTART) / LSTRIDE + 1);
                }
                __builtin_amdgcn_sched_barrier(0);
            });
        } else {
        for_tiles<STAGES>(ktiles, [&](int kt, auto pc) {
            constexpr int P = decltype(pc)::value;  // kt % STAGES
            const char *ta = smem + P * STAGE_BYTES;
            const char *tn = smem + ((P + 1) % STAGES) * STAGE_BYTES;
            const bool more = kt + STAGES - 1 < ktiles;
            const bool next = kt + 1 < ktiles;
            auto step = [&](auto ic) {
                constexpr int i = decltype(ic)::value;
                constexpr int cur = i & 1;
                __builtin_amdgcn_sched_barrier(0);
                if constexpr (i + 1 < NSTEP) {
                    read(ta, cur ^ 1, 16 * (i + 1));
                } else {
                    if (UNI || next) {
                        wait_tiles(UNI ? STAGES - 2 : min(STAGES - 2, ktiles - 2 - kt));  // tile kt + 1 landed (this thread)
                        asm volatile("s_barrier" ::: "memory");  // ... every thread's; stage kt is free
                        read(tn, cur ^ 1, 0);
                    }
                }
                if constexpr (i == 0) {
                    if (UNI || more)
                        issue((P + STAGES - 1) % STAGES, UNI ? min(kt + STAGES - 1, ktiles - 1) : kt + STAGES - 1, 0, LPS);
                }
#pragma unroll
                for (int ii = 0; ii < FM; ++ii)
#pragma unroll
                    for (int j = 0; j < FN; ++j) acc[ii][j] = Mfma<F16>::run(fb[cur][j], fa[cur][ii], acc[ii][j]);
                if constexpr (WN == 2 && i == 0)  // one wave a SIMD: the loads go out among the MFMAs too
                    mfma_ds_vmem_interleave<0, FM * FN, NRD, LPS, i + 1>();
                else
                    mfma_ds_interleave<0, FM * FN, NRD, i + 1>();
                __builtin_amdgcn_sched_barrier(0);
            };
            step(std::integral_constant<int, 0>{});
            step(std::integral_constant<int, 1>{});
            if constexpr (NSTEP > 2) {
                step(std::integral_constant<int, 2>{});
                step(std::integral_constant<int, 3>{});
            }
        });
        }
        if constexpr (UNI) __builtin_amdgcn_s_waitcnt(0x0070);  // the repeated loads land before LDS is reused
    } else {
#pragma unroll
    for (int st = 0; st < STAGES - 1; ++st)
        if (st < ktiles) issue(st, st, 0, LPS);
    for_tiles<STAGES>(ktiles, [&](int kt, auto pc) {
        constexpr int P = decltype(pc)::value;  // kt % STAGES
        // wait for this thread's loads of tile kt: later tiles' loads may stay in flight
        const int later = min(STAGES - 2, ktiles - 1 - kt);
        if (STAGES <= 2 || later <= 0) __builtin_amdgcn_s_waitcnt(0x0070 | 0x0f00);
        else if (later == 1) __builtin_amdgcn_s_waitcnt((LPS & 15) | ((LPS >> 4) << 14) | 0x0070 | 0x0f00);
        else __builtin_amdgcn_s_waitcnt(((2 * LPS) & 15) | (((2 * LPS) >> 4) << 14) | 0x0070 | 0x0f00);
        __syncthreads();  // every thread's loads of tile kt landed; the stage of tile kt - 1 is free
        const bool more = kt + STAGES - 1 < ktiles;
        const char *ta = smem + P * STAGE_BYTES;
        const char *tb = ta + TA::bytes;
        uint4 fa[2][FM], fb[2][FN];
        auto read = [&](int buf, int kk) {  // in the order the MFMAs (i-major) first use them
            fa[buf][0] = frag(ta, wm * WR, kk, std::integral_constant<bool, AT>{});
#pragma unroll
            for (int j = 0; j < FN; ++j) fb[buf][j] = frag(tb, wn * WCOLS + 32 * j, kk, std::integral_constant<bool, BT>{});
#pragma unroll
            for (int i = 1; i < FM; ++i) fa[buf][i] = frag(ta, wm * WR + 32 * i, kk, std::integral_constant<bool, AT>{});
        };
        read(0, 0);
        auto step = [&](auto kkc) {
            constexpr int kk = decltype(kkc)::value;
            constexpr int cur = (kk / 16) & 1;
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (kk + 16 < BK) read(cur ^ 1, kk + 16);
            // the next stage's loads, a quarter (a half for BK 32) each k step: spread among the MFMAs
            // rather than issued in one burst after the barrier
            // (with one wave a SIMD, WN = 2, nothing else covers the loads' latency: all of them go out in the first
            // k step, a whole k tile ahead of their use)
            if constexpr (WN == 2 && TM == 256) {
                if (kk == 0 && more) issue((P + STAGES - 1) % STAGES, kt + STAGES - 1, 0, LPS);
            } else {
                if (more) issue((P + STAGES - 1) % STAGES, kt + STAGES - 1, (kk / 16) * LPS * 16 / BK, (kk / 16 + 1) * LPS * 16 / BK);
            }
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j) acc[i][j] = Mfma<F16>::run(fb[cur][j], fa[cur][i], acc[i][j]);
            if constexpr (kk + 16 < BK) mfma_ds_interleave<0, FM * FN, NRD, kk / 16 + 1>();
            __builtin_amdgcn_sched_barrier(0);
        };
        step(std::integral_constant<int, 0>{});
        step(std::integral_constant<int, 16>{});
        if constexpr (BK > 32) {
            step(std::integral_constant<int, 32>{});
            step(std::integral_constant<int, 48>{});
        }
    });
    }

    // acc[i][j][e]: row m0 + wm*WR + 32 i + l32, column n0 + wn*WCOLS + 32 j + 8 (e / 4) + 4 h + e % 4.
    // Staged through LDS as float32, 64 rows of the wave at a time, then written row-wise.
    const int64_t rbase = m0 + wm * WR, cbase = n0 + wn * WCOLS;
    constexpr int PITCH = gemm_stream_stage_pitch<WN, TM>();
    __syncthreads();  // operand stages are dead: reuse LDS for the output
    char *stage = smem + wave * (64 * PITCH);
    // a generated epilogue reads its other operands with Out::load(row, col) into Out::Pre, kPrefetch chunks of
    // four columns at a time: the first group's loads are issued before the sums are staged, so their latency
    // overlaps the staging and the barrier instead of stalling every chunk
    constexpr int CPR = WCOLS / 4;  // four-column chunks a wave row; a lane takes CPR of the 64 x CPR chunks a half
    // a column-summing epilogue (Out::kColSum): a lane's chunks all hold columns cbase + 4 (lane % CPR) .. + 3,
    // so it sums its rows' values of them here; the lanes of a column combine at the end and the wave adds
    // its 4 x CPR column sums atomically (Out::colsum_add)
    float4 colsum = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    (void)colsum;
#pragma unroll
    for (int half = 0; half < FM / 2; ++half) {
        if constexpr (std::is_same<Out, AnyStore>::value) {
            stage_acc<FM, FN, PITCH>(acc, half, stage, l32, h);
            __syncthreads();
            stream_store_rows<WCOLS, PITCH>(s, out, od, stage, rbase + 64 * half, cbase, lane);
        } else {
            constexpr int G = Out::kPrefetch < CPR ? Out::kPrefetch : CPR;
            static_assert(CPR % G == 0, "prefetch groups must divide a lane's chunks");
            static_assert(64 % CPR == 0, "a lane keeps the same four columns over its chunks");
            typename Out::Pre pre[G];
            auto fetch = [&](int g0) {
#pragma unroll
                for (int q = 0; q < G; ++q) {
                    const int idx = lane + 64 * (g0 + q);
                    const int64_t gr = rbase + 64 * half + idx / CPR, gc = cbase + 4 * (idx % CPR);
                    if (gr < s.m && gc < s.n) pre[q] = out.load(gr, gc);
                }
            };
            fetch(0);
            stage_acc<FM, FN, PITCH>(acc, half, stage, l32, h);
            __syncthreads();
#pragma unroll
            for (int g0 = 0; g0 < CPR; g0 += G) {
                if (g0) fetch(g0);
#pragma unroll
                for (int q = 0; q < G; ++q) {
                    const int idx = lane + 64 * (g0 + q);
                    const int r = idx / CPR, ch = idx % CPR;
                    const int64_t gr = rbase + 64 * half + r, gc = cbase + 4 * ch;
                    if (gr < s.m && gc < s.n) {
                        if constexpr (Out::kColSum) {
                            const float4 c4 = out(gr, gc, *reinterpret_cast<const float4 *>(stage + r * PITCH + ch * 16), pre[q]);
                            colsum.x += c4.x;
                            colsum.y += c4.y;
                            colsum.z += c4.z;
                            colsum.w += c4.w;
                        } else {
                            out(gr, gc, *reinterpret_cast<const float4 *>(stage + r * PITCH + ch * 16), pre[q]);
                        }
                    }
                }
            }
        }
        __syncthreads();
    }
    if constexpr (!std::is_same<Out, AnyStore>::value) {
        if constexpr (Out::kColSum) {
#pragma unroll
            for (int o = CPR; o < 64; o <<= 1) {
                colsum.x += __shfl_xor(colsum.x, o, 64);
                colsum.y += __shfl_xor(colsum.y, o, 64);
                colsum.z += __shfl_xor(colsum.z, o, 64);
                colsum.w += __shfl_xor(colsum.w, o, 64);
            }
            const int64_t gc = cbase + 4 * lane;
            if (lane < CPR && gc < s.n && rbase < s.m) out.colsum_add(gc, colsum);
        }
    }
}

// The persistent 256 x 256 streamed GEMM: a workgroup a CU walks tiles blockIdx.x, + gridDim.x, ... and
// overlaps each tile's end with the next one's start. During a tile's last k step the stage the step does
// not read fills with the next tile's first k tile, and the sums go out through the stage the step did read
// (row-contiguous stores), so the next tile's first loads are in flight across the last MFMAs and the stores,
// and no workgroup launches between tiles. Same operand staging, k loop and results as gemm_stream_tile (one batch, one split: z and split-k
// go through gemm_stream).
template <bool F16, int BK, int WN, bool AT, bool BT, bool BUF>
__device__ __forceinline__ void gemm_stream_persist_run(const GemmShape &s, const uint16_t *__restrict__ a,
                                                        const uint16_t *__restrict__ b, const AnyStore &out,
                                                        char *smem) {
    constexpr int TM = 256;
    constexpr int NW = 2 * WN;
    constexpr int WR = TM / 2;
    constexpr int FM = WR / 32;
    constexpr int WCOLS = TM / WN;
    constexpr int FN = WCOLS / 32;
    constexpr int STAGES = gemm_stream_stages<BK, TM>();
    static_assert(STAGES == 2, "the persistent kernel alternates two stages");
    using TA = StreamTile<BK, AT, TM>;
    using TB = StreamTile<BK, BT, TM>;
    constexpr int STAGE_BYTES = TA::bytes + TB::bytes;
    constexpr int LPS = (TA::segs + TB::segs) / NW;
    constexpr int NRD = (AT ? 2 * FM : FM) + (BT ? 2 * FN : FN);

    const int ntiles = s.tiles_m * s.tiles_n;
    int t = blockIdx.x;
    if (t >= ntiles) return;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave / WN, wn = wave % WN;
    const int h = lane >> 5, l32 = lane & 31, g = lane >> 4, s16 = lane & 15;
    const int64_t od = 0;
    const uint16_t *pa = a, *pb = b;
    const int ktiles = int(s.k / BK);

    struct Ctx {
        int64_t m0, n0;
        __amdgpu_buffer_rsrc_t rsa, rsb;
    };
    auto ctx_of = [&](int tile) {
        int tm, tn;
        tile_of(tile, s.tiles_m, s.tiles_n, tm, tn);
        Ctx c;
        c.m0 = int64_t(tm) * TM;
        c.n0 = int64_t(tn) * TM;
        const int64_t mrem = s.m - c.m0 < TM ? s.m - c.m0 : TM, nrem = s.n - c.n0 < TM ? s.n - c.n0 : TM;
        const int64_t abytes = AT ? ((s.k - 1) * s.a_k + mrem) * 2 : ((mrem - 1) * s.a_m + s.k) * 2;
        const int64_t bbytes = BT ? ((s.k - 1) * s.b_k + nrem) * 2 : ((nrem - 1) * s.b_n + s.k) * 2;
        c.rsa = __builtin_amdgcn_make_buffer_rsrc((void *)(AT ? pa + c.m0 : pa + c.m0 * s.a_m), (short)0,
                                                  int(abytes), 0x00020000);
        c.rsb = __builtin_amdgcn_make_buffer_rsrc((void *)(BT ? pb + c.n0 : pb + c.n0 * s.b_n), (short)0,
                                                  int(bbytes), 0x00020000);
        return c;
    };
    auto issue = [&](const Ctx &c, int st, int kt, int lo, int hi) {
        char *base = smem + st * STAGE_BYTES;
        const int64_t k0 = int64_t(kt) * BK;
#pragma unroll
        for (int i = 0; i < TA::segs / NW; ++i) {
            if (i < lo || i >= hi) continue;
            const int seg = wave + NW * i;
            const int line = seg * TA::lines_per_seg + lane / TA::chunks, ch = lane % TA::chunks;
            if constexpr (BUF) {
                const uint32_t vo = AT ? uint32_t((line * s.a_k + ((ch ^ mnmaj_swz(line)) << 3)) * 2)
                                       : uint32_t((line * s.a_m + ((ch ^ kmaj_swz<BK>(line)) << 3)) * 2);
                const uint32_t so = AT ? uint32_t(k0 * s.a_k * 2) : uint32_t(k0 * 2);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(c.rsa, (glds_void_t *)(base + seg * 1024), 16, vo, so, 0, 0);
                continue;
            }
            const uint16_t *src;
            if (AT) {
                int64_t mm = c.m0 + ((ch ^ mnmaj_swz(line)) << 3);
                mm = mm < s.m ? mm : s.m - 8;
                src = pa + (k0 + line) * s.a_k + mm;
            } else {
                int64_t mm = c.m0 + line;
                mm = mm < s.m ? mm : s.m - 1;
                src = pa + mm * s.a_m + k0 + ((ch ^ kmaj_swz<BK>(line)) << 3);
            }
            __builtin_amdgcn_global_load_lds(src, (glds_void_t *)(base + seg * 1024), 16, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < TB::segs / NW; ++i) {
            if (TA::segs / NW + i < lo || TA::segs / NW + i >= hi) continue;
            const int seg = wave + NW * i;
            const int line = seg * TB::lines_per_seg + lane / TB::chunks, ch = lane % TB::chunks;
            if constexpr (BUF) {
                const uint32_t vo = BT ? uint32_t((line * s.b_k + ((ch ^ mnmaj_swz(line)) << 3)) * 2)
                                       : uint32_t((line * s.b_n + ((ch ^ kmaj_swz<BK>(line)) << 3)) * 2);
                const uint32_t so = BT ? uint32_t(k0 * s.b_k * 2) : uint32_t(k0 * 2);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(c.rsb, (glds_void_t *)(base + TA::bytes + seg * 1024), 16, vo, so, 0, 0);
                continue;
            }
            const uint16_t *src;
            if (BT) {
                int64_t nn = c.n0 + ((ch ^ mnmaj_swz(line)) << 3);
                nn = nn < s.n ? nn : s.n - 8;
                src = pb + (k0 + line) * s.b_k + nn;
            } else {
                int64_t nn = c.n0 + line;
                nn = nn < s.n ? nn : s.n - 1;
                src = pb + nn * s.b_n + k0 + ((ch ^ kmaj_swz<BK>(line)) << 3);
            }
            __builtin_amdgcn_global_load_lds(src, (glds_void_t *)(base + TA::bytes + seg * 1024), 16, 0, 0);
        }
    };
    auto frag = [&](const char *tile, int r0, int kk, auto tr) -> uint4 {
        if constexpr (decltype(tr)::value) {
            const int kl = kk + 8 * h + s16 / 4;
            const int mn = r0 + 16 * (g & 1) + 4 * (s16 & 3);
            const char *p0 = tile + kl * (TM * 2) + (((mn >> 3) ^ mnmaj_swz(kl)) << 4) + ((mn & 7) << 1);
            const char *p1 = tile + (kl + 4) * (TM * 2) + (((mn >> 3) ^ mnmaj_swz(kl + 4)) << 4) + ((mn & 7) << 1);
            gv4i16_t x = __builtin_amdgcn_ds_read_tr16_b64_v4i16((glds_v4i16_t *)(p0));
            gv4i16_t y = __builtin_amdgcn_ds_read_tr16_b64_v4i16((glds_v4i16_t *)(p1));
            uint2 xa = __builtin_bit_cast(uint2, x), ya = __builtin_bit_cast(uint2, y);
            return make_uint4(xa.x, xa.y, ya.x, ya.y);
        } else {
            const int r = r0 + l32;
            return *reinterpret_cast<const uint4 *>(tile + r * (BK * 2) + ((((kk >> 3) + h) ^ kmaj_swz<BK>(r)) << 4));
        }
    };

    Ctx cur = ctx_of(t);
    int stage = 0;  // stage holding the current k tile
    issue(cur, 0, 0, 0, LPS);
    for (;;) {
        const int tnext = t + int(gridDim.x);
        const bool has_next = tnext < ntiles;
        const Ctx nxt = ctx_of(has_next ? tnext : t);
        f32x16_t acc[FM][FN];
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j)
#pragma unroll
                for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;
        for (int kt = 0; kt < ktiles; ++kt) {
            // every load of this thread has landed (the previous tile's stores count too: vmcnt holds both)
            __builtin_amdgcn_s_waitcnt(0x0070 | 0x0f00);
            __syncthreads();  // all threads' loads of this k tile landed; the other stage is free
            const bool more = kt + 1 < ktiles;
            const bool prefetch = !more && has_next;
            const char *ta = smem + stage * STAGE_BYTES;
            const char *tb = ta + TA::bytes;
            uint4 fa[2][FM], fb[2][FN];
            auto read = [&](int bsel, int kk) {
                fa[bsel][0] = frag(ta, wm * WR, kk, std::integral_constant<bool, AT>{});
#pragma unroll
                for (int j = 0; j < FN; ++j) fb[bsel][j] = frag(tb, wn * WCOLS + 32 * j, kk, std::integral_constant<bool, BT>{});
#pragma unroll
                for (int i = 1; i < FM; ++i) fa[bsel][i] = frag(ta, wm * WR + 32 * i, kk, std::integral_constant<bool, AT>{});
            };
            read(0, 0);
            auto step = [&](auto kkc) {
                constexpr int kk = decltype(kkc)::value;
                constexpr int cb = (kk / 16) & 1;
                __builtin_amdgcn_sched_barrier(0);
                if constexpr (kk + 16 < BK) read(cb ^ 1, kk + 16);
                constexpr int lo = (kk / 16) * LPS * 16 / BK, hi = (kk / 16 + 1) * LPS * 16 / BK;
                if (more) issue(cur, stage ^ 1, kt + 1, lo, hi);
                else if (prefetch) issue(nxt, stage ^ 1, 0, lo, hi);
#pragma unroll
                for (int i = 0; i < FM; ++i)
#pragma unroll
                    for (int j = 0; j < FN; ++j) acc[i][j] = Mfma<F16>::run(fb[cb][j], fa[cb][i], acc[i][j]);
                if constexpr (kk + 16 < BK) mfma_ds_interleave<0, FM * FN, NRD, kk / 16 + 1>();
                __builtin_amdgcn_sched_barrier(0);
            };
            step(std::integral_constant<int, 0>{});
            step(std::integral_constant<int, 16>{});
            if constexpr (BK > 32) {
                step(std::integral_constant<int, 32>{});
                step(std::integral_constant<int, 48>{});
            }
            stage ^= 1;
        }
        // the sums go out through LDS, 32 rows of the wave at a time, as row-contiguous 16-byte stores (stores
        // straight from the accumulators, 32 rows x 32 bytes an instruction, take several times longer): the
        // stage the last k step read is free once every wave is past its reads (the other stage holds the next
        // tile's first k tile); seven waves stage there, the eighth in the LDS past the two stages
        __syncthreads();
        {
            constexpr int PITCH = WCOLS * 4 + 16;
            char *rows = wave < 7 ? smem + (stage ^ 1) * STAGE_BYTES + wave * (32 * PITCH) : smem + 2 * STAGE_BYTES;
#pragma unroll
            for (int i = 0; i < FM; ++i) {
#pragma unroll
                for (int j = 0; j < FN; ++j)
#pragma unroll
                    for (int e4 = 0; e4 < 4; ++e4)
                        *reinterpret_cast<float4 *>(rows + l32 * PITCH + (32 * j + 8 * e4 + 4 * h) * 4) =
                            make_float4(acc[i][j][4 * e4], acc[i][j][4 * e4 + 1], acc[i][j][4 * e4 + 2], acc[i][j][4 * e4 + 3]);
                // the wave's own rows: its writes land before its lanes read them back
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                stream_store_rows<WCOLS, PITCH, 32>(s, out, od, rows, cur.m0 + wm * WR + 32 * i, cur.n0 + wn * WCOLS, lane);
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            }
        }
        if (!has_next) break;
        t = tnext;
        cur = nxt;
    }
}

template <bool F16, int BK, int WN, bool AT, bool BT, bool BUF>
__global__ __launch_bounds__(128 * WN) __attribute__((amdgpu_waves_per_eu(WN / 2, WN / 2))) void gemm_stream_persist(
    GemmShape s, const uint16_t *__restrict__ a, const uint16_t *__restrict__ b, AnyStore out) {
    extern __shared__ __align__(1024) char smem[];
    gemm_stream_persist_run<F16, BK, WN, AT, BT, BUF>(s, a, b, out, smem);
}

template <bool F16, int BK, int WN, bool AT, bool BT, bool BUF, int KL = 0>
__global__ __launch_bounds__(128 * WN) __attribute__((amdgpu_waves_per_eu(WN / 2, WN / 2))) void gemm_stream(
    GemmShape s, const uint16_t *__restrict__ a, const uint16_t *__restrict__ b, AnyStore out) {
    extern __shared__ __align__(1024) char smem[];
    gemm_stream_tile<F16, BK, WN, AT, BT, BUF, AnyStore, 256, KL>(s, a, b, out, smem);
}

// The 128 x 128 tile: 4 wavefronts of 64 x 64, two 32 KiB stages, two workgroups a CU (dots with too few
// 256 x 256 tiles to fill the chip).
template <bool F16, bool AT, bool BT, bool BUF>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void gemm_stream128(
    GemmShape s, const uint16_t *__restrict__ a, const uint16_t *__restrict__ b, AnyStore out) {
    extern __shared__ __align__(1024) char smem[];
    gemm_stream_tile<F16, 64, 2, AT, BT, BUF, AnyStore, 128>(s, a, b, out, smem);
}

// Whether every operand byte a 256 x 256 tile of `s` reads lies within 2^31 bytes of the tile's first
// element (the buffer-load path's 32-bit offsets); the launch picks the 64-bit global-address path otherwise.
__host__ __device__ inline bool stream_buffer_ok(int64_t m, int64_t n, int64_t k, bool at, bool bt, int64_t a_m,
                                                 int64_t a_k, int64_t b_k, int64_t b_n) {
    const int64_t lim = int64_t(1) << 31;
    const int64_t abytes = at ? ((k - 1) * a_k + 256) * 2 : (255 * a_m + k) * 2;
    const int64_t bbytes = bt ? ((k - 1) * b_k + 256) * 2 : (255 * b_n + k) * 2;
    (void)m, (void)n;
    return abytes < lim && bbytes < lim;
}

// Split-k reduction: D[z, r, c] = sum over splits of the float32 partials P[split][z][r][c] (contiguous,
// `mn` = m * n elements a batch), in split order, rounded once to D's dtype.
__global__ __launch_bounds__(256) void gemm_splitk_reduce(GemmShape s, const float *__restrict__ part, int splits,
                                                           int64_t total, AnyStore out) {
    const int64_t mn = s.m * s.n;
    out.visit([&](auto stf) {
        for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < total; i += int64_t(gridDim.x) * 256) {
            float acc = part[i];
            for (int sp = 1; sp < splits; ++sp) acc += part[int64_t(sp) * total + i];
            const int64_t z = i / mn, rc = i % mn;
            int64_t oa, ob, od;
            batch_offsets(s, z, oa, ob, od);
            stf(s, od, rc / s.n, rc % s.n, acc);
        }
    });
}

}  // namespace nhipk
