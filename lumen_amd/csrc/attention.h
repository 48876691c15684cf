// Flash attention for gfx950: forward, and the FlashAttention-2 backward as three kernels (prep: delta and
// base-2 LSE; dK/dV per key block; dQ per query block), following the algorithm of
// lumen/codegen/attention/triton/kernel.py:34-256.
//
// Layout choices (all MFMA v_mfma_f32_32x32x16_{bf16,f16}, float32 accumulation):
//  * The forward computes S^T = K Q^T, so the 32x32 C layout puts one query in each lane (lane % 32) and its
//    keys in the accumulator registers: the running max and sum of a query row never leave its lane but for
//    one exchange between the two half-waves. P^T then is, register for register, the B operand of
//    O^T = V^T P^T once the k order of the MFMA is permuted to match: lane half h holds keys
//    {4h..4h+3, 8+4h..8+4h+3} of each 16-key step, and V^T is read with that same key order from LDS by two
//    ds_read_tr16_b64 (4 consecutive keys at one head-dim column each). O^T accumulates in registers, one
//    query a lane, so the per-query rescale of the online softmax is a multiply by a lane scalar.
//  * P is rounded to the inputs' dtype before P V, as the reference does (kernel.py:99).
#pragma once

#include <type_traits>

#include "device_common.h"
#include "nhip_internal.h"

namespace nhipk {

typedef short v4i16_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4i16_t lds_v4i16_t;

template <bool F16>
__device__ __forceinline__ uint16_t to_half_bits(float f) {
    return F16 ? f32_to_f16(f) : f32_to_bf16(f);
}

// Two floats rounded (nearest even) to the 16-bit dtype and packed, the first in the low half. bf16 uses the
// gfx950 conversion v_cvt_pk_bf16_f32.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
template <bool F16>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
    if constexpr (F16) {
        f16x2_t v = {_Float16(a), _Float16(b)};
        return __builtin_bit_cast(uint32_t, v);
    } else {
        bf16x2_t v = {__bf16(a), __bf16(b)};
        return __builtin_bit_cast(uint32_t, v);
    }
}

template <bool F16>
__device__ __forceinline__ f32x16_t mfma32(uint4 a, uint4 b, f32x16_t c) {
    if constexpr (F16)
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), c,
                                                       0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                        c, 0, 0, 0);
}

// Two transposed 64-bit LDS reads: 4 consecutive rows at one column each, concatenated (8 x 16-bit).
__device__ __forceinline__ uint4 read_tr_pair(const uint16_t *p0, const uint16_t *p1) {
    v4i16_t a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_t *)(p0));
    v4i16_t b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_t *)(p1));
    uint2 x = __builtin_bit_cast(uint2, a), y = __builtin_bit_cast(uint2, b);
    return make_uint4(x.x, x.y, y.x, y.y);
}

struct AttnParams {
    const uint16_t *q, *k, *v, *o_in, *d_o;
    uint16_t *o, *dq, *dk, *dv;
    float *lse;
    const float *lse_in;
    float *delta;
    float *dqacc;  // float32 [B, N, Sq, D] dQ accumulated atomically by the dK/dV kernel (null: deterministic)
    uint16_t *ds;  // dS tiles [B, N, Sk / 128, Sq / 64][128 keys][64 queries] the dK/dV kernel stores (or null)
    int64_t sq, sk, heads, kv_heads, batch;
    int64_t hd, hdv;  // Q/K's and V/O/dO's head dims; the kernels run at D >= both (kernel_head_dim), columns past
                      // them read as zeros
    int64_t q_b, q_s, q_n, k_b, k_s, k_n, v_b, v_s, v_n, o_b, o_s, o_n;
    int64_t do_b, do_s, do_n, dq_b, dq_s, dq_n, dk_b, dk_s, dk_n, dv_b, dv_s, dv_n;
    float scale;
};

// ---- forward ------------------------------------------------------------------------------------
//
// Same algorithm and lane layout as above, arranged for the CDNA4 pipeline:
//  * K and V tiles go from HBM straight into LDS (global_load_lds_dwordx4: no VGPR staging), double
//    buffered: tile t+1 is in flight while tile t is computed; two workgroups share a CU (<= 256 registers
//    a lane, 64 KiB LDS), so one's softmax VALU work overlaps the other's MFMAs.
//  * A wave's 16-byte LDS writes are contiguous (lane i writes bytes 16i..16i+15 of a 1 KiB segment), so
//    rows are unpadded and bank conflicts are avoided by an XOR swizzle of the 16-byte chunks of each row
//    (chunk c of row r holds the row's chunk c ^ swz(r)); swz keeps both the row-wise K reads (16 rows,
//    one chunk) and the transposed V reads (4 rows, 4 chunks) on distinct banks.
//  * Softmax in base 2: p = 2^(s * scale * log2 e - m), with m a running maximum that is only raised
//    when a row's maximum grows by more than 2^8 (so the O rescale runs rarely; P stays below 2^8 and
//    its bf16 rounding has the same relative error). LSE = (m + log2 l) ln 2.
//  * Masking code runs only on tiles that cross the causal diagonal or the end of the keys.
//  * Causal workgroups start with the longest rows (query blocks in reverse order).

// 2^x by the hardware v_exp_f32 (no denormal-range fixup: results below 2^-126 may flush to zero, which
// rounds away in P's 16-bit dtype anyway).
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Workgroup order: `units` independent units (a batch-head pair) of `per` workgroups each. Workgroups are
// dispatched round-robin over the 8 XCDs by linear id, so when units divide evenly each XCD gets whole
// units, in order, and the workgroups running together on an XCD share their unit's K/V (or Q/dO) in its
// L2. Returns the unit and the workgroup's index in it.
__device__ __forceinline__ void xcd_order(int64_t units, int64_t per, int64_t &unit, int64_t &idx) {
    const int64_t lin = blockIdx.x;
    if (units % 8 == 0) {
        const int64_t x = lin % 8, j = lin / 8;
        unit = (j / per) * 8 + x;
        idx = j % per;
    } else {
        unit = lin / per;
        idx = lin % per;
    }
}

template <int D>
__device__ __forceinline__ int kv_swz(int r) {
    if constexpr (D >= 128) return ((r & 3) << 2) | ((r >> 2) & 3);
    else return ((((r >> 1) & 1) << 2) | ((r >> 2) & 3));
}

// Byte offset of element `col` (a multiple of 4) of row `r` in a swizzled tile of D-element rows.
template <int D>
__device__ __forceinline__ int kv_off(int r, int col) {
    return r * (D * 2) + ((((col >> 3) ^ kv_swz<D>(r))) << 4) + ((col & 7) << 1);
}

typedef __attribute__((address_space(3))) void lds_void_t;

// Zeros `elems` 16-bit elements of LDS (a multiple of 8) when the kernel's tiles can be partial (rows past the
// operand's end, or a head dim padded to D), so that the chunks load_tile_async leaves unloaded hold zeros rather
// than what an earlier kernel left there; every thread takes part, and a barrier follows.
__device__ __forceinline__ void zero_tiles(uint16_t *p, int elems, bool partial) {
    if (!partial) return;
    for (int i = int(threadIdx.x) * 8; i < elems; i += int(blockDim.x) * 8)
        *reinterpret_cast<uint4 *>(p + i) = make_uint4(0, 0, 0, 0);
    __syncthreads();
}

// Issues the loads of rows [k0, k0 + 64) of a [*, D] operand (row stride `rs` elements, `rows` rows) into
// the swizzled tile `dst`. When the operand spans less than 2^31 bytes the loads are buffer loads (the row
// offset a uniform operand, the lane's offset fixed); otherwise 64-bit global loads with rows past `rows`
// clamped to the last row. On the buffer path the lanes of rows past `rows` and of columns from `cols` on (a
// head dim padded to D; the launcher checks that padded operands take this path) issue no load: their LDS
// chunks keep what they held, which zero_tiles set to zeros when the kernel started (or an earlier tile's
// finite values). Rows past `rows` have their scores masked; padded columns meet zeros in the other operand.
template <int D, int NW = 4>
__device__ __forceinline__ void load_tile_async(const uint16_t *src, int64_t rs, int64_t k0, int64_t rows,
                                                uint16_t *dst, int wave, int lane, int64_t cols = D) {
    constexpr int RPS = 1024 / (D * 2);  // rows a wave instruction covers
    constexpr int SEGS = 64 / RPS;       // 1 KiB segments in the tile
    const int64_t bytes = ((rows - 1) * rs + D) * 2;
    if (bytes < (int64_t(1) << 31) && (k0 + 64) * rs * 2 < (int64_t(1) << 31)) {
        const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc((void *)src, (short)0, int(bytes), 0x00020000);
        const uint32_t so = uint32_t(k0 * rs * 2);
        // the wave index as a scalar: the segment, its LDS destination and the trip count are then uniform
        const int wu = __builtin_amdgcn_readfirstlane(wave);
        constexpr int PER = (SEGS + NW - 1) / NW;
        auto seg_load = [&](int i, bool masked) {
            const int seg = wu + NW * i;
            if (SEGS % NW != 0 && seg >= SEGS) return;
            const int r = seg * RPS + lane / (D / 8);
            const int c = lane % (D / 8);
            const int sc = c ^ kv_swz<D>(r);
            const uint32_t vo = uint32_t((r * rs + (sc << 3)) * 2);
            if (!masked || (8 * sc < cols && k0 + r < rows))
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_void_t *)(dst + seg * 512), 16, vo, so, 0, 0);
        };
        if (k0 + 64 <= rows && cols >= D) {  // a whole tile: no lane is masked
#pragma unroll
            for (int i = 0; i < PER; ++i) seg_load(i, false);
        } else {
#pragma unroll
            for (int i = 0; i < PER; ++i) seg_load(i, true);
        }
        return;
    }
#pragma unroll
    for (int seg = wave; seg < SEGS; seg += NW) {
        const int r = seg * RPS + lane / (D / 8);
        const int c = lane % (D / 8);
        int64_t row = k0 + r;
        row = row < rows ? row : rows - 1;
        const uint16_t *g = src + row * rs + ((c ^ kv_swz<D>(r)) << 3);
        __builtin_amdgcn_global_load_lds(g, (lds_void_t *)(dst + seg * 512), 16, 0, 0);
    }
}

// Workgroup sizes of the forward kernel (the attention tile configs): NW waves of 32 queries each share every
// K/V tile a workgroup streams through LDS. More waves read K and V fewer times per query; fewer fill the CUs
// when there are few query blocks. Two workgroups a CU hold the 64 KiB (D = 128) double-buffered tiles, so
// each wave keeps 256 VGPRs at 4 waves a workgroup and 8 (one workgroup a CU at 8).
template <int NW, int D = 128> struct FwdOccupancy {
    static constexpr int kBlocks = D > 128 ? 1 : (NW >= 8 ? 1 : (NW >= 4 ? 2 : 4));
};

template <int D, bool F16, bool CAUSAL, int NW = 4>
__global__ __launch_bounds__(64 * NW, (FwdOccupancy<NW, D>::kBlocks)) void flash_fwd_kernel(AttnParams p) {
    constexpr int QB = 32 * NW;  // queries a workgroup
    constexpr int BN = 64;
    constexpr int DS = D / 16, DT = D / 32;
    constexpr int TILE = BN * D;  // elements
    __shared__ __align__(1024) uint16_t smem[4 * TILE];  // K0 V0 K1 V1

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, h = lane >> 5, l32 = lane & 31;
    const int g = lane >> 4, s16 = lane & 15;
    const int64_t nqb = (p.sq + QB - 1) / QB;
    int64_t unit, qblk;
    xcd_order(int64_t(gridDim.x) / nqb, nqb, unit, qblk);
    if (CAUSAL) qblk = nqb - 1 - qblk;  // longest rows first
    const int64_t b = unit / p.heads, n = unit % p.heads;
    const int64_t nkv = n / (p.heads / p.kv_heads);
    const int64_t q0 = qblk * QB;
    const int64_t qi = q0 + wave * 32 + l32;
    const bool qvalid = qi < p.sq;
    const int64_t wq_last = q0 + wave * 32 + 31;  // the wave's last query

    const uint16_t *qp = p.q + b * p.q_b + n * p.q_n;
    const uint16_t *kp = p.k + b * p.k_b + nkv * p.k_n;
    const uint16_t *vp = p.v + b * p.v_b + nkv * p.v_n;

    const int64_t shift = p.sk - p.sq;  // key j is visible to query i when j <= i + shift
    int64_t kend = p.sk;
    if (CAUSAL) kend = min(p.sk, q0 + QB + shift);
    const int ntiles = kend > 0 ? int((kend + BN - 1) / BN) : 0;
    // tiles before `nfull` need no mask for any query of the workgroup
    int64_t full_end = p.sk;
    if (CAUSAL) full_end = min(full_end, q0 + shift + 1);
    const int nfull = full_end > 0 ? int(full_end / BN) : 0;

    zero_tiles(smem, 4 * TILE, p.sk % BN || p.hd < D || p.hdv < D);
    if (ntiles > 0) {
        load_tile_async<D, NW>(kp, p.k_s, 0, p.sk, smem, wave, lane, p.hd);
        load_tile_async<D, NW>(vp, p.v_s, 0, p.sk, smem + TILE, wave, lane, p.hdv);
    }

    uint4 qf[DS];
#pragma unroll
    for (int t = 0; t < DS; ++t)
        qf[t] = qvalid && 16 * t + 8 * h < p.hd ? *reinterpret_cast<const uint4 *>(qp + qi * p.q_s + 16 * t + 8 * h)
                                                : make_uint4(0, 0, 0, 0);

    f32x16_t acc[DT];
#pragma unroll
    for (int i = 0; i < DT; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[i][e] = 0.0f;
    const float c2 = p.scale * 1.4426950408889634f;  // scale * log2(e)
    float m = -1e30f, l = 0.0f;                       // running max (base 2, scaled) and sum

    for (int kt = 0; kt < ntiles; ++kt) {
        const int64_t k0 = int64_t(kt) * BN;
        const uint16_t *Ks = smem + (kt & 1) * 2 * TILE;
        const uint16_t *Vs = Ks + TILE;
        __builtin_amdgcn_s_waitcnt(0);  // this thread's loads of tile kt have landed
        __syncthreads();                // ... and every thread's; tile kt-1's buffer is free
        if (kt + 1 < ntiles) {
            uint16_t *nk = smem + ((kt + 1) & 1) * 2 * TILE;
            load_tile_async<D, NW>(kp, p.k_s, k0 + BN, p.sk, nk, wave, lane, p.hd);
            load_tile_async<D, NW>(vp, p.v_s, k0 + BN, p.sk, nk + TILE, wave, lane, p.hdv);
        }
        if (CAUSAL && k0 > wq_last + shift) continue;  // every key of the tile is masked for this wave
        const char *Kb = reinterpret_cast<const char *>(Ks);
        const char *Vb = reinterpret_cast<const char *>(Vs);

        f32x16_t s[2];
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
            for (int e = 0; e < 16; ++e) s[ks][e] = 0.0f;
#pragma unroll
            for (int t = 0; t < DS; ++t) {
                uint4 a = *reinterpret_cast<const uint4 *>(Kb + kv_off<D>(32 * ks + l32, 16 * t + 8 * h));
                s[ks] = mfma32<F16>(a, qf[t], s[ks]);
            }
        }
        float mx = -INFINITY;
        if (kt >= nfull) {  // diagonal or ragged tile
            const int64_t lim = min(CAUSAL ? qi + shift : p.sk - 1, p.sk - 1) - k0 - 4 * h;
#pragma unroll
            for (int ks = 0; ks < 2; ++ks)
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const int kk = 32 * ks + 8 * (e / 4) + (e % 4);
                    s[ks][e] = (kk <= lim) ? s[ks][e] : -INFINITY;
                }
        }
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
#pragma unroll
            for (int e = 0; e < 16; ++e) mx = fmaxf(mx, s[ks][e]);
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64)) * c2;
        // raise m only when some row's maximum outgrew it by 2^8
        if (__any(mx > m + 8.0f)) {
            const float mnew = fmaxf(m, mx);
            const float alpha = fast_exp2(m - mnew);
            l *= alpha;
#pragma unroll
            for (int i = 0; i < DT; ++i)
#pragma unroll
                for (int e = 0; e < 16; ++e) acc[i][e] *= alpha;
            m = mnew;
        }
        float rs = 0.0f;
        uint4 pb[4];
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
#pragma unroll
            for (int half = 0; half < 2; ++half) {
                uint32_t w[4];
#pragma unroll
                for (int j = 0; j < 8; j += 2) {
                    const float e0 = fast_exp2(fmaf(s[ks][8 * half + j], c2, -m));
                    const float e1 = fast_exp2(fmaf(s[ks][8 * half + j + 1], c2, -m));
                    rs += e0 + e1;
                    w[j / 2] = pack2<F16>(e0, e1);
                }
                pb[2 * ks + half] = make_uint4(w[0], w[1], w[2], w[3]);
            }
        l += rs + __shfl_xor(rs, 32, 64);
#pragma unroll
        for (int t2 = 0; t2 < 4; ++t2) {
            const int key = 16 * t2 + 4 * h + s16 / 4;
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) {
                const int col = 32 * dt + 16 * (g & 1) + 4 * (s16 & 3);
                v4i16_t x = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_t *)(Vb + kv_off<D>(key, col)));
                v4i16_t y = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_t *)(Vb + kv_off<D>(key + 8, col)));
                uint2 xa = __builtin_bit_cast(uint2, x), ya = __builtin_bit_cast(uint2, y);
                acc[dt] = mfma32<F16>(make_uint4(xa.x, xa.y, ya.x, ya.y), pb[t2], acc[dt]);
            }
        }
    }

    if (!qvalid) return;
    const float inv = l > 0.0f ? 1.0f / l : 0.0f;
    uint16_t *op = p.o + b * p.o_b + n * p.o_n + qi * p.o_s;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int e4 = 0; e4 < 4; ++e4) {
            if (32 * dt + 8 * e4 >= p.hdv) continue;  // padded columns
            const uint32_t w0 = pack2<F16>(acc[dt][4 * e4 + 0] * inv, acc[dt][4 * e4 + 1] * inv);
            const uint32_t w1 = pack2<F16>(acc[dt][4 * e4 + 2] * inv, acc[dt][4 * e4 + 3] * inv);
            *reinterpret_cast<uint2 *>(op + 32 * dt + 8 * e4 + 4 * h) = make_uint2(w0, w1);
        }
    if (h == 0 && p.lse) p.lse[(b * p.heads + n) * p.sq + qi] = l > 0.0f ? (m + __log2f(l)) * 0.6931471805599453f : -INFINITY;
}

template <bool F16>
__device__ __forceinline__ float half_to_f32(uint16_t v) {
    return F16 ? f16_to_f32(v) : bf16_to_f32(v);
}

// ---- backward -----------------------------------------------------------------------------------
//
// The FA-2 backward arranged like the pipelined forward: operand tiles stream HBM -> LDS with
// global_load_lds into swizzled, double-buffered tiles; P = 2^(s * scale * log2 e - lse * log2 e) with the
// base-2 LSE written once by the delta kernel; masks only on tiles that cross the diagonal or the end of the
// queries.

// delta = rowsum(dO * O) * scale and lse2 = lse * log2(e), float32 [B, N, Sq] each; one wavefront a query
// row.
template <int D, bool F16>
__global__ __launch_bounds__(256) void flash_prep_kernel(AttnParams p, float *lse2) {
    const int lane = threadIdx.x & 63;
    const int64_t row = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
    const int64_t b = blockIdx.y;
    if (row >= p.heads * p.sq) return;
    const int64_t n = row / p.sq, q = row % p.sq;
    const uint16_t *o = p.o_in + b * p.o_b + n * p.o_n + q * p.o_s;
    const uint16_t *g = p.d_o + b * p.do_b + n * p.do_n + q * p.do_s;
    float acc = 0.0f;
    for (int d = lane; d < p.hdv; d += 64) acc += half_to_f32<F16>(g[d]) * half_to_f32<F16>(o[d]);
    acc = wave_sum(acc);
    const int64_t i = (b * p.heads + n) * p.sq + q;
    if (p.dqacc)  // the row of the atomic dQ accumulator starts at zero
        for (int d = lane; d < D; d += 64) p.dqacc[i * D + d] = 0.0f;
    if (lane == 0) {
        p.delta[i] = acc * p.scale;  // delta times the softmax scale: dS = P (dP scale - delta scale)
        lse2[i] = p.lse_in[i] * 1.4426950408889634f;
    }
}

// The same with 16-byte loads: D / 8 lanes a query row (a wavefront takes 64 / (D / 8) rows), the lanes'
// products summed in fixed order (each lane's eight, then a butterfly across the lanes of the row). Needs D
// a multiple of 8 dividing 512 and 16-byte aligned rows (the launcher checks).
template <int D, bool F16>
__global__ __launch_bounds__(256) void flash_prep_vec_kernel(AttnParams p, float *lse2) {
    constexpr int LPR = D / 8;          // lanes a row
    constexpr int RPB = 256 / LPR;      // rows a workgroup
    static_assert(D % 8 == 0 && 64 % LPR == 0, "rows must tile a wavefront");
    const int sub = threadIdx.x % LPR;
    const int64_t row = int64_t(blockIdx.x) * RPB + threadIdx.x / LPR;
    const int64_t b = blockIdx.y;
    const bool live = row < p.heads * p.sq;
    const int64_t n = live ? row / p.sq : 0, q = live ? row % p.sq : 0;
    float acc = 0.0f;
    if (live) {
        const uint4 ov = *reinterpret_cast<const uint4 *>(p.o_in + b * p.o_b + n * p.o_n + q * p.o_s + 8 * sub);
        const uint4 gv = *reinterpret_cast<const uint4 *>(p.d_o + b * p.do_b + n * p.do_n + q * p.do_s + 8 * sub);
        const uint32_t ow[4] = {ov.x, ov.y, ov.z, ov.w}, gw[4] = {gv.x, gv.y, gv.z, gv.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            acc += half_to_f32<F16>(uint16_t(gw[e] & 0xffffu)) * half_to_f32<F16>(uint16_t(ow[e] & 0xffffu));
            acc += half_to_f32<F16>(uint16_t(gw[e] >> 16)) * half_to_f32<F16>(uint16_t(ow[e] >> 16));
        }
    }
#pragma unroll
    for (int o = LPR / 2; o > 0; o >>= 1) acc += __shfl_xor(acc, o, 64);
    if (live && p.dqacc) {  // the row of the atomic dQ accumulator starts at zero
        float4 *z = reinterpret_cast<float4 *>(p.dqacc + ((b * p.heads + n) * p.sq + q) * D + 8 * sub);
        z[0] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        z[1] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
    if (live && sub == 0) {
        const int64_t i = (b * p.heads + n) * p.sq + q;
        p.delta[i] = acc * p.scale;
        lse2[i] = p.lse_in[i] * 1.4426950408889634f;
    }
}

// Component i (a constant) of a float4.
__device__ __forceinline__ float f4_at(const float4 &v, int i) { return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w; }

// 64 floats [k0, k0 + 64) of `src` (clamped to `rows`) into LDS by one wavefront.
__device__ __forceinline__ void load_row64_async(const float *src, int64_t k0, int64_t rows, float *dst, int lane) {
    int64_t r = k0 + lane;
    r = r < rows ? r : rows - 1;
    __builtin_amdgcn_global_load_lds(src + r, (lds_void_t *)dst, 4, 0, 0);
}

// dK and dV for 128 keys (32 a wavefront, one key a lane of the C layout), looping over 64-query tiles of
// every query head sharing the key/value head.
//
// ATOMIC_DQ (the non-deterministic mode): the workgroup also adds each tile's dQ = dS K into the float32
// accumulator p.dqacc, so no second kernel recomputes S and dP. The 128 keys' K rows stay in LDS for the
// whole loop; each wave writes its dS (one key a lane) into a [query][key] LDS tile, and after a barrier each
// wave computes dQ for its share of the 64 x D tile (32 head-dim columns, both query halves at D = 128; one
// half at D = 64) over all 128 keys: A = dS rows (one query a lane), B = K read transposed (one head-dim
// column a lane). Its adds are issued at the start of the next tile, so the wait for that tile's loads does
// not also wait for adds just issued.
template <int D> struct DkdvLds {
    static constexpr int kTile = 64 * D;              // a Q or dO tile, elements
    static constexpr int kDsPitch = 128 + 8;          // dS row pitch (elements): rows on distinct banks
    static constexpr int kBase = 4 * kTile;           // Q0 dO0 Q1 dO1
    static constexpr int kAtomic = kBase + 128 * D + 64 * kDsPitch;  // + K (128 keys) + dS
    static constexpr int kStagePitch = 72;                           // STORE_DS staging row pitch (elements)
    static constexpr int kStore = kBase + 4 * 32 * kStagePitch;      // + each wave's [32 keys][64 queries] dS
};

// Whether a dK/dV workgroup takes a pair of causal key blocks.
template <bool CAUSAL, bool ATOMIC_DQ> struct DkdvPaired { static constexpr bool value = CAUSAL && !ATOMIC_DQ; };

// STORE_DS (the deterministic mode's default): each tile's dS (rounded as for dK) is stored to p.ds for the
// dQ = dS K kernel, instead of a second kernel recomputing S and dP.
template <int D, bool F16, bool CAUSAL, bool ATOMIC_DQ = false, bool STORE_DS = false>
__global__ __launch_bounds__(256) void flash_dkdv_kernel(AttnParams p, const float *lse2) {
    constexpr int BM = 64;
    constexpr int DS = D / 16, DT = D / 32;
    constexpr int TILE = BM * D;
    __shared__ __align__(1024) uint16_t smem[ATOMIC_DQ ? DkdvLds<D>::kAtomic : STORE_DS ? DkdvLds<D>::kStore : DkdvLds<D>::kBase];
    __shared__ __align__(16) float Ls[2][BM];
    __shared__ __align__(16) float Dl[2][BM];
    uint16_t *const Ks = smem + DkdvLds<D>::kBase;    // ATOMIC_DQ: K rows [128][D], swizzled like a Q tile
    uint16_t *const dSb = Ks + 128 * D;               // ATOMIC_DQ: dS [64 queries][kDsPitch]
    (void)Ks;
    (void)dSb;

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, h = lane >> 5, l32 = lane & 31;
    const int g = lane >> 4, s16 = lane & 15;
    const int64_t nkb = (p.sk + 127) / 128;
    // causal (but for the atomic mode, whose registers it would spill): a workgroup takes key blocks i and
    // nkb - 1 - i (every workgroup then has the same number of query tiles but for the middle block of an odd
    // count), so no workgroup is left running alone at the end
    constexpr bool PAIR = DkdvPaired<CAUSAL, ATOMIC_DQ>::value;
    const int64_t per = PAIR ? (nkb + 1) / 2 : nkb;
    int64_t unit, pidx;
    xcd_order(int64_t(gridDim.x) / per, per, unit, pidx);
    const int64_t b = unit / p.kv_heads, nkv = unit % p.kv_heads;
    zero_tiles(smem, ATOMIC_DQ ? DkdvLds<D>::kBase + 128 * D : DkdvLds<D>::kBase,
               p.sq % BM || (ATOMIC_DQ && p.sk % 128) || p.hd < D || p.hdv < D);
    for (int pass = 0; pass < (PAIR ? 2 : 1); ++pass) {
    const int64_t kblk = pass == 0 ? pidx : nkb - 1 - pidx;
    if (pass == 1) {
        if (kblk == pidx) break;
        __syncthreads();  // every wave is done with the first block's LDS tiles
    }
    [&]() {
    const int64_t kb0 = kblk * 128;
    const int64_t kj = kb0 + wave * 32 + l32;
    const bool kvalid = kj < p.sk;
    const int64_t group = p.heads / p.kv_heads;
    const int64_t shift = p.sk - p.sq;

    const uint16_t *kp = p.k + b * p.k_b + nkv * p.k_n;
    const uint16_t *vp = p.v + b * p.v_b + nkv * p.v_n;

    // query tiles: [qstart, sq) for every head of the group; tile j < nfull needs no mask
    int64_t qstart = 0;
    if (CAUSAL) qstart = max<int64_t>(0, kb0 - shift) / BM * BM;
    const int per_head = p.sq > qstart ? int((p.sq - qstart + BM - 1) / BM) : 0;
    const int total = per_head * int(group);
    auto tile_src = [&](int j, const uint16_t *&qp, const uint16_t *&gp, const float *&ls, const float *&dl,
                        int64_t &q0) {
        const int64_t gi = j / per_head;
        q0 = qstart + int64_t(j % per_head) * BM;
        const int64_t n = nkv * group + gi;
        qp = p.q + b * p.q_b + n * p.q_n;
        gp = p.d_o + b * p.do_b + n * p.do_n;
        ls = lse2 + (b * p.heads + n) * p.sq;
        dl = p.delta + (b * p.heads + n) * p.sq;
    };
    auto issue = [&](int j) {
        const uint16_t *qp, *gp;
        const float *ls, *dl;
        int64_t q0;
        tile_src(j, qp, gp, ls, dl, q0);
        uint16_t *dst = smem + (j & 1) * 2 * TILE;
        load_tile_async<D>(qp, p.q_s, q0, p.sq, dst, wave, lane, p.hd);
        load_tile_async<D>(gp, p.do_s, q0, p.sq, dst + TILE, wave, lane, p.hdv);
        if (wave == 0) load_row64_async(ls, q0, p.sq, Ls[j & 1], lane);
        if (wave == 1) load_row64_async(dl, q0, p.sq, Dl[j & 1], lane);
    };
    if constexpr (ATOMIC_DQ) {  // waited for with the first tile's loads
        load_tile_async<D>(kp, p.k_s, kb0, p.sk, Ks, wave, lane, p.hd);
        load_tile_async<D>(kp, p.k_s, kb0 + 64, p.sk, Ks + 64 * D, wave, lane, p.hd);
    }
    if (total > 0) issue(0);

    // ATOMIC_DQ: this wave's dQ share of the previous tile, waiting to be added: NQ accumulators of 32 queries
    // x 32 head-dim columns (query half qh0 + c, columns 32 * dblk ...)
    constexpr int NQ = D == 128 ? 2 : 1;
    const int dblk = D == 128 ? wave : (wave & 1), qh0 = D == 128 ? 0 : (wave >> 1);
    f32x16_t adq[NQ];
    float *dq_rows = nullptr;  // the previous tile's first dQ accumulator row (query q0, head n)
    int64_t dq_left = 0;       // rows of that tile inside the queries
    (void)qh0;
    auto flush_dq = [&]() {
        if constexpr (ATOMIC_DQ) {
            if (!dq_rows) return;
#pragma unroll
            for (int c = 0; c < NQ; ++c)
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const int r = 32 * (qh0 + c) + 8 * (e / 4) + 4 * h + (e % 4);
                    if (r < dq_left) unsafeAtomicAdd(dq_rows + int64_t(r) * D + 32 * dblk + l32, adq[c][e]);
                }
            dq_rows = nullptr;
        }
    };

    uint4 kf[DS], vf[DS];
#pragma unroll
    for (int t = 0; t < DS; ++t) {
        kf[t] = kvalid && 16 * t + 8 * h < p.hd ? *reinterpret_cast<const uint4 *>(kp + kj * p.k_s + 16 * t + 8 * h)
                                                : make_uint4(0, 0, 0, 0);
        vf[t] = kvalid && 16 * t + 8 * h < p.hdv ? *reinterpret_cast<const uint4 *>(vp + kj * p.v_s + 16 * t + 8 * h)
                                                 : make_uint4(0, 0, 0, 0);
    }
    f32x16_t adk[DT], adv[DT];
#pragma unroll
    for (int i = 0; i < DT; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) adk[i][e] = adv[i][e] = 0.0f;
    const float c2 = p.scale * 1.4426950408889634f;

    for (int j = 0; j < total; ++j) {
        int64_t q0;
        {
            const uint16_t *qp, *gp;
            const float *ls, *dl;
            tile_src(j, qp, gp, ls, dl, q0);
        }
        // this thread's loads of tile j have landed; with STORE_DS the previous tile's 4 dS stores, issued after
        // them, may stay in flight (vector memory operations complete in order: vmcnt <= 4)
        if (STORE_DS && j > 0) __builtin_amdgcn_s_waitcnt(4 | (7 << 4));
        else __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        flush_dq();  // the previous tile's dQ adds, ahead of this iteration's loads
        if (j + 1 < total) issue(j + 1);
        const char *Qb = reinterpret_cast<const char *>(smem + (j & 1) * 2 * TILE);
        const char *Gb = Qb + TILE * 2;
        const float *Lt = Ls[j & 1], *Dt = Dl[j & 1];
        // rows q with q > sq - 1 or (causal) kj > q + shift are masked: tile row r is kept when rmin <= r < rmax
        // (with ATOMIC_DQ or STORE_DS also the key block past sk: its keys' P is zeroed)
        const bool masked = q0 + BM > p.sq || (CAUSAL && q0 + shift < kb0 + 127) ||
                            ((ATOMIC_DQ || STORE_DS) && kb0 + 128 > p.sk);
        const int rmin = CAUSAL ? int(min<int64_t>(max<int64_t>(kj - shift - q0, 0), BM)) : 0;
        const int rmax = int(min<int64_t>(p.sq - q0, BM));

        // phase 1: S and dP of both 32-query halves (4 independent MFMA chains), row fragments of Q and dO read
        // one k step ahead
        f32x16_t sv[2], dp[2];
#pragma unroll
        for (int qs = 0; qs < 2; ++qs)
#pragma unroll
            for (int e = 0; e < 16; ++e) sv[qs][e] = dp[qs][e] = 0.0f;
        uint4 fq[2][2], fg[2][2];
        auto rows = [&](int buf, int t) {
#pragma unroll
            for (int qs = 0; qs < 2; ++qs) {
                const int off = kv_off<D>(32 * qs + l32, 16 * t + 8 * h);
                fq[buf][qs] = *reinterpret_cast<const uint4 *>(Qb + off);
                fg[buf][qs] = *reinterpret_cast<const uint4 *>(Gb + off);
            }
        };
        rows(0, 0);
#pragma unroll
        for (int t = 0; t < DS; ++t) {
            const int cur = t & 1;
            if (t + 1 < DS) rows(cur ^ 1, t + 1);
#pragma unroll
            for (int qs = 0; qs < 2; ++qs) {
                sv[qs] = mfma32<F16>(fq[cur][qs], kf[t], sv[qs]);
                dp[qs] = mfma32<F16>(fg[cur][qs], vf[t], dp[qs]);
            }
        }
        // issue order: two k steps of reads, then one read of k step t + 2 after each MFMA of step t
        __builtin_amdgcn_sched_group_barrier(0x100, 8, 1);
        mfma_then_ds<4 * DS - 8, 1, 1>();
        __builtin_amdgcn_sched_group_barrier(0x008, 8, 1);
        __builtin_amdgcn_sched_barrier(0);

        // phase 2: P = 2^(S scale log2 e - lse log2 e) and dS = P (dP - delta) scale, packed as B operands
        uint4 pb[2][2], sb[2][2];
        auto probs = [&](auto maskedc) {
            constexpr bool MASKED = decltype(maskedc)::value;
#pragma unroll
            for (int qs = 0; qs < 2; ++qs)
#pragma unroll
                for (int half = 0; half < 2; ++half) {
                    // the rows' base-2 LSE and scaled delta, four consecutive rows a 16-byte LDS read
                    float4 l4[2], d4[2];
#pragma unroll
                    for (int j4 = 0; j4 < 2; ++j4) {
                        const int r4 = 32 * qs + 8 * (2 * half + j4) + 4 * h;
                        l4[j4] = *reinterpret_cast<const float4 *>(Lt + r4);
                        d4[j4] = *reinterpret_cast<const float4 *>(Dt + r4);
                    }
                    uint32_t wp[4], ws[4];
#pragma unroll
                    for (int jj = 0; jj < 8; jj += 2) {
                        float pv[2], dv2[2];
#pragma unroll
                        for (int u = 0; u < 2; ++u) {
                            const int e = 8 * half + jj + u;
                            const int r = 32 * qs + 8 * (e / 4) + 4 * h + (e % 4);
                            const float lr = f4_at(l4[(jj + u) / 4], (jj + u) % 4);
                            const float dr = f4_at(d4[(jj + u) / 4], (jj + u) % 4);
                            float pe = fast_exp2(fmaf(sv[qs][e], c2, -lr));
                            if constexpr (MASKED) pe = ((r >= rmin) & (r < rmax)) ? pe : 0.0f;
                            if constexpr (MASKED && (ATOMIC_DQ || STORE_DS)) pe = kvalid ? pe : 0.0f;  // keys past sk add nothing to dQ
                            pv[u] = pe;
                            dv2[u] = pe * fmaf(dp[qs][e], p.scale, -dr);
                        }
                        wp[jj / 2] = pack2<F16>(pv[0], pv[1]);
                        ws[jj / 2] = pack2<F16>(dv2[0], dv2[1]);
                    }
                    pb[qs][half] = make_uint4(wp[0], wp[1], wp[2], wp[3]);
                    sb[qs][half] = make_uint4(ws[0], ws[1], ws[2], ws[3]);
                }
        };
        if (masked) probs(std::true_type{});
        else probs(std::false_type{});
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (STORE_DS) {
            // The tile's dS goes out in the dQ kernel's operand order (flash_dq_ds_kernel): for each 16-key step
            // ks and 32-query half qb of the tile, 64 lanes x 8 values, lane (q = lane & 31, h = lane >> 5)
            // holding dS[q][16 ks + 4 h + {0..3}] and dS[q][16 ks + 8 + 4 h + {0..3}] (1 KiB a fragment, 16 a
            // tile). sb[qs][half] holds the lane's key's queries r0 .. r0 + 3 and r0 + 8 .. r0 + 11 (r0 = 32 qs
            // + 16 half + 4 h); written into the wave's own LDS rows [32 keys][64 queries], they are read back
            // transposed (the B-operand read), each wave's two key steps x two query halves, and stored 16 bytes
            // a lane, 1 KiB contiguous an instruction. Masked rows and keys past sk hold zeros.
            uint16_t *stg = smem + DkdvLds<D>::kBase + wave * (32 * DkdvLds<D>::kStagePitch);
#pragma unroll
            for (int qs = 0; qs < 2; ++qs)
#pragma unroll
                for (int half = 0; half < 2; ++half) {
                    uint16_t *row = stg + l32 * DkdvLds<D>::kStagePitch + 32 * qs + 16 * half + 4 * h;
                    *reinterpret_cast<uint2 *>(row) = make_uint2(sb[qs][half].x, sb[qs][half].y);
                    *reinterpret_cast<uint2 *>(row + 8) = make_uint2(sb[qs][half].z, sb[qs][half].w);
                }
            const int64_t n_ = nkv * group + j / per_head;
            uint16_t *blk = p.ds + (((b * p.heads + n_) * nkb + kblk) * ((p.sq + 63) / 64) + q0 / 64) * (128 * 64);
            const char *sg = reinterpret_cast<const char *>(stg);
#pragma unroll
            for (int ksl = 0; ksl < 2; ++ksl)
#pragma unroll
                for (int qb = 0; qb < 2; ++qb) {
                    const int krow = 16 * ksl + 4 * h + s16 / 4;
                    const int col = 32 * qb + 16 * (g & 1) + 4 * (s16 & 3);
                    v4i16_t x = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                        (lds_v4i16_t *)(sg + (krow * DkdvLds<D>::kStagePitch + col) * 2));
                    v4i16_t y = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                        (lds_v4i16_t *)(sg + ((krow + 8) * DkdvLds<D>::kStagePitch + col) * 2));
                    const uint2 xa = __builtin_bit_cast(uint2, x), ya = __builtin_bit_cast(uint2, y);
                    const int f = (2 * wave + ksl) * 2 + qb;
                    // written once and read once by the next kernel, far beyond the caches: nontemporal
                    typedef unsigned int ntv4 __attribute__((ext_vector_type(4)));
                    ntv4 v = {xa.x, xa.y, ya.x, ya.y};
                    __builtin_nontemporal_store(v, reinterpret_cast<ntv4 *>(blk + f * 512 + lane * 8));
                }
        }

        // phase 3: dV^T += dO^T P and dK^T += Q^T dS (8 independent chains), transposed fragments read one step
        // ahead
        uint4 tg[2][DT], tq[2][DT];
        auto trs = [&](int buf, int step) {
            const int qs = step >> 1, half = step & 1;
            const int r0 = 32 * qs + 16 * half + 4 * h + s16 / 4;
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) {
                const int col = 32 * dt + 16 * (g & 1) + 4 * (s16 & 3);
                const int o0 = kv_off<D>(r0, col), o1 = kv_off<D>(r0 + 8, col);
                v4i16_t x = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_t *)(Gb + o0));
                v4i16_t y = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_t *)(Gb + o1));
                uint2 xa = __builtin_bit_cast(uint2, x), ya = __builtin_bit_cast(uint2, y);
                tg[buf][dt] = make_uint4(xa.x, xa.y, ya.x, ya.y);
                x = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_t *)(Qb + o0));
                y = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_t *)(Qb + o1));
                xa = __builtin_bit_cast(uint2, x), ya = __builtin_bit_cast(uint2, y);
                tq[buf][dt] = make_uint4(xa.x, xa.y, ya.x, ya.y);
            }
        };
        trs(0, 0);
#pragma unroll
        for (int step = 0; step < 4; ++step) {
            const int cur = step & 1, qs = step >> 1, half = step & 1;
            if (step + 1 < 4) trs(cur ^ 1, step + 1);
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) {
                adv[dt] = mfma32<F16>(tg[cur][dt], pb[qs][half], adv[dt]);
                adk[dt] = mfma32<F16>(tq[cur][dt], sb[qs][half], adk[dt]);
            }
        }
        // issue order: the first step's reads, then two reads of the next step after each MFMA
        __builtin_amdgcn_sched_group_barrier(0x100, 4 * DT, 2);
        mfma_then_ds<6 * DT, 2, 2>();
        __builtin_amdgcn_sched_group_barrier(0x008, 2 * DT, 2);
        __builtin_amdgcn_sched_barrier(0);

        if constexpr (ATOMIC_DQ) {
            // dS (16-bit, as packed for dK) into the [query][key] tile: this lane's key, its 32 queries
            const int key = 32 * wave + l32;
#pragma unroll
            for (int qs = 0; qs < 2; ++qs)
#pragma unroll
                for (int half = 0; half < 2; ++half) {
                    const uint32_t w[4] = {sb[qs][half].x, sb[qs][half].y, sb[qs][half].z, sb[qs][half].w};
#pragma unroll
                    for (int jj = 0; jj < 8; ++jj) {
                        const int e = 8 * half + jj;
                        const int r = 32 * qs + 8 * (e / 4) + 4 * h + (e % 4);
                        dSb[r * DkdvLds<D>::kDsPitch + key] = uint16_t(jj & 1 ? w[jj / 2] >> 16 : w[jj / 2] & 0xffffu);
                    }
                }
            __syncthreads();
            // dQ[q, d] = sum over the 128 keys of dS[q, key] K[key, d]: A = dS (one query a lane), B = K read
            // transposed (one head-dim column a lane). The transposed read gives lane half h the keys
            // k0 + 4 h + {0..3, 8..11} of a 16-key step, so the dS fragment takes the same keys.
#pragma unroll
            for (int c = 0; c < NQ; ++c)
#pragma unroll
                for (int e = 0; e < 16; ++e) adq[c][e] = 0.0f;
#pragma unroll
            for (int ks = 0; ks < 8; ++ks) {
                const int k0 = 16 * ks;
                const int krow = k0 + 4 * h + s16 / 4;
                const int col = 32 * dblk + 16 * (g & 1) + 4 * (s16 & 3);
                v4i16_t x = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_t *)(reinterpret_cast<char *>(Ks) + kv_off<D>(krow, col)));
                v4i16_t y = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_t *)(reinterpret_cast<char *>(Ks) + kv_off<D>(krow + 8, col)));
                const uint2 xa = __builtin_bit_cast(uint2, x), ya = __builtin_bit_cast(uint2, y);
                const uint4 kb = make_uint4(xa.x, xa.y, ya.x, ya.y);
#pragma unroll
                for (int c = 0; c < NQ; ++c) {
                    const int q = 32 * (qh0 + c) + l32;
                    const uint16_t *row = dSb + q * DkdvLds<D>::kDsPitch + k0 + 4 * h;
                    const uint2 lo = *reinterpret_cast<const uint2 *>(row), hi = *reinterpret_cast<const uint2 *>(row + 8);
                    const uint4 da = make_uint4(lo.x, lo.y, hi.x, hi.y);
                    adq[c] = mfma32<F16>(da, kb, adq[c]);
                }
            }
            {
                const uint16_t *qp_, *gp_;
                const float *ls_, *dl_;
                int64_t q0_;
                tile_src(j, qp_, gp_, ls_, dl_, q0_);
                const int64_t n_ = nkv * group + j / per_head;
                dq_rows = p.dqacc + ((b * p.heads + n_) * p.sq + q0_) * D;
                dq_left = p.sq - q0_;
            }
        }
    }
    if constexpr (ATOMIC_DQ) flush_dq();
    if (!kvalid) return;
    uint16_t *dkp = p.dk + b * p.dk_b + nkv * p.dk_n + kj * p.dk_s;
    uint16_t *dvp = p.dv + b * p.dv_b + nkv * p.dv_n + kj * p.dv_s;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int e4 = 0; e4 < 4; ++e4) {
            const int d = 32 * dt + 8 * e4 + 4 * h;
            if (32 * dt + 8 * e4 < p.hd)  // padded columns are not stored
                *reinterpret_cast<uint2 *>(dkp + d) =
                    make_uint2(pack2<F16>(adk[dt][4 * e4], adk[dt][4 * e4 + 1]), pack2<F16>(adk[dt][4 * e4 + 2], adk[dt][4 * e4 + 3]));
            if (32 * dt + 8 * e4 < p.hdv)
                *reinterpret_cast<uint2 *>(dvp + d) =
                    make_uint2(pack2<F16>(adv[dt][4 * e4], adv[dt][4 * e4 + 1]), pack2<F16>(adv[dt][4 * e4 + 2], adv[dt][4 * e4 + 3]));
        }
    }();
    }
}

// The atomic dQ accumulator (float32 [B, N, Sq, D]) rounded into dq (its strides): eight head-dim elements a
// thread, a 16-byte store when dq's rows allow it.
template <int D, bool F16>
__global__ __launch_bounds__(256) void flash_dq_round_kernel(AttnParams p) {
    const int64_t t = int64_t(blockIdx.x) * 256 + threadIdx.x;
    const int64_t row = t / (D / 8), c = (t % (D / 8)) * 8;
    const int64_t rows_all = p.heads * p.sq;
    if (row >= p.batch * rows_all) return;
    const int64_t b = row / rows_all, rem = row % rows_all, n = rem / p.sq, q = rem % p.sq;
    if (c >= p.hd) return;  // padded columns
    const float4 x = *reinterpret_cast<const float4 *>(p.dqacc + row * D + c);
    const float4 y = *reinterpret_cast<const float4 *>(p.dqacc + row * D + c + 4);
    uint16_t *dst = p.dq + b * p.dq_b + n * p.dq_n + q * p.dq_s + c;
    const uint4 v = make_uint4(pack2<F16>(x.x, x.y), pack2<F16>(x.z, x.w), pack2<F16>(y.x, y.y), pack2<F16>(y.z, y.w));
    if ((reinterpret_cast<uintptr_t>(dst) & 15) == 0) {
        *reinterpret_cast<uint4 *>(dst) = v;
    } else {
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            dst[2 * i] = uint16_t(w[i] & 0xffffu);
            dst[2 * i + 1] = uint16_t(w[i] >> 16);
        }
    }
}

// dQ = dS K from the dS tiles the dK/dV kernel stored (deterministic, nothing recomputed): 256 queries of one
// head a workgroup of 4 wavefronts, 64 keys a step; wave w owns the 64 queries of dS tile q0 / 64 + w and the
// whole head dim: C[d][q] += K^T dS^T (2 x D / 32 MFMA tiles), keys the k dimension. The dS operand comes from
// HBM straight into registers (the tiles are stored in operand order: 16 bytes a lane, 1 KiB a fragment, each
// read by one wave once); the K rows stream into LDS for the transposed reads, shared by the 4 waves. Both
// run two steps ahead (three LDS stages, three register sets; every wave issues every load, so the wait
// counts are uniform). Steps a wave's queries do not reach (causal) are skipped; so are key blocks whose dS
// tile the dK/dV kernel never wrote (all its keys after the tile's queries). dS is read once from HBM: 128
// bf16 products a byte at D = 128, so the kernel is HBM-bound below ~1 PFLOP/s.
template <int D, bool F16, bool CAUSAL>
__global__ __launch_bounds__(256, 2) void flash_dq_ds_kernel(AttnParams p) {
    constexpr int KT = 64, QB = 256, KS = KT / 16;
    constexpr int DSB = 128 * 64;                                     // one dS tile, elements
    constexpr int FN = D / 32;                                        // 32-column MFMA tiles of the head dim
    constexpr int KSTAGE = KT * D;                                    // K rows of a step in LDS, elements
    constexpr int KOPS = (64 / (1024 / (D * 2))) / 4;                 // K-row loads a lane a step
    __shared__ __align__(1024) uint16_t smem[3 * KSTAGE];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, h = lane >> 5, l32 = lane & 31;
    const int g = lane >> 4, s16 = lane & 15;
    const int64_t nqb = (p.sq + QB - 1) / QB;
    const int64_t units = int64_t(gridDim.x) / nqb;  // batch x heads
    const int64_t unit = blockIdx.x % units;
    const int64_t qb = nqb - 1 - blockIdx.x / units;  // causal: the last query blocks see the most keys; issued first
    const int64_t b = unit / p.heads, n = unit % p.heads;
    const int64_t nkv = n / (p.heads / p.kv_heads);
    const int64_t q0 = qb * QB;
    const int64_t nkb = (p.sk + 127) / 128, nqt = (p.sq + 63) / 64;
    const int64_t shift = p.sk - p.sq;
    int nk = int((p.sk + KT - 1) / KT);
    if (CAUSAL) nk = int(min<int64_t>(nk, (q0 + QB - 1 + shift) / KT + 1));
    const uint16_t *kp = p.k + b * p.k_b + nkv * p.k_n;
    const int64_t qt = q0 / 64 + wave;  // this wave's dS tile (64 queries)
    const int64_t qtc = qt < nqt ? qt : nqt - 1;
    const uint16_t *dsw = p.ds + ((b * p.heads + n) * nkb * nqt + qtc) * DSB + lane * 8;
    uint4 fs[2][KS][2];
    // K rows of step kt into LDS stage B (three stages: issued two steps ahead)
    auto issue_k = [&](auto bufc, int kt) {
        constexpr int B = decltype(bufc)::value;
        load_tile_async<D, 4>(kp, p.k_s, int64_t(kt) * KT, p.sk, smem + B * KSTAGE, wave, lane, p.hd);
    };
    // dS fragments of step kt into register set B (two sets: issued one step ahead): 16-key steps 4 (kt & 1) + kk
    // and query halves qh of the 128-key block kt / 2
    auto issue_ds = [&](auto bufc, int kt) {
        constexpr int B = decltype(bufc)::value;
        const uint16_t *src = dsw + int64_t(kt / 2) * nqt * DSB + (kt & 1) * 4 * 2 * 512;
#pragma unroll
        for (int kk = 0; kk < KS; ++kk)
#pragma unroll
            for (int qh = 0; qh < 2; ++qh) {
                // read once: nontemporal, so the stream of dS does not evict the K rows every query block re-reads
                typedef unsigned int ntv4 __attribute__((ext_vector_type(4)));
                const ntv4 v = __builtin_nontemporal_load(reinterpret_cast<const ntv4 *>(src + (2 * kk + qh) * 512));
                fs[B][kk][qh] = make_uint4(v.x, v.y, v.z, v.w);
            }
    };
    f32x16_t acc[2][FN];
#pragma unroll
    for (int qh = 0; qh < 2; ++qh)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[qh][j][e] = 0.0f;
    // step kt: its K rows were issued two steps ago and its dS one step ago, before the K rows of step kt + 1,
    // which alone may stay in flight (vmcnt <= the K loads of one step)
    auto step = [&](auto bdc, auto bkc, int kt) {
        constexpr int BD = decltype(bdc)::value, BK = decltype(bkc)::value;
        if (kt + 1 < nk) __builtin_amdgcn_s_waitcnt((KOPS & 15) | ((KOPS >> 4) << 14) | (7 << 4));
        else __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();  // every wave's K rows of step kt are in LDS; the stage of step kt - 1 is free
        if (kt + 1 < nk) issue_ds(std::integral_constant<int, 1 - BD>{}, kt + 1);
        if (kt + 2 < nk) issue_k(std::integral_constant<int, (BK + 2) % 3>{}, kt + 2);
        const bool live = qt < nqt && (!CAUSAL || (int64_t(kt) * KT <= qt * 64 + 63 + shift &&
                                                   qt >= max<int64_t>(0, int64_t(kt / 2) * 128 - shift) / 64));
        if (!live) return;
        const char *ks_ = reinterpret_cast<const char *>(smem + BK * KSTAGE);
#pragma unroll
        for (int kk = 0; kk < KS; ++kk) {
            const int krow = 16 * kk + 4 * h + s16 / 4;
#pragma unroll
            for (int j = 0; j < FN; ++j) {
                const int cold = 32 * j + 16 * (g & 1) + 4 * (s16 & 3);
                v4i16_t x = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_t *)(ks_ + kv_off<D>(krow, cold)));
                v4i16_t y = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_t *)(ks_ + kv_off<D>(krow + 8, cold)));
                const uint2 xa = __builtin_bit_cast(uint2, x), ya = __builtin_bit_cast(uint2, y);
                const uint4 kf = make_uint4(xa.x, xa.y, ya.x, ya.y);
#pragma unroll
                for (int qh = 0; qh < 2; ++qh) acc[qh][j] = mfma32<F16>(kf, fs[BD][kk][qh], acc[qh][j]);
            }
        }
    };
    zero_tiles(smem, 3 * KSTAGE, p.sk % KT || p.hd < D);
    if (nk > 0) {
        issue_k(std::integral_constant<int, 0>{}, 0);
        issue_ds(std::integral_constant<int, 0>{}, 0);
    }
    if (nk > 1) issue_k(std::integral_constant<int, 1>{}, 1);
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;
    for (int kt = 0; kt < nk; kt += 6) {
        step(I0{}, I0{}, kt);
        if (kt + 1 < nk) step(I1{}, I1{}, kt + 1);
        if (kt + 2 < nk) step(I0{}, I2{}, kt + 2);
        if (kt + 3 < nk) step(I1{}, I0{}, kt + 3);
        if (kt + 4 < nk) step(I0{}, I1{}, kt + 4);
        if (kt + 5 < nk) step(I1{}, I2{}, kt + 5);
    }
#pragma unroll
    for (int qh = 0; qh < 2; ++qh) {
        const int64_t q = qt * 64 + 32 * qh + l32;
        if (q >= p.sq) continue;
        uint16_t *dqp = p.dq + b * p.dq_b + n * p.dq_n + q * p.dq_s;
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int e4 = 0; e4 < 4; ++e4) {
                const int d = 32 * j + 8 * e4 + 4 * h;
                if (32 * j + 8 * e4 >= p.hd) continue;  // padded columns
                *reinterpret_cast<uint2 *>(dqp + d) = make_uint2(pack2<F16>(acc[qh][j][4 * e4], acc[qh][j][4 * e4 + 1]),
                                                                 pack2<F16>(acc[qh][j][4 * e4 + 2], acc[qh][j][4 * e4 + 3]));
            }
    }
}

// dQ for 128 queries (32 a wavefront), looping over 64-key tiles: S^T and dP^T one query a lane, dQ^T
// accumulated in registers (deterministic: no atomics).
template <int D, bool F16, bool CAUSAL>
__global__ __launch_bounds__(256, 2) void flash_dq_kernel(AttnParams p, const float *lse2) {
    constexpr int BN = 64;
    constexpr int DS = D / 16, DT = D / 32;
    constexpr int TILE = BN * D;
    __shared__ __align__(1024) uint16_t smem[4 * TILE];  // K0 V0 K1 V1

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, h = lane >> 5, l32 = lane & 31;
    const int g = lane >> 4, s16 = lane & 15;
    const int64_t nqb = (p.sq + 127) / 128;
    int64_t unit, qblk;
    xcd_order(int64_t(gridDim.x) / nqb, nqb, unit, qblk);
    if (CAUSAL) qblk = nqb - 1 - qblk;
    const int64_t b = unit / p.heads, n = unit % p.heads;
    const int64_t nkv = n / (p.heads / p.kv_heads);
    const int64_t q0 = qblk * 128;
    const int64_t qi = q0 + wave * 32 + l32;
    const bool qvalid = qi < p.sq;
    const int64_t shift = p.sk - p.sq;
    const int64_t wq_last = q0 + wave * 32 + 31;

    const uint16_t *qp = p.q + b * p.q_b + n * p.q_n;
    const uint16_t *gp = p.d_o + b * p.do_b + n * p.do_n;
    const uint16_t *kp = p.k + b * p.k_b + nkv * p.k_n;
    const uint16_t *vp = p.v + b * p.v_b + nkv * p.v_n;

    int64_t kend = p.sk;
    if (CAUSAL) kend = min(p.sk, q0 + 128 + shift);
    const int ntiles = kend > 0 ? int((kend + BN - 1) / BN) : 0;
    int64_t full_end = p.sk;
    if (CAUSAL) full_end = min(full_end, q0 + shift + 1);
    const int nfull = full_end > 0 ? int(full_end / BN) : 0;
    zero_tiles(smem, 4 * TILE, p.sk % BN || p.hd < D || p.hdv < D);
    if (ntiles > 0) {
        load_tile_async<D>(kp, p.k_s, 0, p.sk, smem, wave, lane, p.hd);
        load_tile_async<D>(vp, p.v_s, 0, p.sk, smem + TILE, wave, lane, p.hdv);
    }

    uint4 qf[DS], gf[DS];
#pragma unroll
    for (int t = 0; t < DS; ++t) {
        qf[t] = qvalid && 16 * t + 8 * h < p.hd ? *reinterpret_cast<const uint4 *>(qp + qi * p.q_s + 16 * t + 8 * h)
                                                : make_uint4(0, 0, 0, 0);
        gf[t] = qvalid && 16 * t + 8 * h < p.hdv ? *reinterpret_cast<const uint4 *>(gp + qi * p.do_s + 16 * t + 8 * h)
                                                 : make_uint4(0, 0, 0, 0);
    }
    const float l2 = qvalid ? lse2[(b * p.heads + n) * p.sq + qi] : 0.0f;
    const float dl = qvalid ? p.delta[(b * p.heads + n) * p.sq + qi] : 0.0f;
    const float c2 = p.scale * 1.4426950408889634f;
    f32x16_t acc[DT];
#pragma unroll
    for (int i = 0; i < DT; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[i][e] = 0.0f;

    for (int kt = 0; kt < ntiles; ++kt) {
        const int64_t k0 = int64_t(kt) * BN;
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (kt + 1 < ntiles) {
            uint16_t *nk = smem + ((kt + 1) & 1) * 2 * TILE;
            load_tile_async<D>(kp, p.k_s, k0 + BN, p.sk, nk, wave, lane, p.hd);
            load_tile_async<D>(vp, p.v_s, k0 + BN, p.sk, nk + TILE, wave, lane, p.hdv);
        }
        if (CAUSAL && k0 > wq_last + shift) continue;
        const char *Kb = reinterpret_cast<const char *>(smem + (kt & 1) * 2 * TILE);
        const char *Vb = Kb + TILE * 2;
        const bool masked = kt >= nfull;
        const int64_t lim = min(CAUSAL ? qi + shift : p.sk - 1, p.sk - 1) - k0 - 4 * h;
        uint4 sb[4];
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            f32x16_t sv, dp;
#pragma unroll
            for (int e = 0; e < 16; ++e) sv[e] = dp[e] = 0.0f;
#pragma unroll
            for (int t = 0; t < DS; ++t) {
                const int off = kv_off<D>(32 * ks + l32, 16 * t + 8 * h);
                uint4 a = *reinterpret_cast<const uint4 *>(Kb + off);
                uint4 c = *reinterpret_cast<const uint4 *>(Vb + off);
                sv = mfma32<F16>(a, qf[t], sv);
                dp = mfma32<F16>(c, gf[t], dp);
            }
#pragma unroll
            for (int half = 0; half < 2; ++half) {
                uint32_t w[4];
#pragma unroll
                for (int jj = 0; jj < 8; jj += 2) {
                    float ds2[2];
#pragma unroll
                    for (int u = 0; u < 2; ++u) {
                        const int e = 8 * half + jj + u;
                        float pe = fast_exp2(fmaf(sv[e], c2, -l2));
                        if (masked) {
                            const int kk = 32 * ks + 8 * (e / 4) + (e % 4);
                            pe = (qvalid && kk <= lim) ? pe : 0.0f;
                        }
                        ds2[u] = pe * fmaf(dp[e], p.scale, -dl);
                    }
                    w[jj / 2] = pack2<F16>(ds2[0], ds2[1]);
                }
                sb[2 * ks + half] = make_uint4(w[0], w[1], w[2], w[3]);
            }
        }
#pragma unroll
        for (int t2 = 0; t2 < 4; ++t2) {
            const int r0 = 16 * t2 + 4 * h + s16 / 4;
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) {
                const int col = 32 * dt + 16 * (g & 1) + 4 * (s16 & 3);
                v4i16_t x = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_t *)(Kb + kv_off<D>(r0, col)));
                v4i16_t y = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_t *)(Kb + kv_off<D>(r0 + 8, col)));
                uint2 xa = __builtin_bit_cast(uint2, x), ya = __builtin_bit_cast(uint2, y);
                acc[dt] = mfma32<F16>(make_uint4(xa.x, xa.y, ya.x, ya.y), sb[t2], acc[dt]);
            }
        }
    }
    if (!qvalid) return;
    uint16_t *dqp = p.dq + b * p.dq_b + n * p.dq_n + qi * p.dq_s;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int e4 = 0; e4 < 4; ++e4)
            if (32 * dt + 8 * e4 < p.hd)  // padded columns are not stored
            *reinterpret_cast<uint2 *>(dqp + 32 * dt + 8 * e4 + 4 * h) =
                make_uint2(pack2<F16>(acc[dt][4 * e4], acc[dt][4 * e4 + 1]), pack2<F16>(acc[dt][4 * e4 + 2], acc[dt][4 * e4 + 3]));
}

}  // namespace nhipk

namespace nhip {

// delta and the base-2 LSE, float32 [B, N, Sq] each.
// delta and the base-2 LSE (float32 [B, N, Sq] each), then, when not deterministic, the float32 dQ
// accumulator [B, N, Sq, D], 16-byte aligned after them.
// Backward workspace: delta and the base-2 LSE (2 floats a query row), then by mode (nhip_attn_desc.deterministic)
// 0: the float32 dQ accumulator [B, N, Sq, D]; 1: the dS tiles [B, N, ceil(Sk/128), ceil(Sq/64)][128][64] (16-bit);
// 2: nothing (dQ recomputes S and dP).
// The head dim the kernels run at: 64, 128 or 256, the operands' own head dim (a multiple of 8) padded up to it
// with zero columns.
inline int64_t kernel_head_dim(int64_t hd) { return hd <= 64 ? 64 : hd <= 128 ? 128 : 256; }
// V's (and O's, dO's) head dim: value_head_dim, or the query's when 0.
inline int64_t value_head_dim(const nhip_attn_desc *d) { return d->value_head_dim ? d->value_head_dim : d->head_dim; }
// The head dim the kernels run at for both.
inline int64_t kernel_dim(const nhip_attn_desc *d) {
    return kernel_head_dim(d->head_dim > value_head_dim(d) ? d->head_dim : value_head_dim(d));
}

inline size_t flash_bwd_dq_offset(const nhip_attn_desc *d) {
    return (2 * size_t(d->batch) * d->heads * d->sq * sizeof(float) + 255) / 256 * 256;
}
inline size_t flash_bwd_ds_bytes(const nhip_attn_desc *d) {
    return size_t(d->batch) * d->heads * size_t((d->sk + 127) / 128) * size_t((d->sq + 63) / 64) * 128 * 64 * 2;
}
inline size_t flash_bwd_workspace_bytes(const nhip_attn_desc *d) {
    if (d->deterministic == 2) return 2 * size_t(d->batch) * d->heads * d->sq * sizeof(float);
    if (d->deterministic == 1) return flash_bwd_dq_offset(d) + flash_bwd_ds_bytes(d);
    return flash_bwd_dq_offset(d) + size_t(d->batch) * d->heads * d->sq * kernel_dim(d) * sizeof(float);
}

inline nhipk::AttnParams attn_params(const nhip_attn_desc *d) {
    nhipk::AttnParams p{};
    p.sq = d->sq;
    p.sk = d->sk;
    p.heads = d->heads;
    p.kv_heads = d->kv_heads;
    p.batch = d->batch;
    p.hd = d->head_dim;
    p.hdv = value_head_dim(d);
    p.q_b = d->q_b, p.q_s = d->q_s, p.q_n = d->q_n;
    p.k_b = d->k_b, p.k_s = d->k_s, p.k_n = d->k_n;
    p.v_b = d->v_b, p.v_s = d->v_s, p.v_n = d->v_n;
    p.o_b = d->o_b, p.o_s = d->o_s, p.o_n = d->o_n;
    p.do_b = d->do_b, p.do_s = d->do_s, p.do_n = d->do_n;
    p.dq_b = d->dq_b, p.dq_s = d->dq_s, p.dq_n = d->dq_n;
    p.dk_b = d->dk_b, p.dk_s = d->dk_s, p.dk_n = d->dk_n;
    p.dv_b = d->dv_b, p.dv_s = d->dv_s, p.dv_n = d->dv_n;
    p.scale = d->scale;
    return p;
}

// The forward's tile configs (nhip_attn_desc.config; -1 is config 0): 0 = 4 waves (128 queries) a
// workgroup, 1 = 8 waves (256 queries), 2 = 2 waves (64 queries). The backward kernels have one tile each.
constexpr int kNumAttnConfigs = 3;

// A padded head dim reads its zero columns through buffer loads, which take 32-bit offsets: every (batch, head)
// slice of an operand must then span under 2 GiB (rows rounded up to the 64-row tiles).
inline bool attn_span_ok(int64_t rows, int64_t rs, int64_t hd) {
    return (((rows + 63) / 64 * 64) * rs + hd) * 2 < (int64_t(1) << 31);
}

inline int check_attn(const nhip_attn_desc *d, const char *what, int64_t max_hd = 128) {
    for (int64_t hd : {d->head_dim, value_head_dim(d)})
        if (hd <= 0 || hd % 8 || hd > max_hd)
            return fail(std::string(what) + ": head dim " + std::to_string(hd) +
                        " (the hip kernels take multiples of 8 up to " + std::to_string(max_hd) + ")");
    for (int64_t st : {d->q_b, d->q_s, d->q_n, d->k_b, d->k_s, d->k_n, d->v_b, d->v_s, d->v_n, d->o_b, d->o_s, d->o_n,
                       d->do_b, d->do_s, d->do_n, d->dq_b, d->dq_s, d->dq_n, d->dk_b, d->dk_s, d->dk_n, d->dv_b, d->dv_s,
                       d->dv_n})
        if (st % 8) return fail(std::string(what) + ": every stride must be a multiple of 8 elements (16-byte rows)");
    const int64_t hv = value_head_dim(d), kd = kernel_dim(d);
    if ((d->head_dim != kd || hv != kd) &&
        !(attn_span_ok(d->sq, d->q_s, d->head_dim) && attn_span_ok(d->sk, d->k_s, d->head_dim) &&
          attn_span_ok(d->sk, d->v_s, hv) && attn_span_ok(d->sq, d->o_s, hv) && attn_span_ok(d->sq, d->do_s, hv)))
        return fail(std::string(what) + ": head dims " + std::to_string(d->head_dim) + " / " + std::to_string(hv) +
                    " are padded to " + std::to_string(kd) + ", which needs each (batch, head) of an operand within 2 GiB");
    if (d->dtype != NHIP_BF16 && d->dtype != NHIP_F16) return fail(std::string(what) + ": bf16 or f16 operands only");
    if (d->kv_heads <= 0 || d->heads % d->kv_heads) return fail(std::string(what) + ": heads must be a multiple of kv_heads");
    if (d->deterministic < 0 || d->deterministic > 2)
        return fail(std::string(what) + ": backward mode (deterministic) " + std::to_string(d->deterministic) +
                    " (0 atomic dQ, 1 stored dS, 2 recomputed dQ)");
    if (d->config >= kNumAttnConfigs)
        return fail(std::string(what) + ": no attention tile config " + std::to_string(d->config));
    if (d->causal && d->sk < d->sq)
        return fail(std::string(what) + ": causal with fewer keys than queries (rows without keys) has no kernel");
    if ((d->sq + 63) / 64 * d->heads * d->batch >= (int64_t(1) << 31) || (d->sk + 127) / 128 * d->heads * d->batch >= (int64_t(1) << 31))
        return fail(std::string(what) + ": more than 2^31 workgroups");
    return 0;
}

template <int D, bool F16, bool CAUSAL, int NW>
int launch_fwd_nw(hipStream_t s, const nhipk::AttnParams &p, const nhip_attn_desc *d) {
    dim3 grid(unsigned((d->sq + 32 * NW - 1) / (32 * NW) * d->heads * d->batch));
    hipLaunchKernelGGL((nhipk::flash_fwd_kernel<D, F16, CAUSAL, NW>), grid, dim3(64 * NW), 0, s, p);
    return check(hipGetLastError(), "flash_fwd launch");
}

template <int D, bool F16, bool CAUSAL>
int launch_fwd(hipStream_t s, const nhipk::AttnParams &p, const nhip_attn_desc *d) {
    if constexpr (D > 128) {
        // head dim 256: 4 waves, one workgroup a CU (its K/V tiles fill 128 KiB of LDS), whatever the config
        return launch_fwd_nw<D, F16, CAUSAL, 4>(s, p, d);
    } else {
        switch (d->config < 0 ? 0 : d->config) {
            case 1: return launch_fwd_nw<D, F16, CAUSAL, 8>(s, p, d);
            case 2: return launch_fwd_nw<D, F16, CAUSAL, 2>(s, p, d);
            default: return launch_fwd_nw<D, F16, CAUSAL, 4>(s, p, d);
        }
    }
}

int flash_fwd_on(hipStream_t s, const nhip_attn_desc *d, const void *q, const void *k, const void *v, void *o,
                 float *lse) {
    if (check_attn(d, "flash attention", 256)) return 1;
    if (d->sq == 0 || d->batch == 0 || d->heads == 0) return 0;
    nhipk::AttnParams p = attn_params(d);
    p.q = static_cast<const uint16_t *>(q);
    p.k = static_cast<const uint16_t *>(k);
    p.v = static_cast<const uint16_t *>(v);
    p.o = static_cast<uint16_t *>(o);
    p.lse = lse;
    bool f16 = d->dtype == NHIP_F16;
#define NHIP_FWD(DD, FF, CC) return launch_fwd<DD, FF, CC>(s, p, d)
    const int64_t kd = kernel_dim(d);
    if (kd == 256) {
        if (f16) { if (d->causal) NHIP_FWD(256, true, true); NHIP_FWD(256, true, false); }
        if (d->causal) NHIP_FWD(256, false, true);
        NHIP_FWD(256, false, false);
    }
    if (kd == 128) {
        if (f16) { if (d->causal) NHIP_FWD(128, true, true); NHIP_FWD(128, true, false); }
        if (d->causal) NHIP_FWD(128, false, true);
        NHIP_FWD(128, false, false);
    }
    if (f16) { if (d->causal) NHIP_FWD(64, true, true); NHIP_FWD(64, true, false); }
    if (d->causal) NHIP_FWD(64, false, true);
    NHIP_FWD(64, false, false);
#undef NHIP_FWD
}

template <int D, bool F16, bool CAUSAL>
int launch_bwd(hipStream_t s, const nhipk::AttnParams &p, const nhip_attn_desc *d) {
    const bool atomic = p.dqacc != nullptr;
    dim3 gd(unsigned((d->heads * d->sq + 3) / 4), unsigned(d->batch));
    // dK/dV: a workgroup per key block, or per pair of key blocks (i, nkb - 1 - i) (nhipk::DkdvPaired)
    const int64_t nkb = (d->sk + 127) / 128;
    dim3 gk(unsigned((nhipk::DkdvPaired<CAUSAL, false>::value ? (nkb + 1) / 2 : nkb) * d->kv_heads * d->batch));
    dim3 gka(unsigned((nhipk::DkdvPaired<CAUSAL, true>::value ? (nkb + 1) / 2 : nkb) * d->kv_heads * d->batch));
    dim3 gq(unsigned((d->sq + 127) / 128 * d->heads * d->batch));
    float *lse2 = p.delta + size_t(d->batch) * d->heads * d->sq;
    // 16-byte rows: D / 8 lanes each; else one wavefront a row
    const bool vec = d->head_dim == D && value_head_dim(d) == D && D % 8 == 0 && 64 % (D / 8 > 0 ? D / 8 : 1) == 0 && D / 8 <= 64 &&
                     ((reinterpret_cast<uintptr_t>(p.o_in) | reinterpret_cast<uintptr_t>(p.d_o)) & 15) == 0 &&
                     (p.o_b | p.o_n | p.o_s | p.do_b | p.do_n | p.do_s) % 8 == 0;
    if constexpr (D % 8 == 0 && D >= 8 && D <= 512 && 64 % (D / 8) == 0) {
        if (vec) {
            constexpr int RPB = 256 / (D / 8);
            dim3 gv(unsigned((d->heads * d->sq + RPB - 1) / RPB), unsigned(d->batch));
            hipLaunchKernelGGL((nhipk::flash_prep_vec_kernel<D, F16>), gv, dim3(256), 0, s, p, lse2);
        } else {
            hipLaunchKernelGGL((nhipk::flash_prep_kernel<D, F16>), gd, dim3(256), 0, s, p, lse2);
        }
    } else {
        hipLaunchKernelGGL((nhipk::flash_prep_kernel<D, F16>), gd, dim3(256), 0, s, p, lse2);
    }
    if (check(hipGetLastError(), "flash delta launch")) return 1;
    if (atomic) {
        hipLaunchKernelGGL((nhipk::flash_dkdv_kernel<D, F16, CAUSAL, true>), gka, dim3(256), 0, s, p, lse2);
        if (check(hipGetLastError(), "flash dkdv+dq launch")) return 1;
        const int64_t rows = d->batch * d->heads * d->sq;
        dim3 gc(unsigned((rows * (D / 8) + 255) / 256));
        hipLaunchKernelGGL((nhipk::flash_dq_round_kernel<D, F16>), gc, dim3(256), 0, s, p);
        return check(hipGetLastError(), "flash dq rounding launch");
    }
    if (p.ds) {
        hipLaunchKernelGGL((nhipk::flash_dkdv_kernel<D, F16, CAUSAL, false, true>), gk, dim3(256), 0, s, p, lse2);
        if (check(hipGetLastError(), "flash dkdv+dS launch")) return 1;
        dim3 gs(unsigned((d->sq + 255) / 256 * d->heads * d->batch));
        hipLaunchKernelGGL((nhipk::flash_dq_ds_kernel<D, F16, CAUSAL>), gs, dim3(256), 0, s, p);
        return check(hipGetLastError(), "flash dq from dS launch");
    }
    hipLaunchKernelGGL((nhipk::flash_dkdv_kernel<D, F16, CAUSAL>), gk, dim3(256), 0, s, p, lse2);
    if (check(hipGetLastError(), "flash dkdv launch")) return 1;
    hipLaunchKernelGGL((nhipk::flash_dq_kernel<D, F16, CAUSAL>), gq, dim3(256), 0, s, p, lse2);
    return check(hipGetLastError(), "flash dq launch");
}

int flash_bwd_on(hipStream_t s, const nhip_attn_desc *d, const void *q, const void *k, const void *v, const void *o,
                 const void *d_o, const float *lse, void *dq, void *dk, void *dv, void *ws) {
    if (check_attn(d, "flash attention backward")) return 1;
    if (d->batch == 0 || d->heads == 0) return 0;
    nhipk::AttnParams p = attn_params(d);
    p.q = static_cast<const uint16_t *>(q);
    p.k = static_cast<const uint16_t *>(k);
    p.v = static_cast<const uint16_t *>(v);
    p.o_in = static_cast<const uint16_t *>(o);
    p.d_o = static_cast<const uint16_t *>(d_o);
    p.lse_in = lse;
    p.dq = static_cast<uint16_t *>(dq);
    p.dk = static_cast<uint16_t *>(dk);
    p.dv = static_cast<uint16_t *>(dv);
    p.delta = static_cast<float *>(ws);
    p.dqacc = d->deterministic ? nullptr : reinterpret_cast<float *>(static_cast<char *>(ws) + flash_bwd_dq_offset(d));
    p.ds = d->deterministic == 1 ? reinterpret_cast<uint16_t *>(static_cast<char *>(ws) + flash_bwd_dq_offset(d)) : nullptr;
    bool f16 = d->dtype == NHIP_F16;
#define NHIP_BWD(DD, FF, CC) return launch_bwd<DD, FF, CC>(s, p, d)
    if (kernel_dim(d) == 128) {
        if (f16) { if (d->causal) NHIP_BWD(128, true, true); NHIP_BWD(128, true, false); }
        if (d->causal) NHIP_BWD(128, false, true);
        NHIP_BWD(128, false, false);
    }
    if (f16) { if (d->causal) NHIP_BWD(64, true, true); NHIP_BWD(64, true, false); }
    if (d->causal) NHIP_BWD(64, false, true);
    NHIP_BWD(64, false, false);
#undef NHIP_BWD
}

}  // namespace nhip
