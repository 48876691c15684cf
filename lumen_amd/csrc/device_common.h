// Device helpers shared by the built-in kernels and the generated loop kernels: storage types, exact
// conversions and wavefront reductions for gfx950 (wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace nhipk {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

// 16-bit floats are stored as their bit patterns.
struct bf16_t {
    uint16_t bits;
};
struct f16_t {
    uint16_t bits;
};

__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __uint_as_float(uint32_t(b) << 16); }

// float32 -> bfloat16, round to nearest even; a NaN keeps its sign and top payload bits with the quiet bit
// set. A float32 value is the exact value here, so this is the reference's one correct rounding
// (lumen/tensor/dtype.rs:215-239). gfx950's conversion instruction (v_cvt_pk_bf16_f32) does exactly this: on
// MI355X it equals the integer form (u + 0x7fff + lsb) >> 16, NaN -> (u >> 16) | 0x40, on all 2^32 inputs.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }

__device__ __forceinline__ float f16_to_f32(uint16_t b) {
    _Float16 h = __builtin_bit_cast(_Float16, b);
    return float(h);
}

// float32 -> float16 by the hardware conversion (v_cvt_f16_f32: round to nearest even, overflow to inf).
__device__ __forceinline__ uint16_t f32_to_f16(float f) {
    _Float16 h = _Float16(f);
    return __builtin_bit_cast(uint16_t, h);
}

template <typename T>
struct Storage;
template <>
struct Storage<float> {
    __device__ static float load(const float *p) { return *p; }
    __device__ static void store(float *p, float v) { *p = v; }
};

__device__ __forceinline__ float load_as_f32(const float *p) { return *p; }
__device__ __forceinline__ float load_as_f32(const bf16_t *p) { return bf16_to_f32(p->bits); }
__device__ __forceinline__ float load_as_f32(const f16_t *p) { return f16_to_f32(p->bits); }
__device__ __forceinline__ void store_f32_as(float *p, float v) { *p = v; }
__device__ __forceinline__ void store_f32_as(bf16_t *p, float v) { p->bits = f32_to_bf16(v); }
__device__ __forceinline__ void store_f32_as(f16_t *p, float v) { p->bits = f32_to_f16(v); }

// Sum over the 64 lanes of a wavefront (every lane gets the total).
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// Maximum over the 64 lanes of a wavefront, NaN-propagating as the reference's fmax.
__device__ __forceinline__ float nan_max(float a, float b) { return (a != a || b != b) ? __builtin_nanf("") : fmaxf(a, b); }
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = nan_max(v, __shfl_xor(v, off, 64));
    return v;
}

// Scheduling constraint: M MFMAs with NR LDS reads spread evenly between them (sched_group_barrier groups
// of sync id ID, in issue order).
template <int T, int M, int NR, int ID>
__device__ __forceinline__ void mfma_ds_interleave() {
    if constexpr (T < M) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, ID);
        constexpr int r = NR * (T + 1) / M - NR * T / M;
        if constexpr (r > 0) __builtin_amdgcn_sched_group_barrier(0x100, r, ID);
        mfma_ds_interleave<T + 1, M, NR, ID>();
    }
}

// The same with NV global loads (VMEM reads, the loads into LDS) spread between the MFMAs as well.
template <int T, int M, int NR, int NV, int ID>
__device__ __forceinline__ void mfma_ds_vmem_interleave() {
    if constexpr (T < M) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, ID);
        constexpr int r = NR * (T + 1) / M - NR * T / M;
        if constexpr (r > 0) __builtin_amdgcn_sched_group_barrier(0x100, r, ID);
        constexpr int v = NV * (T + 1) / M - NV * T / M;
        if constexpr (v > 0) __builtin_amdgcn_sched_group_barrier(0x020, v, ID);
        mfma_ds_vmem_interleave<T + 1, M, NR, NV, ID>();
    }
}

// Scheduling constraint: N times {one MFMA, then R LDS reads} (sync id ID).
template <int N, int R, int ID>
__device__ __forceinline__ void mfma_then_ds() {
    if constexpr (N > 0) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, ID);
        if constexpr (R > 0) __builtin_amdgcn_sched_group_barrier(0x100, R, ID);
        mfma_then_ds<N - 1, R, ID>();
    }
}

}  // namespace nhipk
