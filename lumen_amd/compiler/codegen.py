"""HIP source for fused loop kernels (the hip counterpart of ``lumen/codegen/elementwise/cuda/mod.rs``,
``codegen/row/triton.rs``, ``codegen/reduction/triton.rs`` and the emitter ``codegen/emitter/cuda.rs``).

Every value of a kernel is evaluated at an index derived from the kernel's iteration index by walking its
producers (layout ops are index maps, never copies). Each primitive's result is rounded to its dtype exactly
where the reference rounds it: 16-bit floats are computed in float32 and rounded to nearest even after every
op (for + - * / and sqrt that is the one correct rounding of the reference's float64 result), float32 in
float32, float64 in float64; no FMA contraction (the generated code is compiled with -ffp-contract=off).

Kernels:
  * loop: flat iteration over the output elements, V consecutive elements a thread, 16-byte vector loads and
    stores for operands read at the iteration's own flat index, grid-stride over the whole tensor;
  * row: one workgroup (or one wavefront) a row of a row space R x C; each reduction over the row is a
    stage (wavefront shuffles, then LDS across wavefronts), its result a per-row scalar later stages read;
    element values a later stage needs again stay in registers (the row's work is unrolled);
  * reduce: any other reduction: threads over the outputs, workgroups over chunks of the reduced range,
    float32 partial sums added atomically into a zero-filled output.
"""

from __future__ import annotations

import math
import re
import struct

from lumen_amd import dtypes as D
from lumen_amd.graph.ir import Graph, TensorType


class Unfusable(Exception):
    """A fused group the generator cannot express (the plan then splits it)."""

    def __init__(self, var, msg):
        super().__init__(msg)
        self.var = var


HEADER = r"""
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <math.h>
#define DEV __device__ __forceinline__
DEV float lb_bf16(uint16_t b) { return __uint_as_float(uint32_t(b) << 16); }
// float32 -> bfloat16 round to nearest even, NaN -> (bits >> 16) | 0x40: gfx950's v_cvt_pk_bf16_f32, equal to
// that integer rounding on all 2^32 float32 inputs (checked on MI355X)
DEV uint16_t sb_bf16(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }
typedef float lk_f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 lk_bf16x2 __attribute__((ext_vector_type(2)));
// float32 rounded to bfloat16 and widened back: the pair {0, f} converted in one v_cvt_pk_bf16_f32 puts bf16(f)
// in the high half over a zero low half, which is that value as a float32 (the same bits as
// lb_bf16(sb_bf16(f)), NaN included), without the shift
DEV float r_bf16(float f) { return __builtin_bit_cast(float, __builtin_convertvector((lk_f32x2){0.0f, f}, lk_bf16x2)); }
// two float32 -> bfloat16 (a in the low half) in one v_cvt_pk_bf16_f32
DEV uint32_t sb2_bf16(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((lk_f32x2){a, b}, lk_bf16x2));
}
// a vector of 4, 8 or 16 bytes loaded nontemporal: the generated kernels' full-size operands are read once a
// launch, and keeping their lines would evict what other loads re-read
template <class T> DEV T ld_nt(const T *p) {
  if constexpr (sizeof(T) == 4) {
    return __builtin_bit_cast(T, __builtin_nontemporal_load(reinterpret_cast<const uint32_t *>(p)));
  } else {
    typedef uint32_t nv __attribute__((ext_vector_type(sizeof(T) / 4)));
    return __builtin_bit_cast(T, __builtin_nontemporal_load(reinterpret_cast<const nv *>(p)));
  }
}
// a vector stored nontemporal: for values no kernel reads until much later
template <class T> DEV void st_nt(T *p, const T &v) {
  if constexpr (sizeof(T) == 4) {
    __builtin_nontemporal_store(__builtin_bit_cast(uint32_t, v), reinterpret_cast<uint32_t *>(p));
  } else {
    typedef uint32_t nv __attribute__((ext_vector_type(sizeof(T) / 4)));
    __builtin_nontemporal_store(__builtin_bit_cast(nv, v), reinterpret_cast<nv *>(p));
  }
}
DEV float lb_f16(uint16_t b) { return float(__builtin_bit_cast(_Float16, b)); }
DEV uint16_t sb_f16(float f) { return __builtin_bit_cast(uint16_t, _Float16(f)); }
DEV float r_f16(float f) { return lb_f16(sb_f16(f)); }
// float64 -> float32 rounding to odd: composes with a later round to nearest into one correct rounding
// (lumen/tensor/dtype.rs:215-224), for float64 values cast to 16-bit floats.
DEV float ro_f32(double x) {
  float f = (float)x;
  uint32_t b = __float_as_uint(f);
  if (!isfinite(f) || (double)f == x || (b & 1u)) return f;
  bool outward = ((double)f < x) != (f < 0.0f || (f == 0.0f && signbit(f)));
  return __uint_as_float(outward ? b + 1u : b - 1u);
}
// tanh in float32: below 0.55 in magnitude x + x^3 q(x^2), q a degree-4 polynomial fitted (iteratively
// reweighted least squares) to (tanh x - x) / x^3 on [0, 0.55] for relative error under 3e-9; above it
// sign(x) (1 - 2 / (2^(2|x| log2 e) + 1)) on the hardware exp2 and reciprocal (2^... overflows to inf past
// |x| = 44, giving +-1; NaN propagates). Within 2 ulp of the exact value with correctly rounded exp2 and
// division (checked over [2^-31, 12] on the host).
// Both branches are evaluated and one selected: lanes of a wave straddle 0.55, so a branch would run both
// anyway, plus the exec-mask bookkeeping.
DEV float tanh_f32(float x) {
  const float ax = fabsf(x);
  const float x2 = x * x;
  float p = fmaf(x2, -6.349337287e-03f, 2.112270333e-02f);
  p = fmaf(x2, p, -5.386411399e-02f);
  p = fmaf(x2, p, 1.333269179e-01f);
  p = fmaf(x2, p, -3.333331943e-01f);
  const float small = fmaf(x * x2, p, x);
  const float e = __builtin_amdgcn_exp2f(2.8853900817779268f * ax);
  const float big = 1.0f - 2.0f * __builtin_amdgcn_rcpf(e + 1.0f);
  return copysignf(ax < 0.55f ? small : big, x);  // keeps the sign of -0; NaN propagates through big
}
// exp in float32: x log2 e split into the rounded product hi and its error lo (fma residual plus x times
// the low part of log2 e), then 2^hi on the hardware exp2 times (1 + lo ln 2). Within 2 ulp of the exact
// value for normal results with a correctly rounded exp2 (checked on the host over every 13th float); results
// below 2^-126 flush to zero; +-inf and NaN map to inf / 0 / NaN.
DEV float exp_f32(float x) {
  const float hi = x * 1.4426950216293335f;
  float lo = fmaf(x, 1.4426950216293335f, -hi) + x * 1.9259629890910901e-08f;
  lo = __builtin_isinf(x) ? 0.0f : lo;
  const float r = __builtin_amdgcn_exp2f(hi);
  return r * fmaf(lo, 0.6931471805599453f, 1.0f);
}
// a / b in float32 within 1 ulp (Markstein): the hardware reciprocal refined by one Newton step (rcp_f32), the
// quotient a * r corrected once by its residual a - b q. A zero quotient keeps a's sign (the correction would
// give +0 for -0 / b); an infinite or NaN dividend, or a quotient past the float range, is a * r's (inf, NaN,
// or the overflow) instead of the correction's NaN: one class test (NaN, +-inf, +-0) picks q. Divisors near
// the ends of the exponent range, zero, infinities and NaN take the IEEE division.
DEV float rcp_f32(float b) {
  const float r = __builtin_amdgcn_rcpf(b);
  return fmaf(fmaf(-b, r, 1.0f), r, r);
}
DEV int fdiv_ok(float b) {
  const float ab = fabsf(b);
  return ab > 0x1p-125f && ab < 0x1p+125f;
}
DEV float fdiv_q(float a, float b, float r) {
  const float q = a * r;
  const float q2 = fmaf(fmaf(-b, q, a), r, q);
  return __builtin_amdgcn_classf(q2, 0x267) ? q : q2;
}
DEV float fdiv_f32(float a, float b) { return fdiv_ok(b) ? fdiv_q(a, b, rcp_f32(b)) : a / b; }
// the same quotient for a divisor shared by a row's lanes (a row's sum or deviation): its reciprocal r and
// range flag computed once, the flag wave-uniform so the IEEE fallback is a scalar branch
DEV float fdiv_row(float a, float b, float r, int ok) {
  if (!ok) return a / b;
  return fdiv_q(a, b, r);
}
// a / b for a row-uniform divisor as a times its refined reciprocal r (within 2 ulp: r within 1 ulp of 1 / b,
// one more rounding in the product); divisors near the ends of the exponent range, zero, infinities and NaN
// take the IEEE division by the same scalar branch
DEV float fdiv_rowm(float a, float b, float r, int ok) {
  if (!ok) return a / b;
  return a * r;
}
// 1 + tanh(u) in float32 as 2 / (1 + 2^(-2 u log2 e)) = 2 sigmoid(2u): no cancellation as tanh(u) nears -1,
// one exp2 and one reciprocal where tanh_f32 evaluates a polynomial and an exp2/reciprocal form and selects.
// The exponent's rounding (relative 2^-24 of |2u log2 e|) bounds the error: under 1e-6 relative for |u| < 8,
// 2e-5 at the underflow end; u = +-inf gives 2 and 0, NaN propagates.
DEV float onep_tanh_f32(float u) { return 2.0f * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-2.8853900817779268f * u)); }
// tanh(u) as 1 - 2 / (1 + 2^(2u log2 e)): one exp2 and one reciprocal, absolute error under 3e-7 everywhere but
// not relative near 0, so it serves readers that use tanh(u) in 1 +- tanh(u) and tanh(u)^2 (GELU's derivative),
// whose values carry that absolute error in float32 anyway; +-inf give +-1, NaN propagates
DEV float tanh_abs_f32(float u) { return fmaf(-2.0f, __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(2.8853900817779268f * u)), 1.0f); }
// the same with u = c x folded into one product (the tanh argument of GELU's tanh form): k = -2 c log2 e
DEV float onep_tanh_k(float x, float k) { return 2.0f * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(k * x)); }
// GELU's tanh form 0.5 x (1 + tanh(c1 (x + c2 x^3))) as x sigmoid(2 c1 x (1 + c2 x^2)) = x / (1 + 2^(x (k + k c2 x^2)))
// with k = -2 c1 log2 e: three products, one exp2 and one reciprocal. Within 2e-6 relative of the exact value for
// |x| < 8 (the exponent's rounding, relative 2^-24 of its magnitude, and the two hardware approximations); +inf
// gives inf, -inf NaN and large negative x -0, as the traced form does in float32
DEV float gelu_tanh_f32(float x, float k, float kc2) {
  const float p = fmaf(x * x, kc2, k);
  return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(x * p));
}
// dy times the derivative of that GELU, d/dx 0.5 x (1 + tanh u) with u = c1 (x + c2 x^3):
// 0.5 (1 + tanh u) + 0.5 x (1 - tanh^2 u) c1 (1 + 3 c2 x^2) = s (1 + 2 c1 x (1 - s) (1 + 3 c2 x^2)), where
// s = sigmoid(2u) = 1 / (1 + e) and 1 - s = e s, e = exp(-2u) = 2^(x (k + k c2 x^2)): no cancellation where tanh u
// nears +-1 (the traced 1 - tanh^2 loses its digits there). a = 2 c1, b = 3 c2. Within 3e-6 relative of the exact
// value for |x| < 8 (the exponent's rounding and the hardware exp2 and reciprocal). e overflowing (x below about
// -10) makes s 0 and e s NaN, which the minimum with 1 (its value's bound) replaces, so the result is 0 as the
// traced form gives; x = +-inf or NaN give NaN, as the traced form does
DEV float gelu_tanh_grad_f32(float x, float dy, float k, float kc2, float a, float b) {
  const float x2 = x * x;
  const float e = __builtin_amdgcn_exp2f(x * fmaf(x2, kc2, k));
  const float s = __builtin_amdgcn_rcpf(1.0f + e);
  const float es = fminf(e * s, 1.0f);
  return (dy * s) * fmaf((a * x) * es, fmaf(x2, b, 1.0f), 1.0f);
}
// exp(d) of a row-shifted value d = x - (a row's statistic), softmax's exponent: 2^(d log2 e) on the hardware
// exp2. The product's rounding bounds the error to 2^-24 |d log2 e| ln 2 relative: under 5.2e-6 for every d
// whose exponential is a normal float (d > -87.3); -inf gives 0, NaN propagates
DEV float exp_shifted_f32(float d) { return __builtin_amdgcn_exp2f(d * 1.4426950408889634f); }
// NaN-propagating float32 maximum and minimum (-0 below +0): gfx950's v_maximum3_f32 / v_minimum3_f32, one
// instruction for two operands or a chain of three
DEV float fmax_n(float a, float b) { return __builtin_elementwise_maximum(a, b); }
DEV double dmax_n(double a, double b) { return (a != a || b != b) ? __builtin_nan("") : fmax(a, b); }
DEV float fmin_n(float a, float b) { return __builtin_elementwise_minimum(a, b); }
DEV double dmin_n(double a, double b) { return (a != a || b != b) ? __builtin_nan("") : fmin(a, b); }
// float -> integer saturating at the result dtype's limits, NaN -> 0 (lumen/reference/mod.rs saturate). lo and
// hi are the dtype's limits as doubles (T is its compute type, which may be wider); the 64-bit maxima round to
// 2^63 / 2^64 as doubles, which do not convert back, so those return T's own maximum instead.
template <typename T> DEV T sat_cast(double x, double lo, double hi) {
  if (x != x) return T(0);
  if (x <= lo) return T(lo);
  if (x >= hi) return hi < 9.2233720368547758e18 ? T(hi) : (T(0) < T(-1) ? T(~T(0)) : T(~(T(1) << (8 * sizeof(T) - 1))));
  return T(x);
}
// float wave reductions on DPP moves, every lane of the wave active: lanes exchanged within quads (xor 1, xor 2),
// half rows and rows (mirrors), then rows 0+1 and 2+3 joined by the row broadcasts of lanes 15 and 31, so lane
// 63 holds the total, read back as a wave-uniform value. Disabled rows of a broadcast read the identity.
#define LK_DPP(v, ctrl, rows, id) \
  __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, (float)(id)), \
                                                        __builtin_bit_cast(int, v), ctrl, rows, 0xF, false))
DEV float lane63(float v) { return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63)); }
DEV float wsum(float v) {
  v += LK_DPP(v, 0xB1, 0xF, 0.0f);
  v += LK_DPP(v, 0x4E, 0xF, 0.0f);
  v += LK_DPP(v, 0x141, 0xF, 0.0f);
  v += LK_DPP(v, 0x140, 0xF, 0.0f);
  v += LK_DPP(v, 0x142, 0xA, 0.0f);
  v += LK_DPP(v, 0x143, 0xC, 0.0f);
  return lane63(v);
}
// the maximum propagates NaN (fmax_n): a NaN on any lane reaches lane 63
DEV float wmax(float v) {
  v = fmax_n(v, LK_DPP(v, 0xB1, 0xF, -INFINITY));
  v = fmax_n(v, LK_DPP(v, 0x4E, 0xF, -INFINITY));
  v = fmax_n(v, LK_DPP(v, 0x141, 0xF, -INFINITY));
  v = fmax_n(v, LK_DPP(v, 0x140, 0xF, -INFINITY));
  v = fmax_n(v, LK_DPP(v, 0x142, 0xA, -INFINITY));
  v = fmax_n(v, LK_DPP(v, 0x143, 0xC, -INFINITY));
  return lane63(v);
}
DEV double wsum(double v) { for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64); return v; }
DEV double wmax(double v) { for (int o = 32; o > 0; o >>= 1) v = dmax_n(v, __shfl_xor(v, o, 64)); return v; }
// integer wavefront sums wrap (unsigned adds, two's complement: any order gives the same bits) and maxima;
// 64-bit values cross lanes as two 32-bit halves
DEV uint64_t shfl64(uint64_t v, int o) {
  const uint32_t lo = __shfl_xor((unsigned)(v & 0xffffffffu), o, 64), hi = __shfl_xor((unsigned)(v >> 32), o, 64);
  return ((uint64_t)hi << 32) | lo;
}
DEV int32_t wsum(int32_t v) { for (int o = 32; o > 0; o >>= 1) v = (int32_t)((uint32_t)v + (uint32_t)__shfl_xor(v, o, 64)); return v; }
DEV uint32_t wsum(uint32_t v) { for (int o = 32; o > 0; o >>= 1) v += (uint32_t)__shfl_xor(v, o, 64); return v; }
DEV int64_t wsum(int64_t v) { for (int o = 32; o > 0; o >>= 1) v = (int64_t)((uint64_t)v + shfl64((uint64_t)v, o)); return v; }
DEV uint64_t wsum(uint64_t v) { for (int o = 32; o > 0; o >>= 1) v += shfl64(v, o); return v; }
DEV int32_t wmax(int32_t v) { for (int o = 32; o > 0; o >>= 1) { int32_t w = __shfl_xor(v, o, 64); v = w > v ? w : v; } return v; }
DEV uint32_t wmax(uint32_t v) { for (int o = 32; o > 0; o >>= 1) { uint32_t w = __shfl_xor(v, o, 64); v = w > v ? w : v; } return v; }
DEV int64_t wmax(int64_t v) { for (int o = 32; o > 0; o >>= 1) { int64_t w = (int64_t)shfl64((uint64_t)v, o); v = w > v ? w : v; } return v; }
DEV uint64_t wmax(uint64_t v) { for (int o = 32; o > 0; o >>= 1) { uint64_t w = shfl64(v, o); v = w > v ? w : v; } return v; }
// integer add with wraparound in the width of T (no signed overflow)
template <typename T> DEV T wrap_add(T a, T b) { return (T)((uint64_t)(int64_t)a + (uint64_t)(int64_t)b); }
template <int N> struct alignas(N * 2) u16v { uint16_t e[N]; };
template <int N> struct alignas(N * 4) f32v { float e[N]; };
template <int N> struct alignas(N * 4) u32v { uint32_t e[N]; };
template <int N> struct alignas(N * 8) u64v { uint64_t e[N]; };
"""

# Storage C type of each dtype in memory.
STORE_T = {
    "bool": "uint8_t", "uint8": "uint8_t", "uint16": "uint16_t", "uint32": "uint32_t", "uint64": "uint64_t",
    "int8": "int8_t", "int16": "int16_t", "int32": "int32_t", "int64": "int64_t",
    "float16": "uint16_t", "bfloat16": "uint16_t", "float32": "float", "float64": "double",
}
# Compute C type of each dtype.
COMP_T = {
    "bool": "int", "uint8": "uint32_t", "uint16": "uint32_t", "uint32": "uint32_t", "uint64": "uint64_t",
    "int8": "int32_t", "int16": "int32_t", "int32": "int32_t", "int64": "int64_t",
    "float16": "float", "bfloat16": "float", "float32": "float", "float64": "double",
}
VEC_T = {2: "u16v", 4: "f32v", 8: "u64v"}


def _lit(value, dtype):
    """A C literal of ``value`` rounded to ``dtype`` (in its compute type)."""
    if D.is_float(dtype):
        v = float(value)
        if dtype in ("bfloat16", "float16", "float32"):
            import numpy as np

            if dtype == "bfloat16":
                v = float(D.bf16_to_f32(D.bf16_bits(np.array([v], np.float64)))[0])
            elif dtype == "float16":
                from lumen_amd.dtypes import _round_to_odd_f32

                v = float(np.float16(_round_to_odd_f32(np.array([v]))[0]))
            else:
                v = float(np.float32(v))
            if math.isnan(v):
                return "__builtin_nanf(\"\")"
            if math.isinf(v):
                return "__builtin_inff()" if v > 0 else "(-__builtin_inff())"
            return f"{v.hex()}f" if v != 0 or math.copysign(1, v) > 0 else "(-0.0f)"
        if math.isnan(v):
            return "__builtin_nan(\"\")"
        if math.isinf(v):
            return "__builtin_inf()" if v > 0 else "(-__builtin_inf())"
        return v.hex()
    if dtype == "bool":
        return "1" if value else "0"
    return f"(({COMP_T[dtype]})({int(value)}LL))"


def _contig(shape):
    st, s = [], 1
    for n in reversed(shape):
        st.append(s)
        s *= n
    return tuple(reversed(st))


class View:
    """Where a kernel operand lives: element offset and strides from its buffer's base pointer."""

    def __init__(self, dtype, shape, offset=0, strides=None):
        self.dtype, self.shape, self.offset = dtype, tuple(shape), offset
        self.strides = tuple(strides) if strides is not None else _contig(shape)

    def contiguous(self):
        return self.strides == _contig(self.shape) or math.prod(self.shape) <= 1


def _block_offset(src, out, start):
    """The flat offset of a slice [start, start + out) of a row-major ``src`` when the slice is one contiguous
    block of it (leading dims of size 1, then one partial dim, then full dims), else None."""
    for d0 in range(len(out) + 1):
        if all(out[d] == 1 for d in range(d0)) and all(out[d] == src[d] for d in range(d0 + 1, len(out))):
            st = _contig(src)
            return sum(s * t for s, t in zip(start, st))
    return None


class Emitter:
    """Evaluates graph values of one kernel at index expressions, writing C statements."""

    # float32 division as a refined reciprocal and one quotient correction (fdiv_f32, within 1 ulp) instead of
    # the correctly rounded division sequence; the reciprocal of a row statistic is then computed once a row
    FAST_DIV = True
    # a quotient by a row statistic (layer norm's deviation, softmax's sum) as one multiply by the row's refined
    # reciprocal (within 2 ulp) instead of the corrected quotient (within 1 ulp, four more instructions)
    ROW_RECIP_MUL = True
    # 1 + tanh(u) whose tanh nothing else reads (GELU's tanh form) evaluated as 2 sigmoid(2u) (onep_tanh_f32)
    ONEP_TANH = True
    # the traced derivative of the tanh GELU times its cotangent as one closed form (gelu_tanh_grad_f32)
    GELU_GRAD = True
    # exp of a row-shifted value (softmax) as one exp2 of the scaled argument (within 5.2e-6 relative)
    # instead of exp_f32's split product (within 4 ulp)
    SHIFTED_EXP = True

    def __init__(self, graph: Graph, nodes, inputs: dict, rows=None):
        self.graph = graph
        self.prod = {n.output: n for n in nodes}
        self.inputs = inputs          # var -> (arg index, View)
        self.lines: list[str] = []
        self.memo: dict = {}
        self.count = 0
        self.rows = rows
        self.row_scalars: dict = {}   # reduction var -> C name of its per-row value
        self.flat_loads: dict = {}    # (arg, fbase) -> element names (vectorized loads)
        self.vec = 1
        self.given: dict = {}         # var -> fn(idx) -> C name: values the caller computes (a GEMM's sums)
        self.uniform: set = set()     # C names of per-row values (the same on every lane of a row's wave)
        # whether a row's values are the same on every lane of a wave (a row kernel's; not a GEMM epilogue's,
        # whose lanes hold different rows)
        self.rows_uniform = True
        self.recips: dict = {}        # uniform divisor name -> (reciprocal name, range-flag name)
        self.rounded: dict = {}       # name of a bf16-rounded float -> the name it was rounded from
        self._users = None            # readers of each value, built on first need
        # the values the kernel stores (None: unknown, so every reader in the graph counts): a value another
        # step reads is one of them, or that step computes it again from stored operands
        self.outputs = None
        self._gelu_grads: dict = {}   # var -> _gelu_tanh_grad's answer

    def tmp(self, prefix="t"):
        self.count += 1
        return f"{prefix}{self.count}"

    _ROUNDED = re.compile(r"const float (\w+) = r_bf16\((\w+)\);$")

    def emit(self, line):
        m = self._ROUNDED.match(line)
        if m:
            self.rounded[m.group(1)] = m.group(2)
        self.lines.append(line)

    def unrounded(self, name):
        """The float that ``name`` was rounded to bf16 from, when it was (storing that float as bf16 gives the
        same bits, rounding being idempotent), else ``name``."""
        return self.rounded.get(name, name)

    def quotient(self, a, b):
        """``a / b`` in float32 (within 1 ulp): a per-row divisor's reciprocal and range flag are computed once."""
        if b in self.uniform and a not in self.uniform:
            if b not in self.recips:
                r, ok = self.tmp("rcp"), self.tmp("dok")
                self.emit(f"const float {r} = rcp_f32({b});")
                self.emit(f"const int {ok} = __builtin_amdgcn_readfirstlane(fdiv_ok({b}));")
                self.recips[b] = (r, ok)
            r, ok = self.recips[b]
            return f"{'fdiv_rowm' if Emitter.ROW_RECIP_MUL else 'fdiv_row'}({a}, {b}, {r}, {ok})"
        return f"fdiv_f32({a}, {b})"

    # ---- indices
    def multi(self, idx, shape):
        """``idx`` as one expression per dimension of ``shape``."""
        kind = idx[0]
        if kind == "multi":
            return list(idx[1])
        if kind == "rc" and self.rows is not None and shape:
            # a row kernel's (row, column) index over a value whose trailing dims span the row: the leading
            # indices from the row alone (the same for the whole row, computed once) and the trailing ones from
            # the column, instead of decomposing r * C + c with 64-bit divisions for every element
            R, C = self.rows
            for k in range(len(shape), -1, -1):
                if math.prod(shape[k:]) == C and math.prod(shape[:k]) == R:
                    return self._split(idx[1], shape[:k]) + self._split(idx[2], shape[k:])
                if math.prod(shape[k:]) > C:
                    break
        f = self.flat(idx, shape)
        if not shape:
            return []
        out = []
        st = _contig(shape)
        for d, n in enumerate(shape):
            if n == 1:
                out.append("0")
            elif d == 0:
                out.append(f"(({f}) / {st[0]}LL)")
            else:
                out.append(f"((({f}) / {st[d]}LL) % {n}LL)")
        return out

    @staticmethod
    def _split(e, shape):
        """The row-major multi-index of flat index expression ``e`` over ``shape``."""
        if not shape:
            return []
        st = _contig(shape)
        out = []
        for d, n in enumerate(shape):
            if n == 1:
                out.append("0")
            elif len(shape) == 1:
                out.append(f"({e})")
            elif d == 0:
                out.append(f"(({e}) / {st[0]}LL)")
            else:
                out.append(f"((({e}) / {st[d]}LL) % {n}LL)")
        return out

    def flat(self, idx, shape):
        kind = idx[0]
        if kind == "flat":
            return idx[1]
        if kind == "rc":
            return f"({idx[1]} * {self.rows[1]}LL + {idx[2]})"
        if kind == "r":
            return idx[1]
        st = _contig(shape)
        terms = [f"({e}) * {s}LL" for e, s in zip(idx[1], st) if s and e != "0"]
        return "(" + (" + ".join(terms) if terms else "0") + ")"

    # ---- values
    def value(self, var, idx):
        ty = self.graph.types[var]
        key = (var, self._key(idx, ty.shape))
        if key in self.memo:
            return self.memo[key]
        name = self._compute(var, idx, ty)
        self.memo[key] = name
        if idx[0] == "r" and self.rows is not None and self.rows_uniform:
            self.uniform.add(name)
        return name

    def _key(self, idx, shape):
        if idx[0] in ("rc", "r", "flat"):
            return idx
        return ("multi", tuple(idx[1]))

    def load(self, var, idx, ty):
        arg, view = self.inputs[var]
        ct = COMP_T[ty.dtype]
        if idx[0] in ("flat", "rc") and view.contiguous() and view.offset % max(1, self.vec) == 0 and self.vec > 1:
            f = self.flat(idx, ty.shape)
            base, lane = self._split_vec(idx)
            if base is not None:
                names = self.flat_loads.setdefault((arg, base), [None] * self.vec)
                if names[lane] is None:
                    names[lane] = self.tmp("v")
                raw = names[lane]
                return self._widen(raw, ty.dtype)
            del f
        if idx[0] in ("flat", "rc", "r") and view.contiguous():
            addr = self.flat(idx, ty.shape)
        else:
            m = self.multi(idx, ty.shape)
            terms = [f"({e}) * {s}LL" for e, s in zip(m, view.strides) if s and e != "0"]
            addr = "(" + (" + ".join(terms) if terms else "0") + ")"
        n = self.tmp()
        self.emit(f"const {ct} {n} = {self._widen(f'in{arg}[{addr}]', ty.dtype)};")
        return n

    def _split_vec(self, idx):
        """``(base, lane)`` if ``idx`` is ``base + lane`` of the current vector, else (None, None)."""
        if idx[0] == "flat" and isinstance(idx, tuple) and len(idx) == 4:
            return idx[2], idx[3]
        if idx[0] == "rc" and len(idx) == 5:
            return f"({idx[1]} * {self.rows[1]}LL + {idx[3]})", idx[4]
        return None, None

    @staticmethod
    def _widen(raw, dtype):
        if dtype == "bfloat16":
            return f"lb_bf16({raw})"
        if dtype == "float16":
            return f"lb_f16({raw})"
        return f"(({COMP_T[dtype]})({raw}))"

    def round(self, expr, dtype):
        if dtype == "bfloat16":
            return f"r_bf16({expr})"
        if dtype == "float16":
            return f"r_f16({expr})"
        if dtype == "float32":
            return f"((float)({expr}))"
        if dtype == "float64":
            return f"((double)({expr}))"
        if dtype == "bool":
            return f"(({expr}) != 0)"
        return f"(({COMP_T[dtype]})({STORE_T[dtype]})({expr}))"

    def _const(self, var):
        """The fill value of ``var`` when it is a scalar fill, possibly broadcast or reshaped, else None."""
        n = self.prod.get(var)
        while n is not None and n.prim in ("broadcast_in_dim", "reshape"):
            n = self.prod.get(n.inputs[0])
        return n.params["fill_value"] if n is not None and n.prim == "full" else None

    def _onep_tanh_arg(self, n):
        """For ``n`` = 1 + tanh(u) (either order) where the kernel computes the tanh, does not store it, and
        every reader of it (in the kernel when its stored values are known, else in the graph) is such a sum: u,
        else None."""
        for k in (0, 1):
            t = self.prod.get(n.inputs[k])
            if t is None or t.prim != "tanh" or self._const(n.inputs[1 - k]) != 1.0:
                continue
            if t.inputs[0] in self.given or self.graph.types[t.inputs[0]].dtype != "float32":
                continue
            readers = self._readers(t.output)
            stored = self.graph.outputs if self.outputs is None else self.outputs
            if t.output in stored or not all(
                    r.prim == "add" and any(r.inputs[j] == t.output and self._const(r.inputs[1 - j]) == 1.0
                                            for j in (0, 1)) for r in readers):
                continue
            return t.inputs[0]
        return None

    def _readers(self, var):
        if self._users is None:
            if self.outputs is None:
                self._users = self.graph.users()
            else:  # readers inside the kernel
                self._users = {}
                for m in self.prod.values():
                    for v in m.inputs:
                        self._users.setdefault(v, []).append(m)
        return self._users.get(var, [])

    def _tanh_abs_ok(self, t):
        """Whether every reader of tanh node ``t`` takes 1 + t, 1 - t or t * t (so an absolute error bound
        serves), and the kernel does not store it."""
        stored = self.graph.outputs if self.outputs is None else self.outputs
        if t.output in stored:
            return False
        v = t.output
        for r in self._readers(v):
            if r.prim == "mul" and r.inputs == (v, v):
                continue
            if r.prim == "add" and any(r.inputs[j] == v and self._const(r.inputs[1 - j]) == 1.0 for j in (0, 1)):
                continue
            if r.prim == "sub" and r.inputs[1] == v and self._const(r.inputs[0]) == 1.0:
                continue
            return False
        return bool(self._readers(v))

    def _mul_const(self, var):
        """(c, y) when ``var`` is the product of a finite float scalar fill c and y (either order), else None."""
        m = self.prod.get(var)
        if m is None or m.prim != "mul":
            return None
        for j in (0, 1):
            c = self._const(m.inputs[j])
            if isinstance(c, float) and c == c and abs(c) != float("inf"):
                return c, m.inputs[1 - j]
        return None

    def _times(self, var, x):
        """The operand multiplied by ``x`` when ``var`` is a product with x (either order), else None."""
        m = self.prod.get(var)
        if m is None or m.prim != "mul" or x not in m.inputs:
            return None
        return m.inputs[1] if m.inputs[0] == x else m.inputs[0]

    def _gelu_tanh(self, n):
        """(x, c1, c2) when ``n`` is the traced tanh GELU (0.5 x) (1 + tanh(c1 (x + ((c2 x) x) x))) in float32
        and its tanh qualifies for onep_tanh (nothing else reads it), else None."""
        for j in (0, 1):
            half = self._mul_const(n.inputs[j])
            if half is None or half[0] != 0.5:
                continue
            x = half[1]
            b = self.prod.get(n.inputs[1 - j])
            if b is None or b.prim != "add" or self.graph.types[x].dtype != "float32":
                continue
            u = self._onep_tanh_arg(b)
            cu = self._mul_const(u) if u is not None else None
            if cu is None:
                continue
            c1, s = cu
            sn = self.prod.get(s)
            if sn is None or sn.prim != "add" or x not in sn.inputs:
                continue
            cube = sn.inputs[1] if sn.inputs[0] == x else sn.inputs[0]
            sq = self._times(cube, x)
            lin = self._times(sq, x) if sq is not None else None
            c2 = self._mul_const(lin) if lin is not None else None
            if c2 is None or c2[1] != x:
                continue
            return x, c1, c2[0]
        return None

    # float32 operations a GELU derivative's expression is made of
    _GRAD_OPS = ("add", "sub", "mul", "neg", "tanh")
    # points (x, dy) at which a candidate expression is compared with the derivative in float64
    _GRAD_POINTS = ((-3.1, 0.7), (-1.3, -1.9), (-0.45, 1.1), (0.2, -0.35), (0.8, 2.3), (2.6, -1.2))

    def _gelu_tanh_grad(self, n):
        """(x, dy, c1, c2) when ``n`` is, as a float32 expression of two values x and dy and scalar constants,
        dy times the derivative of the tanh GELU 0.5 x (1 + tanh(c1 (x + c2 x^3))), else None. The expression
        (add, sub, mul, neg and one tanh) is evaluated in float64: the tanh's argument at x = 1 and 2 gives c1
        and c2, and the argument and the whole expression are then compared with their closed forms at fixed
        points, so any arrangement of the terms matches (autograd's is a sum of eight products)."""
        if n.output in self._gelu_grads:
            return self._gelu_grads[n.output]
        self._gelu_grads[n.output] = None
        shape = self.graph.types[n.output].shape
        nodes, leaves, consts, tanhs = {}, set(), {}, []
        stack = [n.output]
        while stack:
            v = stack.pop()
            if v in nodes or v in leaves or v in consts:
                continue
            c = self._const(v)
            if c is not None:
                if not isinstance(c, float):
                    return None
                consts[v] = c
                continue
            m = self.prod.get(v)
            if v in self.given or v in self.inputs or m is None or m.prim not in self._GRAD_OPS:
                if self.graph.types[v].shape != shape or self.graph.types[v].dtype != "float32":
                    return None
                leaves.add(v)
                continue
            if self.graph.types[v].dtype != "float32" or len(nodes) >= 48:
                return None
            nodes[v] = m
            if m.prim == "tanh":
                tanhs.append(m)
            stack.extend(m.inputs)
        if len(tanhs) != 1 or len(leaves) != 2:
            return None
        arg = tanhs[0].inputs[0]

        def ev(v, env):
            if v in env:
                return env[v]
            if v in consts:
                return consts[v]
            m = nodes[v]
            a = [ev(w, env) for w in m.inputs]
            r = {"add": lambda: a[0] + a[1], "sub": lambda: a[0] - a[1], "mul": lambda: a[0] * a[1],
                 "neg": lambda: -a[0], "tanh": lambda: math.tanh(a[0])}[m.prim]()
            env[v] = r
            return r

        def close(a, b):
            return abs(a - b) <= 1e-12 * max(1.0, abs(b))

        for x, dy in (tuple(leaves), tuple(leaves)[::-1]):
            try:
                a1, a2 = ev(arg, {x: 1.0, dy: 0.37}), ev(arg, {x: 2.0, dy: 0.37})
                c1c2 = (a2 - 2.0 * a1) / 6.0  # a(x) = c1 x + c1 c2 x^3
                c1 = a1 - c1c2
                if not (c1 != 0.0 and math.isfinite(c1) and math.isfinite(c1c2)):
                    continue
                c2 = c1c2 / c1
                if not all(close(ev(arg, {x: xv, dy: dv}), c1 * (xv + c2 * xv ** 3)) for xv, dv in self._GRAD_POINTS):
                    continue
                ok = True
                for xv, dv in self._GRAD_POINTS:
                    t = math.tanh(c1 * (xv + c2 * xv ** 3))
                    want = dv * (0.5 * (1 + t) + 0.5 * xv * (1 - t * t) * c1 * (1 + 3 * c2 * xv * xv))
                    ok = ok and close(ev(n.output, {x: xv, dy: dv}), want)
            except (OverflowError, ZeroDivisionError):
                continue
            if ok:
                self._gelu_grads[n.output] = (x, dy, c1, c2)
                return x, dy, c1, c2
        return None

    def _row_shifted(self, var):
        """Whether ``var`` is x - s with s a per-row value of this row kernel (a softmax's shifted logits)."""
        m = self.prod.get(var)
        if self.rows is None or m is None or m.prim != "sub":
            return False
        s = self.prod.get(m.inputs[1])
        while s is not None and s.prim in ("broadcast_in_dim", "reshape"):
            if s.inputs[0] in self.row_scalars:
                return True
            s = self.prod.get(s.inputs[0])
        return m.inputs[1] in self.row_scalars

    def _compute(self, var, idx, ty):
        if var in self.given:
            return self.given[var](idx)
        if var in self.inputs:
            return self.load(var, idx, ty)
        n = self.prod.get(var)
        if n is None:
            raise Unfusable(var, f"value %{var} is neither computed in the kernel nor an input")
        p = n.prim
        dt = ty.dtype
        ct = COMP_T[dt]
        out = self.tmp()
        ins = [self.graph.types[v] for v in n.inputs]

        def same(k=0):
            return self.value(n.inputs[k], idx)

        if p == "mul" and dt == "float32" and Emitter.ONEP_TANH:
            g = self._gelu_tanh(n)
            if g is not None:
                x, c1, c2 = g
                k = -2.0 * c1 * 1.4426950408889634
                self.emit(f"const float {out} = gelu_tanh_f32({self.value(x, idx)}, {_f32_hex(k)}, "
                          f"{_f32_hex(k * c2)});")
                return out
        if p in ("add", "sub", "mul") and dt == "float32" and Emitter.GELU_GRAD:
            g = self._gelu_tanh_grad(n)
            if g is not None:
                x, dy, c1, c2 = g
                k = -2.0 * c1 * 1.4426950408889634
                self.emit(f"const float {out} = gelu_tanh_grad_f32({self.value(x, idx)}, {self.value(dy, idx)}, "
                          f"{_f32_hex(k)}, {_f32_hex(k * c2)}, {_f32_hex(2.0 * c1)}, {_f32_hex(3.0 * c2)});")
                return out
        if p == "add" and dt == "float32" and Emitter.ONEP_TANH:
            u = self._onep_tanh_arg(n)
            if u is not None:
                cu = self._mul_const(u)
                if cu is not None:
                    k = -2.0 * cu[0] * 1.4426950408889634
                    self.emit(f"const float {out} = onep_tanh_k({self.value(cu[1], idx)}, {_f32_hex(k)});")
                else:
                    self.emit(f"const float {out} = onep_tanh_f32({self.value(u, idx)});")
                return out
        if p in ("add", "sub", "mul", "div", "max", "eq", "lt"):
            a, b = same(0), same(1)
            src = ins[0].dtype
            if p in ("eq", "lt"):
                op = "==" if p == "eq" else "<"
                self.emit(f"const int {out} = ({a} {op} {b});")
            elif p == "max":
                if D.is_float(src):
                    fn = "dmax_n" if src == "float64" else "fmax_n"
                    self.emit(f"const {ct} {out} = {fn}({a}, {b});")
                else:
                    self.emit(f"const {ct} {out} = ({a} > {b} ? {a} : {b});")
            else:
                op = {"add": "+", "sub": "-", "mul": "*", "div": "/"}[p]
                if D.is_float(dt) and p == "div" and ct == "float" and Emitter.FAST_DIV:
                    self.emit(f"const {ct} {out} = {self.round(self.quotient(a, b), dt)};")
                elif D.is_float(dt):
                    self.emit(f"const {ct} {out} = {self.round(f'{a} {op} {b}', dt)};")
                elif p == "div":
                    # truncating; x / 0 = -1 and int64 min / -1 wraps to itself (the reference divides in i128
                    # and wraps); narrower types divide exactly in 64 bits
                    if dt == "int64":
                        q = f"({b} == -1 ? (int64_t)(0ULL - (uint64_t){a}) : {a} / {b})"
                    elif dt == "uint64":
                        q = f"({a} / {b})"
                    else:
                        q = self.round(f"(int64_t){a} / (int64_t){b}", dt)
                    self.emit(f"const {ct} {out} = ({b} == 0 ? ({ct})-1 : {q});")
                else:
                    # two's-complement wraparound: the operation in 64-bit unsigned arithmetic, then narrowed
                    expr = f"(uint64_t)(int64_t){a} {op} (uint64_t)(int64_t){b}"
                    self.emit(f"const {ct} {out} = {self.round(expr, dt)};")
            return out
        if p in ("shift_left", "shift_right_logical", "shift_right_arithmetic"):
            # amounts outside [0, width) saturate: 0, or -1 for an arithmetic shift of a negative value
            # (reference mod.rs:571-578); the value's bits are taken in its own width
            a, b = same(0), same(1)
            w = D.bits(dt)
            mask = "0xffffffffffffffffULL" if w == 64 else f"0x{(1 << w) - 1:x}ULL"
            ubits = f"((uint64_t)(int64_t){a} & {mask})"
            sbits = f"(int64_t)({'(int64_t)' + ubits if w == 64 else f'(int64_t)({ubits} << {64 - w}) >> {64 - w}'})"
            amt = f"(int64_t){b}"
            inside = f"({amt} >= 0 && {amt} < {w})"
            if p == "shift_left":
                val, outside = f"({ubits} << {amt})", "0"
            elif p == "shift_right_logical":
                val, outside = f"({ubits} >> {amt})", "0"
            else:
                val, outside = f"(uint64_t)({sbits} >> {amt})", f"({sbits} < 0 ? ~0ULL : 0ULL)"
            self.emit(f"const {ct} {out} = {self.round(f'({inside} ? {val} : {outside})', dt)};")
            return out
        if p in ("population_count", "clz"):
            a = same()
            w = D.bits(dt)
            mask = "0xffffffffffffffffULL" if w == 64 else f"0x{(1 << w) - 1:x}ULL"
            ubits = f"((uint64_t)(int64_t){a} & {mask})"
            if p == "population_count":
                expr = f"__popcll({ubits})"
            else:
                expr = f"({ubits} == 0 ? {w} : __clzll({ubits}) - {64 - w})"
            self.emit(f"const {ct} {out} = ({ct})({expr});")
            return out
        if p == "neg":
            a = same()
            self.emit(f"const {ct} {out} = {self.round(f'-{a}', dt) if not D.is_float(dt) else f'-{a}'};")
            return out
        if p in ("exp", "log", "sqrt", "tanh", "logistic", "sin", "cos", "tan", "asin", "acos", "atan", "sinh",
                 "cosh", "asinh", "acosh", "atanh", "floor", "ceil", "round", "log1p", "expm1", "exp2", "log2",
                 "rsqrt", "cbrt", "abs"):
            a = same()
            if not D.is_float(dt):
                if p == "abs":
                    self.emit(f"const {ct} {out} = {self.round(f'({a} < 0 ? -(int64_t){a} : (int64_t){a})', dt)};")
                    return out
                raise Unfusable(var, f"{p} of {dt}")
            f32 = dt != "float64"
            fn = {
                "exp": "exp", "log": "log", "sqrt": "sqrt", "tanh": "tanh", "sin": "sin", "cos": "cos", "tan": "tan",
                "asin": "asin", "acos": "acos", "atan": "atan", "sinh": "sinh", "cosh": "cosh", "asinh": "asinh",
                "acosh": "acosh", "atanh": "atanh", "floor": "floor", "ceil": "ceil", "round": "rint",
                "log1p": "log1p", "expm1": "expm1", "exp2": "exp2", "log2": "log2", "cbrt": "cbrt", "abs": "fabs",
            }.get(p)
            s = "f" if f32 else ""
            one = "1.0f" if f32 else "1.0"
            if p == "tanh" and f32 and Emitter.ONEP_TANH and dt == "float32" and self._tanh_abs_ok(n):
                expr = f"tanh_abs_f32({a})"
            elif p == "tanh" and f32:
                expr = f"tanh_f32({a})"
            elif p == "exp" and f32 and Emitter.SHIFTED_EXP and self._row_shifted(n.inputs[0]):
                expr = f"exp_shifted_f32({a})"
            elif p == "exp" and f32:
                expr = f"exp_f32({a})"
            elif p == "logistic":
                expr = f"{one} / ({one} + {'exp_f32' if f32 else 'exp'}(-{a}))"
            elif p == "rsqrt":
                expr = f"{one} / sqrt{s}({a})"
            else:
                expr = f"{fn}{s}({a})"
            self.emit(f"const {ct} {out} = {self.round(expr, dt)};")
            return out
        if p == "sign":
            a = same()
            if D.is_float(dt):
                self.emit(f"const {ct} {out} = ({a} == 0 || {a} != {a}) ? {a} : ({a} > 0 ? ({ct})1 : ({ct})-1);")
            else:
                self.emit(f"const {ct} {out} = ({a} > 0) - ({a} < 0);")
            return out
        if p == "is_finite":
            a = same()
            self.emit(f"const int {out} = isfinite({a}) ? 1 : 0;")
            return out
        if p == "not":
            a = same()
            self.emit(f"const {ct} {out} = {('!' + a) if dt == 'bool' else self.round('~' + a, dt)};")
            return out
        if p in ("min", "pow", "rem", "and", "or", "xor"):
            a, b = same(0), same(1)
            if p == "min":
                if D.is_float(dt):
                    self.emit(f"const {ct} {out} = {'dmin_n' if dt == 'float64' else 'fmin_n'}({a}, {b});")
                else:
                    self.emit(f"const {ct} {out} = ({a} < {b} ? {a} : {b});")
            elif p == "pow":
                s = "" if dt == "float64" else "f"
                self.emit(f"const {ct} {out} = {self.round(f'pow{s}({a}, ({ct}){b})', dt)};")
            elif p == "rem":
                if D.is_float(dt):
                    s = "" if dt == "float64" else "f"
                    self.emit(f"const {ct} {out} = {self.round(f'fmod{s}({a}, {b})', dt)};")
                else:
                    # x % 0 = x; int64 min % -1 = 0; narrower types in exact 64-bit arithmetic
                    if dt == "int64":
                        r = f"({b} == -1 ? (int64_t)0 : {a} % {b})"
                    elif dt == "uint64":
                        r = f"({a} % {b})"
                    else:
                        r = f"({ct})((int64_t){a} % (int64_t){b})"
                    self.emit(f"const {ct} {out} = ({b} == 0 ? {a} : {r});")
            else:
                op = {"and": "&", "or": "|", "xor": "^"}[p]
                self.emit(f"const {ct} {out} = {self.round(f'{a} {op} {b}', dt)};")
            return out
        if p == "cast":
            a = same()
            src = ins[0].dtype
            if D.is_float(dt) and D.is_float(src):
                expr = self.round(a, dt) if dt != "float64" else f"(double){a}"
                if src == "float64" and dt in ("bfloat16", "float16"):
                    expr = self.round(f"ro_f32({a})", dt)
            elif D.is_float(dt):
                expr = self.round(f"(float)({a})", dt) if dt != "float64" else f"(double)({a})"
            elif dt == "bool":
                expr = f"(({a}) != 0)"
            elif D.is_float(src):
                info = _int_range(dt)
                expr = f"sat_cast<{COMP_T[dt]}>((double)({a}), {info[0]!r}, {info[1]!r})"
            else:
                expr = self.round(a, dt)
            self.emit(f"const {ct} {out} = {expr};")
            return out
        if p == "select":
            c = same(0)
            a, b = same(1), same(2)
            self.emit(f"const {ct} {out} = ({c}) ? {a} : {b};")
            return out
        if p == "full":
            return _lit(n.params["fill_value"], dt)
        if p == "iota":
            m = self.multi(idx, ty.shape)
            self.emit(f"const {ct} {out} = ({ct})({m[n.params['dimension']]});")
            return out
        if p in ("host_wait", "device_wait"):
            return same()
        if p == "reshape":
            src = ins[0]
            if idx[0] in ("flat", "rc") or (idx[0] == "r" and src.numel() == self.rows[0]):
                return self.value(n.inputs[0], idx)
            return self.value(n.inputs[0], ("flat", self.flat(idx, ty.shape)))
        if p == "broadcast_in_dim":
            src = ins[0]
            dims = n.params["broadcast_dimensions"]
            if idx[0] in ("rc",) and self._row_broadcast(src, ty, dims):
                return self.value(n.inputs[0], ("r", idx[1]))
            lead = len(ty.shape) - len(src.shape)
            if src.shape and tuple(dims) == tuple(range(lead, len(ty.shape))) and tuple(src.shape) == tuple(ty.shape[lead:]):
                # only leading axes are added: the operand's flat index is the trailing part of the output's, and
                # a vector of consecutive output elements reads consecutive operand elements
                sn = math.prod(src.shape)
                if idx[0] == "rc" and self.rows and sn == self.rows[1]:
                    if len(idx) == 5:
                        return self.value(n.inputs[0], ("flat", f"({idx[3]} + {idx[4]})", idx[3], idx[4]))
                    return self.value(n.inputs[0], ("flat", idx[2]))
                if idx[0] == "flat" and len(idx) == 4 and sn % max(1, self.vec) == 0:
                    sb = f"(({idx[2]}) % {sn}LL)"
                    return self.value(n.inputs[0], ("flat", f"({sb} + {idx[3]})", sb, idx[3]))
            m = self.multi(idx, ty.shape)
            sm = [("0" if src.shape[i] == 1 else m[d]) for i, d in enumerate(dims)]
            return self.value(n.inputs[0], ("multi", tuple(sm)))
        if p == "transpose":
            m = self.multi(idx, ty.shape)
            perm = n.params["permutation"]
            sm = [None] * len(perm)
            for i, d in enumerate(perm):
                sm[d] = m[i]
            return self.value(n.inputs[0], ("multi", tuple(sm)))
        if p == "slice":
            st = n.params["start_indices"]
            off = _block_offset(ins[0].shape, ty.shape, st)
            if off is not None and idx[0] == "flat":
                # one contiguous block of the operand: its flat index is the slice's plus the block's offset
                if len(idx) == 4 and off % max(1, self.vec) == 0:
                    nb = f"({idx[2]} + {off}LL)"
                    return self.value(n.inputs[0], ("flat", f"({nb} + {idx[3]})", nb, idx[3]))
                return self.value(n.inputs[0], ("flat", f"({idx[1]} + {off}LL)"))
            m = self.multi(idx, ty.shape)
            return self.value(n.inputs[0], ("multi", tuple(f"({e} + {s}LL)" if s else e for e, s in zip(m, st))))
        if p == "swap_pairs":
            m = self.multi(idx, ty.shape)
            m[-1] = f"(({m[-1]}) ^ 1LL)"
            return self.value(n.inputs[0], ("multi", tuple(m)))
        if p == "concatenate":
            d = n.params["dimension"]
            m = self.multi(idx, ty.shape)
            self.emit(f"{ct} {out};")
            start = 0
            for k, v in enumerate(n.inputs):
                size = ins[k].shape[d]
                cond = f"if (({m[d]}) < {start + size}LL)" if k < len(n.inputs) - 1 else ""
                self.emit(("else " if k else "") + cond + " {")
                saved = self.memo
                self.memo = dict(saved)
                sm = list(m)
                sm[d] = f"(({m[d]}) - {start}LL)" if start else m[d]
                val = self.value(v, ("multi", tuple(sm)))
                self.memo = saved
                self.emit(f"  {out} = {val};")
                self.emit("}")
                start += size
            return out
        if p == "gather":
            axis = n.params["axis"]
            x, ix = ins
            m = self.multi(idx, ty.shape)
            r = len(ix.shape)
            iv = self.value(n.inputs[1], ("multi", tuple(m[axis : axis + r])))
            k = self.tmp()
            hi = max(x.shape[axis] - 1, 0)
            self.emit(f"const int64_t {k} = min(max((int64_t){iv}, 0LL), {hi}LL);")
            sm = m[:axis] + [k] + m[axis + r :]
            return self.value(n.inputs[0], ("multi", tuple(sm)))
        if p == "take_along_axis":
            axis = n.params["axis"]
            x = ins[0]
            m = self.multi(idx, ty.shape)
            iv = self.value(n.inputs[1], ("multi", tuple(m)))
            k = self.tmp()
            self.emit(f"const int64_t {k} = min(max((int64_t){iv}, 0LL), {max(x.shape[axis] - 1, 0)}LL);")
            sm = list(m)
            sm[axis] = k
            return self.value(n.inputs[0], ("multi", tuple(sm)))
        if p == "dynamic_slice":
            x = ins[0]
            m = self.multi(idx, ty.shape)
            sm = []
            for d in range(len(x.shape)):
                s = self.value(n.inputs[1 + d], ("multi", ()))
                hi = x.shape[d] - ty.shape[d]
                k = self.tmp()
                self.emit(f"const int64_t {k} = min(max((int64_t){s}, 0LL), {hi}LL);")
                sm.append(f"({m[d]} + {k})")
            return self.value(n.inputs[0], ("multi", tuple(sm)))
        if p in ("reduce_sum", "reduce_max"):
            if var in self.row_scalars:
                # a row statistic is held for the current row only: reading it at any other index (a transposed
                # broadcast of it, say) would silently take this row's value
                if idx[0] != "r":
                    raise Unfusable(var, f"{p} %{var} read at another row's index ({idx[0]})")
                return self.row_scalars[var]
            raise Unfusable(var, f"{p} %{var} read outside its row")
        raise Unfusable(var, f"{p} has no loop-kernel lowering")

    def _row_broadcast(self, src, out, dims):
        """Whether broadcasting ``src`` repeats each row value over the row's elements of this kernel's row
        space."""
        from lumen_amd.compiler.fusion import row_broadcast

        return self.rows is not None and row_broadcast(src, out, dims, self.rows)


def _f32_hex(v):
    """``v`` rounded to float32, as an exact C hex-float literal."""
    import numpy as np

    return f"{float(np.float32(v)).hex()}f"


def _red_identity(prim, dt):
    """The C literal a reduction of ``dt`` starts from: 0 for sums, -inf or the integer minimum for maxima."""
    if prim == "reduce_sum":
        return "0"
    if D.is_float(dt):
        return "-INFINITY"
    if dt == "bool":
        return "0"
    lo = int(_int_range(dt)[0])
    return f"({COMP_T[dt]})({lo + 1}LL - 1LL)" if lo else "0"


def _red_update(em, prim, dt, acc, val):
    """The expression folding ``val`` into the accumulator ``acc`` of a reduction of ``dt``: rounded float
    sums, wrapping integer sums, NaN-propagating float maxima, integer maxima."""
    ct = COMP_T[dt]
    if prim == "reduce_sum":
        if D.is_float(dt):
            return em.round(f"{acc} + {val}", dt)
        return em.round(f"wrap_add<{ct}>({acc}, ({ct})({val}))", dt)
    if D.is_float(dt):
        return f"{'dmax_n' if ct == 'double' else 'fmax_n'}({acc}, {val})"
    return f"(({ct})({val}) > {acc} ? ({ct})({val}) : {acc})"


def _int_range(dt):
    import numpy as np

    if dt == "bool":
        return (0.0, 1.0)
    info = np.iinfo(D.storage(dt))
    return (float(info.min), float(info.max))


def _store(expr_name, dtype):
    if dtype == "bfloat16":
        return f"sb_bf16({expr_name})"
    if dtype == "float16":
        return f"sb_f16({expr_name})"
    return f"({STORE_T[dtype]})({expr_name})"


def _restrict(v, aliased):
    """The pointer qualifier of value ``v``'s kernel parameter: ``__restrict__`` unless another parameter may
    address the same memory."""
    return "" if v in aliased else " __restrict__"


def _vec_width(numel, elem_bytes):
    for v in (8, 4, 2):
        if numel % v == 0 and v * elem_bytes <= 16 and v * elem_bytes in (4, 8, 16) or (v * elem_bytes == 2 and False):
            return v
    return 1


class LoopKernel:
    """A fused loop kernel of a plan step: its source, name and launch shape."""

    # row kernels: at most this many threads a row (one workgroup a row). A 32000-wide float32 row at 1024
    # threads needs 72 VGPRs a lane, so one row fits a CU and its load, reductions and stores run one after
    # another; at 512 threads two rows share a CU and overlap (0.51 -> 0.37 ms for the [8192, 32000]
    # cross-entropy row on MI355X)
    ROW_MAX_THREADS = 512
    ROW_WAVE_CHUNKS = 64  # rows of at most this many vector chunks run one wavefront a row (4 rows a workgroup)
    ROW_CHUNKS_PER_THREAD = 2
    # sums over leading axes: rows a workgroup sums before its atomic adds, and loads a thread keeps in flight
    LEAD_CHUNK = 128
    LEAD_UNROLL = 8

    def __init__(self, graph, step, name, views: dict, out_views: dict, aliased=frozenset()):
        self.graph, self.step, self.name = graph, step, name
        # values whose memory another argument of the kernel shares (an output written over the input it
        # replaces, element for element): their pointers are not declared __restrict__
        self.aliased = aliased
        self.far = frozenset()  # outputs no kernel reads soon: stored nontemporal
        self.views, self.out_views = views, out_views
        self.args = []  # ("in"|"out", var)
        self.extra_fill = []

    def source(self):
        st = self.step
        if st.kind == "scatter_add":
            return self._scatter()
        if st.kind == "row":
            return self._row()
        if st.kind == "reduce":
            return self._reduce()
        return self._loop()

    def _params(self):
        ps = []
        self.args = []
        for k, v in enumerate(self.step.inputs):
            ps.append(f"const {STORE_T[self.graph.types[v].dtype]}*{_restrict(v, self.aliased)} in{k}")
            self.args.append(("in", v))
        for k, v in enumerate(self.step.outputs):
            ps.append(f"{STORE_T[self.graph.types[v].dtype]}*{_restrict(v, self.aliased)} out{k}")
            self.args.append(("out", v))
        return ", ".join(ps)

    def _emitter(self, rows=None):
        ins = {v: (k, self.views[v]) for k, v in enumerate(self.step.inputs)}
        em = Emitter(self.graph, self.step.nodes, ins, rows)
        em.outputs = set(self.step.outputs)
        return em

    # ---- elementwise
    def _loop(self):
        g, st = self.graph, self.step
        root = st.outputs[0]
        shape = g.types[root].shape
        numel = g.types[root].numel()
        for v in st.outputs:
            if g.types[v].numel() != numel:
                raise Unfusable(v, "loop kernel outputs of different sizes")
        esz = max(D.size_of(g.types[v].dtype) for v in st.outputs)
        esz_min = min(D.size_of(g.types[v].dtype) for v in st.outputs)
        V = 1
        for cand in (8, 4, 2):
            if numel % cand == 0 and cand * esz <= 16 and cand * esz_min >= 4:
                V = cand
                break
        em = self._emitter()
        em.vec = V
        per_v = []
        for lane in range(V):
            idx = ("flat", f"(base + {lane})", "base", lane) if V > 1 else ("flat", "base")
            names = [em.value(v, idx) for v in st.outputs]
            per_v.append(names)
        body = em.lines
        pro = self._vec_prologue(em, V)
        stores = []
        for k, v in enumerate(st.outputs):
            dt = g.types[v].dtype
            if V > 1 and self.out_views[v].contiguous():
                stores.append(self._vec_store(f"out{k}", "base", [per_v[l][k] for l in range(V)], dt, V, em,
                                              nt=v in self.far))
            else:
                view = self.out_views[v]
                for lane in range(V):
                    addr = self._out_addr(view, g.types[v].shape, f"(base + {lane})")
                    stores.append(f"out{k}[{addr}] = {_store(per_v[lane][k], dt)};")
        threads = 256
        blocks = max(1, min(-(-numel // (threads * V)), 8192))
        self.grid, self.block, self.lds = (blocks, 1, 1), (threads, 1, 1), 0
        src = [
            f'extern "C" __global__ __launch_bounds__({threads}) void {self.name}({self._params()}) {{',
            f"  for (int64_t base = ((int64_t)blockIdx.x * {threads} + threadIdx.x) * {V}; base < {numel}LL; "
            f"base += (int64_t)gridDim.x * {threads * V}) {{",
        ]
        src += ["    " + l for l in pro + body + stores]
        src += ["  }", "}"]
        del shape
        return "\n".join(src)

    def _out_addr(self, view, shape, flat):
        if view.contiguous():
            return flat
        st = _contig(shape)
        terms = []
        for d, n in enumerate(shape):
            if n == 1 or view.strides[d] == 0:
                continue
            e = f"(({flat}) / {st[d]}LL)" if d == 0 else f"((({flat}) / {st[d]}LL) % {n}LL)"
            terms.append(f"{e} * {view.strides[d]}LL")
        return "(" + (" + ".join(terms) if terms else "0") + ")"

    def _vec_prologue(self, em, V, inputs=None):
        """Vector loads of the inputs (``inputs``, by default the step's, in argument order) that ``em`` read
        at flat ``base + lane`` indices."""
        inputs = self.step.inputs if inputs is None else inputs
        lines = []
        for (arg, base), names in em.flat_loads.items():
            dt = self.graph.types[inputs[arg]].dtype
            esz = D.size_of(dt)
            vt = {2: "u16v", 4: "u32v", 8: "u64v"}.get(esz)
            if vt is None or V * esz not in (4, 8, 16) or esz == 1:
                for lane, nm in enumerate(names):
                    if nm is not None:
                        lines.append(f"const {STORE_T[dt]} {nm} = in{arg}[{base} + {lane}];")
                continue
            tmp = em.tmp("V")
            lines.append(f"const {vt}<{V}> {tmp} = ld_nt(reinterpret_cast<const {vt}<{V}>*>(in{arg} + {base}));")
            ct = "uint16_t" if esz == 2 else ("uint32_t" if esz == 4 else "uint64_t")
            for lane, nm in enumerate(names):
                if nm is not None:
                    lines.append(f"const {STORE_T[dt]} {nm} = __builtin_bit_cast({STORE_T[dt]}, ({ct}){tmp}.e[{lane}]);")
        return lines

    def _vec_store(self, ptr, base, names, dt, V, em=None, nt=False):
        esz = D.size_of(dt)
        if em is not None and dt == "bfloat16":
            names = [em.unrounded(n) for n in names]
        vt = {2: "u16v", 4: "u32v", 8: "u64v"}.get(esz)
        if vt is None or V * esz not in (4, 8, 16):
            return " ".join(f"{ptr}[{base} + {l}] = {_store(n, dt)};" for l, n in enumerate(names))
        t = f"S{abs(hash((ptr, base))) % 100000}"
        if dt == "bfloat16" and V % 2 == 0:
            # pairs converted together, stored as V / 2 words
            parts = [f"{{ u32v<{V // 2}> {t};"]
            for l in range(0, V, 2):
                parts.append(f"{t}.e[{l // 2}] = sb2_bf16({names[l]}, {names[l + 1]});")
            dst = f"reinterpret_cast<u32v<{V // 2}>*>({ptr} + {base})"
            parts.append(f"st_nt({dst}, {t}); }}" if nt else f"*{dst} = {t}; }}")
            return " ".join(parts)
        ct = "uint16_t" if esz == 2 else ("uint32_t" if esz == 4 else "uint64_t")
        parts = [f"{{ {vt}<{V}> {t};"]
        for l, n in enumerate(names):
            parts.append(f"{t}.e[{l}] = __builtin_bit_cast({ct}, ({STORE_T[dt]}){_store(n, dt)});")
        dst = f"reinterpret_cast<{vt}<{V}>*>({ptr} + {base})"
        parts.append(f"st_nt({dst}, {t}); }}" if nt else f"*{dst} = {t}; }}")
        return " ".join(parts)

    # ---- row kernels
    def _row(self):
        g, st = self.graph, self.step
        R, C = st.rows
        reds = [n for n in st.nodes if n.prim in ("reduce_sum", "reduce_max")]
        outs_elem = [v for v in st.outputs if g.types[v].numel() == R * C and R * C != R]
        outs_row = [v for v in st.outputs if v not in outs_elem]
        # the vector width follows the operands read or written along the columns; per-row values (a row's
        # target class, its statistics) are loaded once a row and do not narrow it
        per_row = {R, 1} if C > 1 else set()
        dts = [g.types[v].dtype for v in outs_elem] + \
              [g.types[v].dtype for v in st.inputs if g.types[v].numel() not in per_row]
        esz = max([D.size_of(d) for d in dts] + [2])
        V = 1
        for cand in (8, 4, 2):
            if C % cand == 0 and cand * esz <= 16 and C // cand >= 64:
                V = cand
                break
        chunks = -(-C // V)
        if chunks <= self.ROW_WAVE_CHUNKS:
            T, rows_per_block = 64, 4
        else:
            # at least ROW_CHUNKS_PER_THREAD chunks a thread: fewer, fuller waves spend less of the row's time
            # in the block-wide reductions (config 2's 4096-wide rows: 69 us at 256 threads, 77-80 at 512)
            per = -(-chunks // self.ROW_CHUNKS_PER_THREAD)
            T = min(self.ROW_MAX_THREADS, max(64, -(-per // 64) * 64))
            rows_per_block = 1
        J = -(-chunks // T)
        exact = C % (T * V) == 0
        # column indices in 32 bits when the row allows (they stay live across the row's passes)
        cty, csuf = ("int", "") if C < (1 << 31) else ("int64_t", "LL")
        em = self._emitter(rows=(R, C))
        # C % V == 0, so a V-element chunk is wholly inside the row or wholly past it: past-the-end chunks load
        # the row's last chunk (a clamped base keeps vector loads in bounds) and are masked out of reductions
        # and stores
        em.vec = V

        def vbase(j):
            b = f"(({j} * {T} + tid) * {V})"
            return b if exact else f"({b} < {C - V} ? (int64_t){b} : {C - V}LL)"
        body = []
        for red in reds:
            acc_dt = g.types[red.output].dtype
            act = COMP_T[acc_dt]
            isf = D.is_float(acc_dt)
            accn = em.tmp("acc")
            em.emit(f"{act} {accn} = {_red_identity(red.prim, acc_dt)};")
            for j in range(J):
                for lane in range(V):
                    cexpr = f"(({j} * {T} + tid) * {V} + {lane})"
                    cidx = f"c{j}_{lane}"
                    if cidx not in _declared(em):
                        em.emit(f"const {cty} {cidx} = {'' if exact else 'min('}{cexpr}{'' if exact else f', {C - 1}{csuf})'};")
                        _declared(em).add(cidx)
                    idx = ("rc", "r", cidx, vbase(j), lane)
                    val = em.value(red.inputs[0], idx)
                    guard = "" if exact else f"if ({cexpr} < {C}LL) "
                    em.emit(f"{guard}{accn} = {_red_update(em, red.prim, acc_dt, accn, val)};")
            total = em.tmp("red")
            op = "wsum" if red.prim == "reduce_sum" else "wmax"
            em.emit(f"{act} {total} = {op}(({act}){accn});")
            if rows_per_block == 1 and T > 64:
                nw = T // 64
                # float partials cross waves as doubles (exact for float32), integers as their 64-bit pattern
                lds = "red_lds" if isf else "red_ldsi"
                em.emit(f"if (lane == 0) {lds}[wave] = ({'double' if isf else 'int64_t'}){total};")
                em.emit("__syncthreads();")
                em.emit(f"{total} = ({act}){lds}[0];")
                for w in range(1, nw):
                    em.emit(f"{total} = {_red_update(em, red.prim, acc_dt, total, f'({act}){lds}[{w}]')};")
                em.emit("__syncthreads();")
            em.row_scalars[red.output] = total
        # element outputs
        stores = []
        for j in range(J):
            lanes = []
            for lane in range(V):
                cexpr = f"(({j} * {T} + tid) * {V} + {lane})"
                cidx = f"c{j}_{lane}"
                if cidx not in _declared(em):
                    em.emit(f"const {cty} {cidx} = {'' if exact else 'min('}{cexpr}{'' if exact else f', {C - 1}{csuf})'};")
                    _declared(em).add(cidx)
                idx = ("rc", "r", cidx, vbase(j), lane)
                lanes.append([em.value(v, idx) for v in outs_elem])
            for k, v in enumerate(outs_elem):
                oi = st.outputs.index(v)
                dt = g.types[v].dtype
                base = f"(r * {C}LL + ({j} * {T} + tid) * {V})"
                if V > 1 and self.out_views[v].contiguous():
                    s = self._vec_store(f"out{oi}", base, [lanes[l][k] for l in range(V)], dt, V, em, nt=v in self.far)
                else:
                    s = " ".join(
                        f"out{oi}[{self._out_addr(self.out_views[v], g.types[v].shape, f'({base} + {l})')}] = "
                        f"{_store(lanes[l][k], dt)};"
                        for l in range(V)
                    )
                if not exact:
                    s = f"if ((({j} * {T} + tid) * {V}) < {C}LL) {{ {s} }}"
                em.emit(s)  # stored as soon as computed: a chunk's results are not held across the row
        for v in outs_row:
            oi = st.outputs.index(v)
            val = em.value(v, ("r", "r"))
            dt = g.types[v].dtype
            addr = self._out_addr(self.out_views[v], g.types[v].shape, "r")
            stores.append(f"if (tid == 0) out{oi}[{addr}] = {_store(val, dt)};")
        body = em.lines
        pro = self._vec_prologue(em, V)
        threads = T * rows_per_block
        self.grid, self.block = (-(-R // rows_per_block), 1, 1), (threads, 1, 1)
        self.lds = 0
        src = [f'extern "C" __global__ __launch_bounds__({threads}) void {self.name}({self._params()}) {{']
        if rows_per_block > 1:
            src += [
                "  const int tid = threadIdx.x & 63; const int lane = tid; const int wave = threadIdx.x >> 6;",
                f"  const int64_t r = (int64_t)blockIdx.x * {rows_per_block} + wave;",
                f"  if (r >= {R}LL) return;",
            ]
        else:
            src += [
                "  const int tid = threadIdx.x; const int lane = tid & 63; const int wave = tid >> 6;",
                "  __shared__ double red_lds[16];",
                "  __shared__ int64_t red_ldsi[16];",
                "  const int64_t r = blockIdx.x;",
            ]
        src += ["  (void)lane; (void)wave;"]
        # vector loads need the c indices declared before them: emit prologue after index decls
        decl = [l for l in body if (l.startswith("const int64_t c") or l.startswith("const int c")) and "(( " not in l]
        rest = [l for l in body if l not in decl]
        src += ["  " + l for l in decl + pro + rest + stores]
        src += ["}"]
        return "\n".join(src)

    # ---- general reductions
    def _reduce(self):
        g, st = self.graph, self.step
        red = [n for n in st.nodes if n.prim in ("reduce_sum", "reduce_max")]
        if len(red) != 1 or red[0].output != st.outputs[0] or len(st.outputs) != 1:
            raise Unfusable(st.outputs[0], "a reduce step computes one reduction")
        red = red[0]
        x = g.types[red.inputs[0]]
        axes = tuple(red.params["axes"])
        kept = [d for d in range(len(x.shape)) if d not in axes]
        oshape = tuple(x.shape[d] for d in kept)
        rshape = tuple(x.shape[d] for d in axes)
        O, Q = math.prod(oshape), math.prod(rshape)
        out_dt = g.types[red.output].dtype
        atomic = red.prim == "reduce_sum" and out_dt == "float32" and Q >= 64
        chunk = max(1, min(Q, 64)) if atomic else Q
        nchunks = -(-Q // chunk)
        if atomic and tuple(axes) == tuple(range(len(axes))) and O % 4 == 0 and O >= 256:
            # narrow sums ([8192, 512] -> [512]) take 64 columns x 16 row lanes a workgroup and longer chunks: as
            # many workgroups as 256 columns x 4 row lanes would give, a quarter of the atomic adds (the adds to
            # the few output columns, not the loads, bound these)
            cl = 64 if O >= 1024 else 16
            chunk = self.LEAD_CHUNK * (64 // cl)
            chunk = max(1, min(Q, chunk))
            return self._reduce_leading(red, Q, O, chunk, -(-Q // chunk), cl)
        em = self._emitter()
        om = em.multi(("flat", "o"), oshape)
        qm = em.multi(("flat", "q"), rshape)
        xm = [None] * len(x.shape)
        for i, d in enumerate(kept):
            xm[d] = om[i]
        for i, d in enumerate(axes):
            xm[d] = qm[i]
        em.lines = []
        val = em.value(red.inputs[0], ("multi", tuple(xm)))
        body = em.lines
        act = COMP_T[out_dt]
        upd = f"acc = {_red_update(em, red.prim, out_dt, 'acc', val)};"
        init = _red_identity(red.prim, out_dt)
        self.atomic = atomic
        threads = 256
        self.grid, self.block, self.lds = (-(-O // threads), nchunks, 1), (threads, 1, 1), 0
        addr = self._out_addr(self.out_views[red.output], oshape, "o")
        store = f"atomicAdd(&out0[{addr}], acc);" if atomic else f"out0[{addr}] = {_store('acc', out_dt)};"
        src = [
            f'extern "C" __global__ __launch_bounds__({threads}) void {self.name}({self._params()}) {{',
            f"  const int64_t o = (int64_t)blockIdx.x * {threads} + threadIdx.x;",
            f"  if (o >= {O}LL) return;",
            f"  const int64_t q0 = (int64_t)blockIdx.y * {chunk}LL;",
            f"  const int64_t q1 = min(q0 + {chunk}LL, {Q}LL);",
            f"  {act} acc = {init};",
            "  for (int64_t q = q0; q < q1; ++q) {",
        ]
        src += ["    " + l for l in body]
        src += ["    " + upd, "  }", "  " + store, "}"]
        return "\n".join(src)


    def _reduce_leading(self, red, Q, O, chunk, nchunks, cl=64):
        """float32 sum over the leading axes of a [Q, O] row-major value (a bias or norm-weight gradient): a
        workgroup covers 4 ``cl`` columns of ``chunk`` rows, each thread 4 consecutive columns (16-byte loads) of
        every (256 / ``cl``)-th row; the row lanes combine through LDS and the workgroup adds its column sums
        atomically into the zero-filled output (one atomic a column per chunk: the adds, not the loads, bound
        this kernel when chunks are short)."""
        rl = 256 // cl
        g = self.graph
        em = self._emitter()
        em.vec = 4
        vals = []
        for lane in range(4):
            vals.append(em.value(red.inputs[0], ("flat", f"(qb + {lane})", "qb", lane)))
        body = self._vec_prologue(em, 4) + em.lines
        self.atomic = True
        threads = 256
        self.grid, self.block, self.lds = (-(-O // (4 * cl)), nchunks, 1), (threads, 1, 1), 0
        view = self.out_views[red.output]
        oshape = g.types[red.output].shape
        adds = [f"atomicAdd(&out0[{self._out_addr(view, oshape, f'(o + {l})')}], "
                + " + ".join(f"part[{r}][tx][{l}]" for r in range(rl)) + ");" for l in range(4)]
        src = [
            f'extern "C" __global__ __launch_bounds__({threads}) void {self.name}({self._params()}) {{',
            f"  __shared__ float part[{rl}][{cl}][4];",
            f"  const int tx = threadIdx.x % {cl}, ty = threadIdx.x / {cl};",
            f"  const int64_t o = ((int64_t)blockIdx.x * {cl} + tx) * 4;",
            f"  const int64_t q0 = (int64_t)blockIdx.y * {chunk}LL;",
            f"  const int64_t q1 = min(q0 + {chunk}LL, {Q}LL);",
            "  float acc0 = 0, acc1 = 0, acc2 = 0, acc3 = 0;",
            f"  if (o < {O}LL) {{",
            f"#pragma unroll {self.LEAD_UNROLL}",
            f"  for (int64_t q = q0 + ty; q < q1; q += {rl}) {{",
            f"    const int64_t qb = q * {O}LL + o;",
        ]
        src += ["    " + l for l in body]
        src += [f"    acc{l} = ((float)(acc{l} + {vals[l]}));" for l in range(4)]
        src += ["  }", "  }"]
        src += [f"  part[ty][tx][{l}] = acc{l};" for l in range(4)]
        src += ["  __syncthreads();", f"  if (ty == 0 && o < {O}LL) {{"] + ["    " + a for a in adds] + ["  }", "}"]
        return "\n".join(src)


class HorizontalKernel:
    """Several loop kernels in one launch (``passes/horizontal.rs:394,566-605`` per-segment grid ranges): the
    grid is the members' grids end to end, and each workgroup runs the member whose range holds it, with that
    member's own block index and grid size."""

    def __init__(self, parts):
        self.parts = parts
        self.name = "KNAME"
        self.args = []

    def source(self):
        import re

        params, bodies, begin = [], [], 0
        self.args = []
        for i, k in enumerate(self.parts):
            src = k.source()
            if k.block != (256, 1, 1) or k.lds:
                raise Unfusable(k.step.outputs[0], "horizontal fusion of a kernel with another block shape")
            head, _, rest = src.partition("{\n")
            sig = re.search(r"void\s+\w+\((.*)\)\s*$", head.strip()).group(1)
            body = rest[: rest.rstrip().rindex("}")]
            ren = lambda t: re.sub(r"\b(in|out)(\d+)\b", lambda m_: f"m{i}_{m_.group(1)}{m_.group(2)}", t)
            params.append(ren(sig))
            body = ren(body).replace("blockIdx.x", "hb_").replace("gridDim.x", "hg_")
            n = k.grid[0]
            cond = f"if (b_ < {begin + n})" if i < len(self.parts) - 1 else ""
            bodies.append(f"  {'else ' if i else ''}{cond} {{\n    const int64_t hb_ = b_ - {begin}, hg_ = {n};\n"
                          + body + "  }")
            begin += n
            self.args += k.args
        self.grid, self.block, self.lds = (begin, 1, 1), (256, 1, 1), 0
        return "\n".join(
            [f'extern "C" __global__ __launch_bounds__(256) void {self.name}({", ".join(params)}) {{',
             "  const int64_t b_ = blockIdx.x;"] + bodies + ["}"]
        )


def _scatter_kernel(self):
    """``scatter_add``: the output already holds the operand (a fill or copy step before it); each update
    element is added atomically at the entry its index picks (float32: the order of the adds differs from the
    reference's sequential one, within float32 rounding; 32/64-bit integers: bit-exact, wrapping)."""
    g, st = self.graph, self.step
    n = st.nodes[0]
    x, ix, u = (g.types[v] for v in n.inputs)
    axis = n.params["axis"]
    # float32 adds are atomic float adds; 32/64-bit integers add as unsigned words, which wrap exactly like
    # the reference's two's-complement sum in any order
    atom = {"float32": ("float", "float"), "int32": ("unsigned int", "unsigned int"),
            "uint32": ("unsigned int", "unsigned int"), "int64": ("unsigned long long", "unsigned long long"),
            "uint64": ("unsigned long long", "unsigned long long")}.get(x.dtype)
    if atom is None:
        raise Unfusable(n.output, f"scatter_add into {x.dtype} (atomic adds are float32 or 32/64-bit integers)")
    em = Emitter(g, [], {v: (k, self.views[v]) for k, v in enumerate(st.inputs)})
    um = em.multi(("flat", "e"), u.shape)
    r = len(ix.shape)
    iv = em.value(n.inputs[1], ("multi", tuple(um[axis : axis + r])))
    val = em.value(n.inputs[2], ("multi", tuple(um)))
    em.emit(f"const int64_t kk = min(max((int64_t){iv}, 0LL), {max(x.shape[axis] - 1, 0)}LL);")
    xm = um[:axis] + ["kk"] + um[axis + r :]
    ov = self.out_views[n.output]
    terms = [f"({e}) * {s_}LL" for e, s_ in zip(xm, ov.strides) if s_ and e != "0"]
    addr = "(" + (" + ".join(terms) if terms else "0") + ")"
    NU = u.numel()
    threads = 256
    self.grid, self.block, self.lds = (max(1, min(-(-NU // threads), 65536)), 1, 1), (threads, 1, 1), 0
    params = []
    self.args = []
    for k, v in enumerate(st.inputs):
        params.append(f"const {STORE_T[g.types[v].dtype]}* __restrict__ in{k}")
        self.args.append(("in", v))
    params.append(f"{atom[0]}* __restrict__ out0")
    self.args.append(("out", n.output))
    src = [
        f'extern "C" __global__ __launch_bounds__({threads}) void {self.name}({", ".join(params)}) {{',
        f"  for (int64_t e = (int64_t)blockIdx.x * {threads} + threadIdx.x; e < {NU}LL; e += (int64_t)gridDim.x * {threads}) {{",
    ]
    src += ["    " + l for l in em.lines]
    cv = f"(float){val}" if x.dtype == "float32" else f"({atom[1]})(int64_t){val}"
    src += [f"    atomicAdd(&out0[{addr}], {cv});", "  }", "}"]
    return "\n".join(src)


LoopKernel._scatter = _scatter_kernel


def _declared(em):
    if not hasattr(em, "_decl"):
        em._decl = set()
    return em._decl


_ = (struct, TensorType, VEC_T)


class GemmEpilogueKernel:
    """A streamed GEMM (``gemm_stream_tile`` in gemm.h, 256 x 256 tiles, 8 wavefronts, k steps of 64) whose
    store is a fused loop step: the loop's elementwise body runs on the dot's sums rounded to the dot's output
    dtype, at the flat index of each [m, n] element, and writes the loop's outputs (plus the dot's own result
    when anything else reads it). The dot's lhs/rhs locations give ``a``/``b`` with the layout flags ``at``/``bt``
    (mn-contiguous operands), as nhip_gemm takes them."""


    # The k loops a generated epilogue kernel can instantiate: (k tile, gemm_stream_tile's k loop KL, waves a
    # row of the 2 x WN wave grid). Variant 0 is gemm_stream's config 7 body; variant 1 its config 11 body (k tile
    # 32, four stages, cross-tile fragment prefetch, buffer loads only); variant 2 its config 12 body (k tile 32,
    # four stages, ping-pong waves); variant 3 its config 14 body (k tile 64, two stages, four waves); variant 4
    # its config 15 body (the same on eight waves).
    VARIANTS = ((64, 0, 4), (32, 1, 4), (32, 2, 4), (64, 3, 2), (64, 3, 4))

    def __init__(self, graph, dot_step, loop_step, desc, at, bt, f16, store_dot, views, out_views, colsum=None,
                 variant=0, aliased=frozenset()):
        self.graph, self.dot, self.loop = graph, dot_step, loop_step
        self.aliased = aliased  # as LoopKernel.aliased
        self.far = frozenset()  # as LoopKernel.far
        self.variant = variant
        self.desc, self.at, self.bt, self.f16, self.store_dot = desc, at, bt, f16, store_dot
        # (value, sum): a float32 loop output summed over the rows into `sum` [n] (atomically, into zeros)
        # instead of being stored
        self.colsum = colsum
        self.views, self.out_views = views, out_views
        self.name = "KNAME"
        d = desc
        self.grid = (-(-d.m // 256) * -(-d.n // 256), 1, 1)
        self.block = (128 * self.VARIANTS[variant][2], 1, 1)
        self.lds = 0
        self.args = []

    def variant_ok(self, variant):
        """Whether k loop ``variant`` can run this dot (its k tile divides k; the cross-tile prefetch needs the
        buffer-load path)."""
        bk, kl, _ = self.VARIANTS[variant]
        return self.desc.k % bk == 0 and (kl != 1 or self.buffer_ok())

    def buffer_ok(self):
        """gemm.h's stream_buffer_ok: the operand bytes a 256 x 256 tile spans fit 32-bit buffer offsets."""
        d = self.desc
        lim = 1 << 31
        ab = ((d.k - 1) * d.a_k + 256) * 2 if self.at else (255 * d.a_m + d.k) * 2
        bb = ((d.k - 1) * d.b_k + 256) * 2 if self.bt else (255 * d.b_n + d.k) * 2
        return ab < lim and bb < lim

    def source(self):
        g, dot, loop = self.graph, self.dot, self.loop
        dv = dot.nodes[0].output
        d = self.desc
        n = d.n
        if n % 4:
            raise Unfusable(dv, "GEMM epilogue over a row length that is not a multiple of 4")
        ddt = g.types[dv].dtype
        lin = [v for v in loop.inputs if v != dv]
        # the loop's body, evaluated 4 columns at a time at row r, columns c + lane of the [m, n] result
        lk = LoopKernel(g, loop, "KNAME", {v: self.views[v] for v in lin}, self.out_views, self.aliased)
        lk.far = self.far
        em = Emitter(g, loop.nodes, {v: (k, self.views[v]) for k, v in enumerate(lin)})
        em.outputs = set(loop.outputs)
        em.vec = 4
        accs = [f"acc.{c}" for c in "xyzw"]
        dnames = []
        for lane in range(4):
            nm = em.tmp("d")
            em.emit(f"const float {nm} = {em.round(accs[lane], ddt) if ddt != 'float32' else accs[lane]};")
            dnames.append(nm)

        def given(idx):
            if idx[0] == "rc" and len(idx) == 5 and idx[1] == "r" and idx[3] == "c":
                return dnames[idx[4]]
            raise Unfusable(dv, "the fused loop reads the dot's result at another index")

        em.given[dv] = given
        # elements are indexed by (row r, column c + lane): an operand broadcast along the row (a per-row
        # statistic) is read at r, not at (r n + c + lane) / n
        em.rows, em.rows_uniform = (d.m, d.n), False
        stored = [v for v in loop.outputs if not (self.colsum and v == self.colsum[0])]
        per_lane = []
        summed = []
        for lane in range(4):
            idx = ("rc", "r", f"(c + {lane})", "c", lane)
            per_lane.append([em.value(v, idx) for v in stored])
            if self.colsum:
                summed.append(em.value(self.colsum[0], idx))
        body = em.lines
        pro = lk._vec_prologue(em, 4, lin)
        stores = []
        outs = ([dv] if self.store_dot else []) + stored
        for k, v in enumerate(outs):
            dt = g.types[v].dtype
            names = dnames if (self.store_dot and k == 0) else [per_lane[l][k - (1 if self.store_dot else 0)] for l in range(4)]
            view = self.out_views[v]
            if view.contiguous():
                stores.append(lk._vec_store(f"out{k}", "base", names, dt, 4, em, nt=v in self.far))
            else:
                for lane in range(4):
                    addr = lk._out_addr(view, g.types[v].shape, f"(base + {lane})")
                    stores.append(f"out{k}[{addr}] = {_store(names[lane], dt)};")
        if self.colsum:
            outs = outs + [self.colsum[1]]  # the float32 [n] sums, last
            ret = f"return make_float4({', '.join(summed)});"
            colsum_fn = ["  __device__ __forceinline__ void colsum_add(int64_t c, float4 v) const {",
                         f"    float* p = out{len(outs) - 1} + c;",
                         "    atomicAdd(p, v.x); atomicAdd(p + 1, v.y); atomicAdd(p + 2, v.z); atomicAdd(p + 3, v.w);",
                         "  }"]
        else:
            ret, colsum_fn = "", []
        self.args = [("in", dot.nodes[0].inputs[0]), ("in", dot.nodes[0].inputs[1])]
        self.args += [("in", v) for v in lin] + [("out", v) for v in outs]
        al = self.aliased
        fields = [f"const {STORE_T[g.types[v].dtype]}*{_restrict(v, al)} in{k};" for k, v in enumerate(lin)]
        fields += [f"{STORE_T[g.types[v].dtype]}*{_restrict(v, al)} out{k};" for k, v in enumerate(outs)]
        params = ["const uint16_t* __restrict__ a", "const uint16_t* __restrict__ b"]
        params += [f"const {STORE_T[g.types[v].dtype]}*{_restrict(v, al)} in{k}" for k, v in enumerate(lin)]
        params += [f"{STORE_T[g.types[v].dtype]}*{_restrict(v, al)} out{k}" for k, v in enumerate(outs)]
        init = ", ".join([f"in{k}" for k in range(len(lin))] + [f"out{k}" for k in range(len(outs))])
        shape = (f"s.m = {d.m}LL; s.n = {d.n}LL; s.k = {d.k}LL; s.nbatch = 0; s.a_m = {d.a_m}LL; "
                 f"s.a_k = {d.a_k}LL; s.b_k = {d.b_k}LL; s.b_n = {d.b_n}LL; s.d_m = {d.n}LL; s.d_n = 1; "
                 f"s.tiles_m = {-(-d.m // 256)}; s.tiles_n = {-(-d.n // 256)}; s.d_split = 0;")
        # the vector loads of the other operands move into load(): gemm.h issues them ahead of the sums' staging
        pre_fields, pre_loads, pre_uses, rest = [], [], [], []
        for l in pro:
            m = re.match(r"const ((?:u16v|u32v|u64v)<\d+>) (\w+) = (.*);$", l)
            if m:
                pre_fields.append(f"{m.group(1)} {m.group(2)};")
                pre_loads.append(f"p.{m.group(2)} = {m.group(3)};")
                pre_uses.append(f"const {m.group(1)} {m.group(2)} = pre.{m.group(2)};")
            else:
                rest.append(l)
        bk, kl, wn = self.VARIANTS[self.variant]
        if not self.variant_ok(self.variant):
            raise Unfusable(dv, f"GEMM epilogue k loop variant {self.variant} does not fit k = {d.k}")
        # chunks read ahead at a time: at most 64 VGPRs of 16-byte loads
        ahead = 16
        while ahead > 1 and ahead * len(pre_fields) > 16:
            ahead //= 2
        lines = [
            '#include "gemm.h"',
            "struct EpiKNAME {",
            *["  " + f for f in fields],
            f"  static constexpr int kPrefetch = {ahead};",
            f"  static constexpr bool kColSum = {'true' if self.colsum else 'false'};",
            *colsum_fn,
            "  struct Pre {", *["    " + f for f in pre_fields], "  };",
            "  __device__ __forceinline__ Pre load(int64_t r, int64_t c) const {",
            f"    const int64_t base = r * {n}LL + c;",
            "    Pre p;", *["    " + l for l in pre_loads], "    return p;",
            "  }",
            f"  __device__ __forceinline__ {'float4' if self.colsum else 'void'} operator()(int64_t r, int64_t c, float4 acc, "
            "const Pre &pre) const {",
            f"    const int64_t base = r * {n}LL + c;",
            *["    " + l for l in pre_uses + rest + body + stores + ([ret] if ret else [])],
            "  }",
            "};",
            f'extern "C" __global__ __launch_bounds__({128 * wn}) __attribute__((amdgpu_waves_per_eu({wn // 2}, {wn // 2}))) '
            f'void KNAME({", ".join(params)}) {{',
            f"  __shared__ __align__(1024) char smem[nhipk::gemm_stream_lds_bytes<{bk}, {wn}>()];",
            "  nhipk::GemmShape s;",
            f"  {shape}",
            f"  nhipk::gemm_stream_tile<{'true' if self.f16 else 'false'}, {bk}, {wn}, {'true' if self.at else 'false'}, "
            f"{'true' if self.bt else 'false'}, {'true' if self.buffer_ok() else 'false'}, EpiKNAME, 256, "
            f"{kl}>(s, a, b, EpiKNAME{{{init}}}, smem);",
            "}",
        ]
        return "\n".join(lines)
