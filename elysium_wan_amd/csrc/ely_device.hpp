// ely_device.hpp -- device-side building blocks shared by the gfx950 kernels.
//
// Numerics follow torch's conversions bit for bit:
//   * fp32 -> bf16: round to nearest even, every NaN -> 0x7FC0
//     (TORCH/include/torch/headeronly/util/BFloat16.h:100-114).
//   * fp32 -> fp8 e4m3fn / e5m2: round to nearest even on the format's grid;
//     e4m3fn values that round past 448 and NaN/Inf give 0x7F|sign, e5m2
//     values that round past 57344 and Inf give 0x7C|sign, NaN 0x7F|sign
//     (Float8_e4m3fn.h:170-232, Float8_e5m2.h:77-143).  `fp8_from_f32_sw` is
//     an integer restatement of that rule; the hot loops use the gfx950
//     conversion instruction (v_cvt_pk_fp8_f32 / v_cvt_pk_bf8_f32) on the
//     domain ely_selftest_fp8_cvt proves it equal on (finite values at or below
//     the format's largest finite value), for bf16 data the scaled
//     conversions (v_cvt_scalef32_pk_*) on the pairs ely_selftest_fp8_scaled
//     proves them equal on, and the restatement elsewhere.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#pragma clang fp contract(off)

namespace ely {

constexpr int kWave = 64;
constexpr int kE4M3 = 0;
constexpr int kE5M2 = 1;

template <int FMT>
struct Fp8Fmt;
template <>
struct Fp8Fmt<kE4M3> {
    static constexpr int M = 3;                       // mantissa bits
    static constexpr int BIAS = 7;
    static constexpr int EBIAS = 8;                   // fp8.py:18, 2^8 > 448
    static constexpr uint32_t kOverflowBits = 0x43F00000u;  // 480.0f: NaN from here up
    static constexpr uint32_t kMaxFiniteBits = 0x43E00000u; // 448.0f
};
template <>
struct Fp8Fmt<kE5M2> {
    static constexpr int M = 2;
    static constexpr int BIAS = 15;
    static constexpr int EBIAS = 15;                  // fp8.py:19, 2^16 > 57344
    static constexpr uint32_t kOverflowBits = 0x47800000u;  // 65536.0f: Inf from here up
    static constexpr uint32_t kMaxFiniteBits = 0x47600000u; // 57344.0f
};

__device__ __forceinline__ float bf16_to_f32(uint32_t h16) { return __uint_as_float(h16 << 16); }

// fp32 -> bf16 bits, RNE, NaN -> 0x7FC0.
__device__ __forceinline__ uint32_t f32_to_bf16(float f) {
    uint32_t u = __float_as_uint(f);
    uint32_t r = (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
    return (f != f) ? 0x7FC0u : r;
}

// Integer restatement of torch's fp32 -> fp8 conversion (see file header).
template <int FMT>
__device__ __forceinline__ uint32_t fp8_from_f32_sw(float f) {
    using F = Fp8Fmt<FMT>;
    constexpr int M = F::M;
    const uint32_t u = __float_as_uint(f);
    const uint32_t sign = (u >> 24) & 0x80u;
    const uint32_t a = u & 0x7FFFFFFFu;
    if (a > 0x7F800000u) return 0x7Fu | sign;                       // NaN
    if (a >= F::kOverflowBits) return (FMT == kE4M3 ? 0x7Fu : 0x7Cu) | sign;
    const int ebits = (int)(a >> 23);
    const uint32_t mant = (a & 0x7FFFFFu) | (ebits ? 0x800000u : 0u);   // value = mant * 2^(E-23)
    const int E = (ebits ? ebits : 1) - 127;
    const int emin = 1 - F::BIAS;
    int Eq = E < emin ? emin : E;                                     // quantum = 2^(Eq - M)
    const int shift = 23 + Eq - M - E;                                // >= 23 - M
    if (shift >= 25) return sign;                                     // below half the smallest subnormal
    uint32_t qv = mant >> shift;
    const uint32_t rem = mant & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (qv & 1u))) ++qv;
    if (qv == (2u << M)) {                                            // carry into the next binade
        ++Eq;
        qv = 1u << M;
    }
    uint32_t code = qv < (1u << M) ? qv : ((uint32_t)(Eq + F::BIAS) << M) | (qv - (1u << M));
    return code | sign;
}

// fp8 code -> fp32 (exact), restated from the format definition.
template <int FMT>
__device__ __forceinline__ float fp8_to_f32_sw(uint32_t c) {
    using F = Fp8Fmt<FMT>;
    constexpr int M = F::M;
    const uint32_t sign = (c & 0x80u) << 24;
    const uint32_t e = (c & 0x7Fu) >> M;
    const uint32_t m = c & ((1u << M) - 1u);
    uint32_t bits;
    if (FMT == kE4M3 && (c & 0x7Fu) == 0x7Fu) {
        bits = 0x7FC00000u;
    } else if (FMT == kE5M2 && e == 31u) {
        bits = m ? 0x7FC00000u : 0x7F800000u;
    } else if (e == 0u) {
        // m * 2^(1 - BIAS - M): a small integer times a power of two, exact
        const float quantum = __uint_as_float((uint32_t)(127 + 1 - F::BIAS - M) << 23);
        bits = __float_as_uint((float)m * quantum);
    } else {
        bits = ((e - F::BIAS + 127u) << 23) | (m << (23 - M));
    }
    return __uint_as_float(bits | sign);
}

// Two fp32 -> two fp8 codes in the low (HI=false) or high half of `old`.
template <int FMT, bool HI>
__device__ __forceinline__ uint32_t cvt_pk_fp8(float a, float b, uint32_t old) {
    if (FMT == kE4M3) return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(a, b, (int)old, HI);
    return (uint32_t)__builtin_amdgcn_cvt_pk_bf8_f32(a, b, (int)old, HI);
}

// Two fp8 codes (low or high 16 bits of `w`) -> two fp32.
template <int FMT, bool HI>
__device__ __forceinline__ void cvt_pk_f32(uint32_t w, float& a, float& b) {
    typedef float float2_ __attribute__((ext_vector_type(2)));
    float2_ r;
    if (FMT == kE4M3) r = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, HI);
    else r = __builtin_amdgcn_cvt_pk_f32_bf8((int)w, HI);
    a = r.x;
    b = r.y;
}

typedef short ely_s16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 ely_bf16x2 __attribute__((ext_vector_type(2)));

// Two bf16 (the low and high half of `w`) -> two fp8 codes, each x / scale
// rounded to the format in one step (v_cvt_scalef32_pk_fp8_bf16 /
// v_cvt_scalef32_pk_bf8_bf16), into the low (HI=false) or high half of
// `old`.  With scale = 2^k this is the code of x * 2^-k for every bf16 x and
// |k| <= 110 with |x| 2^-k below 2^ebias, the pairs the quantize instruction
// path meets (ely_selftest_fp8_scaled checks all of them).
template <int FMT, bool HI>
__device__ __forceinline__ uint32_t cvt_scaled_pk_fp8_bf16(uint32_t w, float scale, uint32_t old) {
    const ely_bf16x2 x = __builtin_bit_cast(ely_bf16x2, w);
    const ely_s16x2 o = __builtin_bit_cast(ely_s16x2, old);
    ely_s16x2 r;
    if (FMT == kE4M3) r = __builtin_amdgcn_cvt_scalef32_pk_fp8_bf16(o, x, scale, HI);
    else r = __builtin_amdgcn_cvt_scalef32_pk_bf8_bf16(o, x, scale, HI);
    return __builtin_bit_cast(uint32_t, r);
}

// Two fp8 codes (low or high 16 bits of `w`) -> two bf16 (one word), each
// code's value times `scale` (v_cvt_scalef32_pk_bf16_fp8 / _bf8).  With
// scale = 2^k, |k| <= 110, the exact product for every code but the NaN
// codes, whose result is a NaN with other bits than torch's 0x7FC0: callers
// keep NaN codes off this path (ely_selftest_fp8_scaled checks the rest).
template <int FMT, bool HI>
__device__ __forceinline__ uint32_t cvt_scaled_pk_bf16(uint32_t w, float scale) {
    ely_bf16x2 r;
    if (FMT == kE4M3) r = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, scale, HI);
    else r = __builtin_amdgcn_cvt_scalef32_pk_bf16_bf8(w, scale, HI);
    return __builtin_bit_cast(uint32_t, r);
}

// Whether any of the four codes of `w` is a NaN code (e4m3: |c| = 0x7F;
// e5m2: |c| in 0x7D..0x7F): adding 1 (3) to every 7-bit magnitude carries
// into bit 7 exactly for those, and never into the next byte.
template <int FMT>
__device__ __forceinline__ uint32_t nan_code_bits(uint32_t w) {
    return ((w & 0x7F7F7F7Fu) + (FMT == kE4M3 ? 0x01010101u : 0x03030303u)) & 0x80808080u;
}

// 2^n rounded once to fp32 (Inf at n >= 128, 0 below 2^-149 with the tie at
// 2^-150 going to 0) and, for bf16 tensors, once more to bf16: torch.exp2 of
// an integer-valued tensor of that dtype (fp8.py:41-42).
__device__ __forceinline__ float pow2_dtype(int n, bool bf16) {
    float f;
    if (n >= 128) f = __uint_as_float(0x7F800000u);
    else if (n >= -126) f = __uint_as_float((uint32_t)(n + 127) << 23);
    else if (n >= -149) f = __uint_as_float(1u << (n + 149));
    else f = 0.0f;
    if (bf16) f = bf16_to_f32(f32_to_bf16(f));
    return f;
}

// frexp exponent of a finite, positive fp32 bit pattern (value = m * 2^e,
// m in [0.5, 1)).
__device__ __forceinline__ int frexp_exp_bits(uint32_t a) {
    const uint32_t eb = a >> 23;
    if (eb) return (int)eb - 126;
    return (31 - __builtin_clz(a)) - 148;  // subnormal: a * 2^-149
}

// k of fp8.scale_exp from the row's |x|max fp32 bits (fp8.py:28-38):
// 0 for an all-zero or NaN row, frexp(Inf) reports 0 so Inf gives -ebias.
template <int FMT>
__device__ __forceinline__ int scale_exp_from_amax(uint32_t abits) {
    if (abits == 0u || abits > 0x7F800000u) return 0;
    if (abits == 0x7F800000u) return -Fp8Fmt<FMT>::EBIAS;
    return frexp_exp_bits(abits) - Fp8Fmt<FMT>::EBIAS;
}

// ------------------------------------------------------------ wave reductions

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        uint32_t w = (uint32_t)__shfl_xor((int)v, o, kWave);
        v = v > w ? v : w;
    }
    return v;
}

__device__ __forceinline__ uint32_t wave_sum_u32(uint32_t v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += (uint32_t)__shfl_xor((int)v, o, kWave);
    return v;
}

// Butterfly sum: every lane ends with the same value, in a fixed order.
__device__ __forceinline__ double wave_sum_f64(double v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}

__device__ __forceinline__ int wave_uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

// ------------------------------------------------------------------- AdamW

struct HostConsts {
    float decay, b1, one_b1, b2, one_b2, inv_bc2_sqrt, eps, step_size;
};

// runtime/optim.py:277-298, one IEEE fp32 rounding per line (contract(off)).
// The sqrt is the correctly rounded fp32 sqrt, which equals the reference's
// fp64 sqrt rounded once to fp32 (53 >= 2*24 + 2 bits, so the double rounding
// is innocuous); the division is IEEE.
// The moments' half and the parameter's half are separate calls, so that a
// kernel can store m and v before the sqrt and the division; p's decay
// touches p alone, so where it runs does not change a bit.
__device__ __forceinline__ void adamw_host_moments(float g, float& m, float& v, const HostConsts& c) {
    m = m * c.b1;
    float t = g * c.one_b1;
    m = m + t;
    v = v * c.b2;
    float s = g * g;
    s = s * c.one_b2;
    v = v + s;
}

__device__ __forceinline__ void adamw_host_param(float& p, float m, float v, const HostConsts& c, bool wd) {
    if (wd) p = p * c.decay;
    float d = __builtin_sqrtf(v);
    d = d * c.inv_bc2_sqrt;
    d = d + c.eps;
    float u = m / d;
    u = u * c.step_size;
    p = p - u;
}

__device__ __forceinline__ void adamw_host_elem(float& p, float g, float& m, float& v,
                                                const HostConsts& c, bool wd) {
    adamw_host_moments(g, m, v, c);
    adamw_host_param(p, m, v, c, wd);
}

struct TorchConsts {
    float decay, w1, b2, one_b2, bc2_sqrt, eps, neg_step, unused;
};

// torch.optim.AdamW's foreach op order (TORCH/optim/adam.py:688-800):
// lerp (ATen Lerp.h), addcmul/addcdiv as a + s * (b op c), as fmas.
__device__ __forceinline__ void adamw_torch_moments(float g, float& m, float& v, const TorchConsts& c) {
    if (__builtin_fabsf(c.w1) < 0.5f) {
        m = __builtin_fmaf(c.w1, g - m, m);
    } else {
        m = __builtin_fmaf(-(g - m), 1.0f - c.w1, g);
    }
    v = v * c.b2;
    v = __builtin_fmaf(c.one_b2, g * g, v);
}

__device__ __forceinline__ void adamw_torch_param(float& p, float m, float v, const TorchConsts& c, bool wd) {
    if (wd) p = p * c.decay;
    float d = __builtin_sqrtf(v);
    d = d / c.bc2_sqrt;
    d = d + c.eps;
    p = __builtin_fmaf(c.neg_step, m / d, p);
}

__device__ __forceinline__ void adamw_torch_elem(float& p, float g, float& m, float& v,
                                                 const TorchConsts& c, bool wd) {
    adamw_torch_moments(g, m, v, c);
    adamw_torch_param(p, m, v, c, wd);
}

}  // namespace ely
