// Device helpers shared by every Mira mixer kernel (gfx950 / CDNA4, wave64).
//
// Element types cross the C-ABI as an int code (MIRA_F32, MIRA_BF16, MIRA_F16) and are widened to
// float on load: every recurrence, readout and gate is computed in float32, as the reference mixer
// does (model/mira_mixer.py:301-307), and only the output is narrowed back to the input type.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mira {

// ---------------------------------------------------------------------------------------------
// element types
// ---------------------------------------------------------------------------------------------
struct bf16_t { uint16_t bits; };
typedef _Float16 f16_t;

__device__ __forceinline__ float to_float(float v) { return v; }
__device__ __forceinline__ float to_float(bf16_t v) {
    return __uint_as_float(static_cast<uint32_t>(v.bits) << 16);
}
__device__ __forceinline__ float to_float(f16_t v) { return static_cast<float>(v); }

// float -> bfloat16, round to nearest even; NaN stays a (quiet) NaN.
__device__ __forceinline__ uint16_t bf16_bits(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return static_cast<uint16_t>(u >> 16);
}

template <typename IO> __device__ __forceinline__ IO from_float(float v);
template <> __device__ __forceinline__ float from_float<float>(float v) { return v; }
template <> __device__ __forceinline__ bf16_t from_float<bf16_t>(float v) {
    bf16_t r; r.bits = bf16_bits(v); return r;
}
template <> __device__ __forceinline__ f16_t from_float<f16_t>(float v) {
    return static_cast<f16_t>(v);
}

template <typename IO>
__device__ __forceinline__ float load(const IO *p) { return to_float(*p); }

// ---------------------------------------------------------------------------------------------
// the stage maps: alpha -> (cos, sin), beta -> r                model/mira_mixer.py:56-155
//
// The arch code is the reference kernel's stage mode (kernel/cuda/mira_dspv2/mira.py:305-309):
// 3 cauchy_x_mobius, 6 cauchy_x_hyperbolic, 7 cauchy_x_identity, then for 8..19 radius
// (mode-8)/3+1 in {gaussian, expexp, expsoftplus, hill} and rotation (mode-8)%3 in
// {mobius, hyperbolic, identity}. Reciprocals and exponentials come from the hardware
// approximation refined to a few ulp (rcp_refined) and the hardware exponential (exp_hw); the
// identity rotation uses sincosf.
// ---------------------------------------------------------------------------------------------
enum Radius { CAUCHY = 0, GAUSSIAN = 1, EXPEXP = 2, EXPSOFTPLUS = 3, HILL = 4 };
enum Rotation { MOBIUS = 0, HYPERBOLIC = 1, IDENTITY = 2 };

__host__ __device__ __forceinline__ bool arch_valid(int mode) {
    return mode == 3 || (mode >= 6 && mode <= 19);
}
__host__ __device__ __forceinline__ int radius_of(int mode) {
    return mode < 8 ? CAUCHY : 1 + (mode - 8) / 3;
}
__host__ __device__ __forceinline__ int rotation_of(int mode) {
    return mode == 3 ? MOBIUS : (mode == 6 ? HYPERBOLIC : (mode == 7 ? IDENTITY : (mode - 8) % 3));
}

// Reciprocal, quotient and exponential from the hardware approximations (v_rcp_f32, v_exp_f32)
// refined to within a few ulp: one Newton step for the reciprocal (r' = r + r (1 - d r)), one
// residual correction for the quotient, and Cody-Waite range reduction for e^x
// (x = k ln2 + f, ln2 split in a high part exact in float and a low part; e^x = 2^k 2^(f/ln2)).
__device__ __forceinline__ float rcp_refined(float d) {
    const float r = __builtin_amdgcn_rcpf(d);
    return fmaf(r, fmaf(-d, r, 1.0f), r);
}
__device__ __forceinline__ float exp_refined(float x) {
    x = fminf(fmaxf(x, -104.0f), 88.7f);             // e^x is 0 / +inf beyond these in float
    const float k = rintf(x * 1.44269504088896341f);
    float f = fmaf(-k, 0.693145751953125f, x);       // ln2 high part: 11 significant bits
    f = fmaf(-k, 1.42860682030941723212e-6f, f);     // ln2 - high part
    return ldexpf(__builtin_amdgcn_exp2f(f * 1.44269504088896341f), (int)k);
}
// e^x as the hardware's 2^y of y = x log2(e): relative error about 2^-24 |x| from rounding y plus
// v_exp_f32's own ulp (|x| <= 36 in the maps: under 3e-6 relative on values below e^-1 wherever
// |x| > 1, so under 1e-6 absolute); the forward stage maps use it, the backward keeps exp_refined
__device__ __forceinline__ float exp_hw(float x) {
    return __builtin_amdgcn_exp2f(x * 1.44269504088896341f);
}

// r cos(theta) and r sin(theta) of one stage.
__device__ __forceinline__ void stage_coefficients(float alpha, float beta, int radius_kind,
                                                   int rotation_kind, float &rc, float &rs) {
    float c, s;
    if (rotation_kind == MOBIUS) {
        // sin = (1 - a^2)/(1 + a^2), cos = 2a/(1 + a^2), written in 1/a above |a| = 1
        const bool small = fabsf(alpha) <= 1.0f;
        const float base = small ? alpha : rcp_refined(alpha);
        const float square = base * base;
        const float inv = rcp_refined(1.0f + square);
        c = 2.0f * base * inv;
        s = (small ? (1.0f - square) : (square - 1.0f)) * inv;
    } else if (rotation_kind == HYPERBOLIC) {
        // with e = exp(-|a|): cos = sech(a) = 2e/(1 + e^2), sin = tanh(a) = sign(a) (1 - e^2)/(1 + e^2)
        const float e = exp_hw(-fabsf(alpha));
        const float inv = rcp_refined(fmaf(e, e, 1.0f));
        c = 2.0f * e * inv;
        s = copysignf(fmaf(-e, e, 1.0f) * inv, alpha);
    } else {
        sincosf(alpha, &s, &c);
    }
    float r;
    if (radius_kind == CAUCHY) {
        r = rcp_refined(fmaf(beta, beta, 1.0f));
    } else if (radius_kind == GAUSSIAN) {
        r = exp_hw(-(beta * beta));
    } else if (radius_kind == EXPEXP) {
        r = exp_hw(-exp_hw(fminf(beta, 80.0f)));
    } else if (radius_kind == EXPSOFTPLUS) {
        r = rcp_refined(1.0f + exp_hw(beta));        // exp(-softplus(beta)) = sigmoid(-beta)
    } else {
        const float q = beta * beta;                 // hill: q/(1+q), 1 - 1/(1+q) above q = 1
        const float inv = rcp_refined(1.0f + q);
        r = q > 1.0f ? 1.0f - inv : q * inv;
    }
    rc = r * c;
    rs = r * s;
}

__device__ __forceinline__ float silu(float g) { return g / (1.0f + expf(-g)); }

// ---------------------------------------------------------------------------------------------
// wave64 helpers
// ---------------------------------------------------------------------------------------------
// Sum over aligned groups of W lanes (W a power of two <= 64), result in every lane of the group.
template <int W>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
    for (int offset = W / 2; offset > 0; offset >>= 1) v += __shfl_xor(v, offset, 64);
    return v;
}

}  // namespace mira
