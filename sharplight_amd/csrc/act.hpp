// The gating activations of the fused-layer-op kernels (gated activation, dual matvec epilogue), as the
// reference's CPU provider computes them (src/Sharplight.Cpu/ScalarMath.cs:552-641):
//   SILU:      g / (1 + exp(-g))
//   GELU_TANH: g / (1 + exp(-u)),  u = (2*0.7978845608) * fma(0.044715*g, g*g, g)
//   GELU_ERF:  0.5*g*(1 + erf(g*0.70710678))
#pragma once

#include "common.hpp"

namespace slhip {

// erf: the published Eigen/XLA rational approximation that the reference CPU provider uses
// (ScalarMath.ErfD / ErfV, src/Sharplight.Cpu/ScalarMath.cs:51-98), p(x)/q(x) on the argument clamped to
// +-3.8325. The reference evaluates it in f64 and narrows to f32; here it is evaluated in f32 (fma Horner
// steps, hardware reciprocal), which is the precision the coefficients were fitted for. Measured against
// the f64 evaluation: at most 6 ulp / 3.6e-7 absolute in erf. f64 arithmetic costs ~30 VALU slots per
// element, which made a bf16 GeGLU compute-bound (1.5x the time of the same bytes copied); this form is
// ~15 slots and keeps it on the HBM roofline. The difference to the reference stays within the f32
// activation tolerance (1e-5 relative, 1e-5 x the row's RMS absolute where 1 + erf cancels for x << 0).
// NaN inputs: the clamp (v_med3_f32) does not propagate NaN, so callers that need erf(NaN) = NaN test it.
__device__ __forceinline__ float erf_rational(float xf)
{
    const float x = __builtin_amdgcn_fmed3f(xf, -3.832506856900711f, 3.832506856900711f);
    const float x2 = x * x;
    float p = -2.72614225801306e-10f;
    p = fmaf(p, x2, 2.77068142495902e-08f);
    p = fmaf(p, x2, -2.10102402082508e-06f);
    p = fmaf(p, x2, -5.69250639462346e-05f);
    p = fmaf(p, x2, -7.34990630326855e-04f);
    p = fmaf(p, x2, -2.95459980854025e-03f);
    p = fmaf(p, x2, -1.60960333262415e-02f);
    p *= x;
    float q = -1.45660718464996e-05f;
    q = fmaf(q, x2, -2.13374055278905e-04f);
    q = fmaf(q, x2, -1.68282697438203e-03f);
    q = fmaf(q, x2, -7.37332916720468e-03f);
    q = fmaf(q, x2, -1.42647390514189e-02f);
    return p * __builtin_amdgcn_rcpf(q);
}

template <int ACT> __device__ __forceinline__ float activate(float g)
{
    constexpr float kLog2e = 1.4426950408889634f;
    if (ACT == SLHIP_ACT_SILU) {
        float e = __builtin_amdgcn_exp2f(-g * kLog2e);
        return g * __builtin_amdgcn_rcpf(1.0f + e);
    } else if (ACT == SLHIP_ACT_GELU_TANH) {
        float u = (0.7978845608028654f * 2.0f) * fmaf(0.044715f * g, g * g, g);
        float e = __builtin_amdgcn_exp2f(-u * kLog2e);
        return g * __builtin_amdgcn_rcpf(1.0f + e);
    } else {
        return 0.5f * g * (1.0f + erf_rational(g * 0.7071067811865476f));
    }
}

}  // namespace slhip
