// The gating activations of the fused-layer-op kernels (gated activation, dual matvec epilogue), as the
// reference's CPU provider computes them (src/Sharplight.Cpu/ScalarMath.cs:552-641):
//   SILU:      g / (1 + exp(-g))
//   GELU_TANH: g / (1 + exp(-u)),  u = (2*0.7978845608) * fma(0.044715*g, g*g, g)
//   GELU_ERF:  0.5*g*(1 + erf(g*0.70710678))
#pragma once

#include "common.hpp"

namespace slhip {

// erf as the reference CPU provider's vector path computes it (ScalarMath.ErfD / ErfV,
// src/Sharplight.Cpu/ScalarMath.cs:51-98): the published Eigen/XLA rational approximation evaluated in
// f64 (fma Horner steps) on the argument clamped to +-3.8325, narrowed to f32. Evaluating it the same
// way keeps 1 + erf(x) -- which cancels for x << 0 -- identical to the reference's.
__device__ __forceinline__ float erf_rational(float xf)
{
    const double clampv = static_cast<double>(3.832506856900711f);
    double x = static_cast<double>(xf);
    x = x < -clampv ? -clampv : (x > clampv ? clampv : x);
    const double x2 = x * x;
    double p = -2.72614225801306e-10;
    p = fma(p, x2, 2.77068142495902e-08);
    p = fma(p, x2, -2.10102402082508e-06);
    p = fma(p, x2, -5.69250639462346e-05);
    p = fma(p, x2, -7.34990630326855e-04);
    p = fma(p, x2, -2.95459980854025e-03);
    p = fma(p, x2, -1.60960333262415e-02);
    p *= x;
    double q = -1.45660718464996e-05;
    q = fma(q, x2, -2.13374055278905e-04);
    q = fma(q, x2, -1.68282697438203e-03);
    q = fma(q, x2, -7.37332916720468e-03);
    q = fma(q, x2, -1.42647390514189e-02);
    return static_cast<float>(p / q);
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
