#pragma once
// The arithmetic of the elementwise ops, shared by the standalone elementwise kernels (elementwise.hip) and
// the fused elementwise groups (ewgroup.hip): BinaryOp and ScalarMath.Unary of the reference CPU provider.
#include "act.hpp"
#include "common.hpp"

#include <math.h>

namespace slhip {

// ---- arithmetic ------------------------------------------------------------------------------------

// IEEE 754-2019 maximum / minimum, as .NET's MathF.Max/Min and Vector*.Max/Min: a NaN operand gives NaN,
// and +0 is above -0.
__device__ __forceinline__ float ieee_max(float a, float b)
{
    if (a != a) return a;
    if (b != b) return b;
    if (a == b) return signbit(a) ? b : a;
    return a > b ? a : b;
}
__device__ __forceinline__ float ieee_min(float a, float b)
{
    if (a != a) return a;
    if (b != b) return b;
    if (a == b) return signbit(a) ? a : b;
    return a < b ? a : b;
}

// BinaryOp.OpS / OpS2 (BinaryOp.cs:309-357). Pow takes the special forms of Apply (:153-196) when the
// exponent is one value along the reference's innermost dim (pow_special), else powf.
__device__ __forceinline__ float binary_op(int op, float a, float b, bool pow_special)
{
    switch (op) {
    case SLHIP_BIN_ADD: return a + b;
    case SLHIP_BIN_SUB: return a - b;
    case SLHIP_BIN_MUL: return a * b;
    case SLHIP_BIN_DIV: return a / b;
    case SLHIP_BIN_MAX: return ieee_max(a, b);
    case SLHIP_BIN_MIN: return ieee_min(a, b);
    case SLHIP_BIN_POW:
        if (!pow_special) return powf(a, b);
        if (b == 2.0f) return a * a;
        if (b == 1.0f) return a;
        if (b == 0.5f) return sqrtf(a);
        if (b == 3.0f) return a * a * a;
        return powf(a, b);
    case SLHIP_BIN_MOD: {  // Python-style: the sign of the divisor
        float r = fmodf(a, b);
        if (r != 0.0f && (r < 0.0f) != (b < 0.0f)) r += b;
        return r;
    }
    case SLHIP_BIN_FMOD: return fmodf(a, b);  // C fmod: the sign of the dividend
    case SLHIP_BIN_PRELU: return a < 0.0f ? a * b : a;
    case SLHIP_BIN_EQUAL: return a == b ? 1.0f : 0.0f;
    case SLHIP_BIN_NOT_EQUAL: return a != b ? 1.0f : 0.0f;
    case SLHIP_BIN_LESS: return a < b ? 1.0f : 0.0f;
    case SLHIP_BIN_LESS_EQUAL: return a <= b ? 1.0f : 0.0f;
    case SLHIP_BIN_GREATER: return a > b ? 1.0f : 0.0f;
    case SLHIP_BIN_GREATER_EQUAL: return a >= b ? 1.0f : 0.0f;
    case SLHIP_BIN_AND: return a != 0.0f && b != 0.0f ? 1.0f : 0.0f;
    case SLHIP_BIN_OR: return a != 0.0f || b != 0.0f ? 1.0f : 0.0f;
    case SLHIP_BIN_XOR: return (a != 0.0f) != (b != 0.0f) ? 1.0f : 0.0f;
    default: return atan2f(a, b);  // SLHIP_BIN_ATAN2
    }
}

// log(1 + exp(v)) in f64 for v <= 20, v above (ScalarMath.cs:643-650; the Mish term at :279-284).
__device__ __forceinline__ float softplus(float v) { return v > 20.0f ? v : static_cast<float>(log(1.0 + exp(static_cast<double>(v)))); }

// ScalarMath.Unary (ScalarMath.cs:173-650): the vector-loop forms where the reference has one.
__device__ __forceinline__ float unary_op(int op, float v, float p0, float p1)
{
    switch (op) {
    case SLHIP_UN_NEG: return -v;
    case SLHIP_UN_EXP: return expf(v);
    case SLHIP_UN_LOG: return logf(v);
    case SLHIP_UN_SQRT: return sqrtf(v);
    case SLHIP_UN_RSQRT: return 1.0f / sqrtf(v);
    case SLHIP_UN_SIGMOID: return 1.0f / (1.0f + expf(-v));
    case SLHIP_UN_SILU: return v / (1.0f + expf(-v));
    case SLHIP_UN_GELU: return activate<SLHIP_ACT_GELU_ERF>(v);
    case SLHIP_UN_GELU_TANH: {
        const float u = (0.7978845608028654f * 2.0f) * fmaf(0.044715f * v, v * v, v);
        return v / (1.0f + expf(-u));
    }
    case SLHIP_UN_TANH: return tanhf(v);
    case SLHIP_UN_SOFTPLUS: return softplus(v);
    case SLHIP_UN_RELU: return v > 0.0f ? v : 0.0f;
    case SLHIP_UN_ABS: return fabsf(v);
    case SLHIP_UN_SQUARE: return v * v;
    case SLHIP_UN_RECIP: return 1.0f / v;
    case SLHIP_UN_SCALE: return fmaf(v, p0, p1);
    case SLHIP_UN_ERF: return v != v ? v : erf_rational(v);
    case SLHIP_UN_HARD_SWISH: return v * ieee_min(ieee_max(fmaf(v, 1.0f / 6.0f, 0.5f), 0.0f), 1.0f);
    case SLHIP_UN_HARD_SIGMOID: return ieee_min(ieee_max(fmaf(v, p0, p1), 0.0f), 1.0f);
    case SLHIP_UN_CLIP: return ieee_min(ieee_max(v, p0), p1);
    case SLHIP_UN_SIN: return sinf(v);
    case SLHIP_UN_COS: return cosf(v);
    case SLHIP_UN_TAN: return tanf(v);
    case SLHIP_UN_ASIN: return asinf(v);
    case SLHIP_UN_ACOS: return acosf(v);
    case SLHIP_UN_ATAN: return atanf(v);
    case SLHIP_UN_SINH: return sinhf(v);
    case SLHIP_UN_COSH: return coshf(v);
    case SLHIP_UN_ASINH: return asinhf(v);
    case SLHIP_UN_ACOSH: return acoshf(v);
    case SLHIP_UN_ATANH: return atanhf(v);
    case SLHIP_UN_FLOOR: return floorf(v);
    case SLHIP_UN_CEIL: return ceilf(v);
    case SLHIP_UN_ROUND: return rintf(v);  // half to even
    case SLHIP_UN_SIGN: return v > 0.0f ? 1.0f : v < 0.0f ? -1.0f : v;
    case SLHIP_UN_SOFTSIGN: return v / (1.0f + fabsf(v));
    case SLHIP_UN_MISH: return v * tanhf(softplus(v));
    case SLHIP_UN_ELU: return v >= 0.0f ? v : p0 * (expf(v) - 1.0f);
    case SLHIP_UN_CELU: return ieee_max(0.0f, v) + ieee_min(0.0f, p0 * (expf(v / p0) - 1.0f));
    case SLHIP_UN_SELU: return v > 0.0f ? p1 * v : p1 * p0 * (expf(v) - 1.0f);
    case SLHIP_UN_LEAKY_RELU: return v >= 0.0f ? v : p0 * v;
    case SLHIP_UN_THRESHOLDED_RELU: return v > p0 ? v : 0.0f;
    case SLHIP_UN_NOT: return v != 0.0f ? 0.0f : 1.0f;
    case SLHIP_UN_IS_NAN: return v != v ? 1.0f : 0.0f;
    default: return isinf(v) ? 1.0f : 0.0f;  // SLHIP_UN_IS_INF
    }
}

}  // namespace slhip
