/*
 * CPU oracle for the Sharplight fused layer ops -- TEST INFRASTRUCTURE ONLY (see sl_oracle.h).
 *
 * Every function restates the arithmetic of the reference's CPU provider and cites the
 * reference file:line it follows (paths relative to the reference repository root). The
 * restatement keeps the reference's operation order where it is visible in the source
 * (accumulator layout of the SIMD reductions, which products are fused, f64 where the
 * reference uses f64); the .NET runtime's own Exp/Cos/Sin polynomials are not in the
 * reference's sources, so libm stands in for them (agreement is to tolerance, not bits).
 *
 * Built with -ffp-contract=off so that only the fmaf() calls written below are fused.
 */
#include "sl_oracle.h"

#include <math.h>

#include "../sharplight_amd/csrc/iq_grids.h" /* ggml's lattice tables: data of the grid IQ formats */
#include "../sharplight_amd/csrc/trellis_codebook.h" /* the trellis formats' codebook: data of the formats */
#include <pthread.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------------------------ */
/* conversions                                                                                */
/* ------------------------------------------------------------------------------------------ */

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* Simd.FloatToBFloat (src/Sharplight.Cpu/Simd.cs:530-540): NaN keeps its top half with the quiet
 * bit set; everything else rounds to nearest even by adding 0x7FFF + lsb. */
uint16_t orc_f32_to_bf16(float f)
{
    uint32_t b = f2u(f);
    if ((b & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((b >> 16) | 0x40u);
    b += 0x7FFFu + ((b >> 16) & 1u);
    return (uint16_t)(b >> 16);
}

/* Simd.BFloatToFloat (Simd.cs:527-528). */
float orc_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

/* Quant.H (src/Sharplight.Cpu/Quant.cs:371-381) for normal codes; zero, subnormal, inf and NaN
 * go through the IEEE half->single conversion (Simd.HalfToFloat, Simd.cs:518), restated here
 * from the binary16 definition: a subnormal m*2^-24 is renormalised, inf/NaN keep the payload. */
float orc_f16_to_f32(uint16_t hh)
{
    uint32_t h = hh;
    uint32_t sign = (h & 0x8000u) << 16;
    uint32_t e = h & 0x7C00u;
    uint32_t m = h & 0x03FFu;
    if (e != 0 && e != 0x7C00u) return u2f(sign | (((h & 0x7FFFu) << 13) + 0x38000000u));
    if (e == 0x7C00u) return u2f(sign | 0x7F800000u | (m << 13));
    if (m == 0) return u2f(sign);
    /* subnormal: value = m * 2^-24, exact in f32 */
    int shift = 0;
    while ((m & 0x0400u) == 0) { m <<= 1; shift++; }
    m &= 0x03FFu;
    uint32_t exp = (uint32_t)(127 - 15 - shift + 1);
    return u2f(sign | (exp << 23) | (m << 13));
}

void orc_f32_to_bf16_n(const float* x, uint16_t* y, int64_t n)
{
    for (int64_t i = 0; i < n; i++) y[i] = orc_f32_to_bf16(x[i]);
}

void orc_bf16_to_f32_n(const uint16_t* x, float* y, int64_t n)
{
    for (int64_t i = 0; i < n; i++) y[i] = orc_bf16_to_f32(x[i]);
}

void orc_f16_to_f32_n(const uint16_t* x, float* y, int64_t n)
{
    for (int64_t i = 0; i < n; i++) y[i] = orc_f16_to_f32(x[i]);
}

/* ------------------------------------------------------------------------------------------ */
/* reductions                                                                                 */
/* ------------------------------------------------------------------------------------------ */

/* Horizontal sum of a vector register, pairwise halving (the lane order of Vector512/256.Sum is
 * the runtime's; pairwise is what its x86 lowering does). */
static float hsum(const float* v, int lanes)
{
    float t[16];
    for (int i = 0; i < lanes; i++) t[i] = v[i];
    for (int w = lanes / 2; w >= 1; w /= 2)
        for (int i = 0; i < w; i++) t[i] = t[i] + t[i + w];
    return t[0];
}

/* Simd.SumSq, AVX-512 tier (src/Sharplight.Cpu/Simd.cs:274-317): two 16-lane FMA accumulators
 * over 32 elements per step, one more 16-lane step, Sum(s0+s1), then a scalar tail. */
float orc_sumsq(const float* a, int64_t n)
{
    int64_t i = 0;
    float s0[16] = {0}, s1[16] = {0};
    for (; i + 32 <= n; i += 32)
        for (int j = 0; j < 16; j++) {
            s0[j] = fmaf(a[i + j], a[i + j], s0[j]);
            s1[j] = fmaf(a[i + 16 + j], a[i + 16 + j], s1[j]);
        }
    for (; i + 16 <= n; i += 16)
        for (int j = 0; j < 16; j++) s0[j] = fmaf(a[i + j], a[i + j], s0[j]);
    float s[16];
    for (int j = 0; j < 16; j++) s[j] = s0[j] + s1[j];
    float sum = hsum(s, 16);
    for (; i < n; i++) sum += a[i] * a[i];
    return sum;
}

/* Simd.Sum, AVX2 tier (Simd.cs:319-340): one 8-lane accumulator, Sum, scalar tail. */
float orc_sum(const float* a, int64_t n)
{
    int64_t i = 0;
    float s[8] = {0};
    for (; i + 8 <= n; i += 8)
        for (int j = 0; j < 8; j++) s[j] += a[i + j];
    float sum = hsum(s, 8);
    for (; i < n; i++) sum += a[i];
    return sum;
}

/* ------------------------------------------------------------------------------------------ */
/* row ops                                                                                    */
/* ------------------------------------------------------------------------------------------ */

/* RowOp.Body, cases RmsNorm and L2Norm (src/Sharplight.Cpu/RowOp.cs:63-84) with Simd.ScaleMul /
 * Simd.Scale (Simd.cs:441-480): scale = 1/sqrt(SumSq/n + eps) (L2: SumSq + eps), y = x*scale*w. */
static void rmsnorm_rows(const float* x, const float* w, float* y, int64_t r0, int64_t r1, int64_t n, float eps,
                         int mode)
{
    for (int64_t r = r0; r < r1; r++) {
        const float* xr = x + r * n;
        float* yr = y + r * n;
        float ss = orc_sumsq(xr, n);
        float scale = mode == 0 ? 1.0f / sqrtf(ss / (float)n + eps) : 1.0f / sqrtf(ss + eps);
        if (w) {
            for (int64_t i = 0; i < n; i++) yr[i] = xr[i] * scale * w[i];
        } else {
            for (int64_t i = 0; i < n; i++) yr[i] = xr[i] * scale;
        }
    }
}

void orc_rmsnorm(const float* x, const float* w, float* y, int64_t rows, int64_t n, float eps, int mode)
{
    rmsnorm_rows(x, w, y, 0, rows, n, eps, mode);
}

/* RowOp.Body, case LayerNorm (RowOp.cs:85-113): mean = Sum(x)/n in f32, variance accumulated in
 * f64 over the f32 differences, inv = 1/sqrt((float)(v/n) + eps), y = ((x-mean)*inv)*w + b. */
static void layernorm_rows(const float* x, const float* w, const float* b, float* y, int64_t r0, int64_t r1, int64_t n,
                           float eps)
{
    for (int64_t r = r0; r < r1; r++) {
        const float* xr = x + r * n;
        float* yr = y + r * n;
        float mean = orc_sum(xr, n) / (float)n;
        double v = 0;
        for (int64_t i = 0; i < n; i++) {
            double d = (double)(xr[i] - mean);
            v += d * d;
        }
        float inv = 1.0f / sqrtf((float)(v / (double)n) + eps);
        for (int64_t i = 0; i < n; i++) {
            float o = (xr[i] - mean) * inv;
            if (w) o *= w[i];
            if (b) o += b[i];
            yr[i] = o;
        }
    }
}

void orc_layernorm(const float* x, const float* w, const float* b, float* y, int64_t rows, int64_t n, float eps)
{
    layernorm_rows(x, w, b, y, 0, rows, n, eps);
}

/* ------------------------------------------------------------------------------------------ */
/* elementwise                                                                                */
/* ------------------------------------------------------------------------------------------ */

/* BinaryOp Add / Mul on dense equal-shape operands (src/Sharplight.Cpu/BinaryOp.cs:60-103). */
void orc_add(const float* a, const float* b, float* y, int64_t n)
{
    for (int64_t i = 0; i < n; i++) y[i] = a[i] + b[i];
}

void orc_mul(const float* a, const float* b, float* y, int64_t n)
{
    for (int64_t i = 0; i < n; i++) y[i] = a[i] * b[i];
}

/* ScalarMath.Erf (src/Sharplight.Cpu/ScalarMath.cs:11-49): f64 series below 2.5, continued
 * fraction for erfc up to 6, 1 beyond. */
double orc_erf(double x)
{
    double ax = fabs(x), r;
    if (ax < 2.5) {
        double x2 = ax * ax, term = ax, sum = ax;
        for (int k = 1; k < 200; k++) {
            term *= 2 * x2 / (2 * k + 1);
            sum += term;
            if (term < sum * 1e-17) break;
        }
        r = 1.1283791670955126 * exp(-x2) * sum;
    } else if (ax > 6) {
        r = 1.0;
    } else {
        double f = ax;
        for (int k = 80; k >= 1; k--) f = ax + 0.5 * k / f;
        r = 1.0 - exp(-ax * ax) / (1.7724538509055159 * f);
    }
    return x < 0 ? -r : r;
}

/* ScalarMath.ErfD / ErfV (ScalarMath.cs:51-98): the Eigen/XLA rational erf evaluated in f64 on
 * the argument clamped to +-3.8325, narrowed to f32. The coefficients are the published ones of
 * that approximation (Eigen's generic_fast_erf_float). */
float orc_erf_rational(float xf)
{
    const double clampv = (double)3.832506856900711f;
    const double A1 = -1.60960333262415e-02, A3 = -2.95459980854025e-03, A5 = -7.34990630326855e-04,
                 A7 = -5.69250639462346e-05, A9 = -2.10102402082508e-06, A11 = 2.77068142495902e-08,
                 A13 = -2.72614225801306e-10, B0 = -1.42647390514189e-02, B2 = -7.37332916720468e-03,
                 B4 = -1.68282697438203e-03, B6 = -2.13374055278905e-04, B8 = -1.45660718464996e-05;
    double x = (double)xf;
    if (x < -clampv) x = -clampv;
    if (x > clampv) x = clampv;
    double x2 = x * x;
    double p = A13;
    p = fma(p, x2, A11);
    p = fma(p, x2, A9);
    p = fma(p, x2, A7);
    p = fma(p, x2, A5);
    p = fma(p, x2, A3);
    p = fma(p, x2, A1);
    p *= x;
    double q = B8;
    q = fma(q, x2, B6);
    q = fma(q, x2, B4);
    q = fma(q, x2, B2);
    q = fma(q, x2, B0);
    return (float)(p / q);
}

/* ScalarMath.Unary (ScalarMath.cs:552-641) over one contiguous range, AVX2 tier: the vector form
 * on whole groups of 8, the scalar form on the tail.
 *   Silu     (552-584): v / (1 + exp(-v)) in both forms.
 *   GeluTanh (593-623): vector v / (1 + exp(-u)), u = 2*0.79788456*fma(0.044715*v, v*v, v);
 *                       tail 0.5*v*(1 + tanh(0.79788456*(v + 0.044715*v^3))).
 *   Gelu     (625-641): vector 0.5*v*(1 + erf_rational(v/sqrt2)); tail in f64 with the series erf. */
static void unary_range(int act, const float* x, float* y, int64_t n)
{
    int64_t vec = n - n % 8;
    int64_t i = 0;
    switch (act) {
    case 0:
        for (; i < n; i++) y[i] = x[i] / (1.0f + expf(-x[i]));
        break;
    case 1: {
        const float c0 = 0.7978845608028654f * 2.0f, c1 = 0.044715f;
        for (; i < vec; i++) {
            float v = x[i];
            float u = c0 * fmaf(c1 * v, v * v, v);
            y[i] = v / (1.0f + expf(-u));
        }
        for (; i < n; i++) {
            float v = x[i];
            y[i] = 0.5f * v * (1.0f + tanhf(0.7978845608028654f * (v + 0.044715f * v * v * v)));
        }
        break;
    }
    case 2:
        for (; i < vec; i++) {
            float v = x[i];
            y[i] = 0.5f * v * (1.0f + orc_erf_rational(v * 0.7071067811865476f));
        }
        for (; i < n; i++) {
            double v = x[i];
            y[i] = (float)(0.5 * v * (1.0 + orc_erf(v * 0.7071067811865476)));
        }
        break;
    default:
        break;
    }
}

void orc_unary(int act, const float* x, float* y, int64_t n) { unary_range(act, x, y, n); }

/* The reference's UnaryKind (src/Sharplight.Cpu/UnaryKind.cs:4-6), numbered as declared there. */
enum { U_NEG, U_EXP, U_LOG, U_SQRT, U_RSQRT, U_SIGMOID, U_SILU, U_GELU, U_GELU_TANH, U_TANH, U_SOFTPLUS, U_RELU,
       U_ABS, U_SQUARE, U_RECIP, U_SCALE, U_ERF, U_HARD_SWISH, U_HARD_SIGMOID, U_CLIP, U_SIN, U_COS, U_TAN, U_ASIN,
       U_ACOS, U_ATAN, U_SINH, U_COSH, U_ASINH, U_ACOSH, U_ATANH, U_FLOOR, U_CEIL, U_ROUND, U_SIGN, U_SOFTSIGN,
       U_MISH, U_ELU, U_CELU, U_SELU, U_LEAKY_RELU, U_THRESHOLDED_RELU, U_NOT, U_IS_NAN, U_IS_INF };

/* MathF.Max / MathF.Min and the Vector*.Max/Min of .NET (IEEE 754-2019 maximum/minimum): NaN if
 * either operand is NaN, +0 above -0. */
static float net_max(float a, float b)
{
    if (a != a) return a;
    if (b != b) return b;
    if (a == b) return signbit(a) ? b : a;
    return a > b ? a : b;
}
static float net_min(float a, float b)
{
    if (a != a) return a;
    if (b != b) return b;
    if (a == b) return signbit(a) ? a : b;
    return a < b ? a : b;
}

/* Softplus (ScalarMath.cs:643-650) and the Mish term (:279-284): log(1 + exp(v)) in f64 up to 20. */
static float softplus(float v) { return v > 20.0f ? v : (float)log(1.0 + exp((double)v)); }

/* ScalarMath.Unary (src/Sharplight.Cpu/ScalarMath.cs:173-650) on one contiguous range, AVX2 tier
 * (CpuIsa.Use256): the kinds with a Vector256 loop take its form on whole groups of 8 from the start of
 * the range and the scalar form on the rest; the others are scalar throughout. Forms that differ:
 *   HardSwish   (349-370): vector v*min(max(fma(v, 1/6, 0.5), 0), 1); tail v*clamp(v*(1/6) + 0.5, 0, 1)
 *   HardSigmoid (371-387): vector min(max(fma(v, a, b), 0), 1);       tail clamp(v*a + b, 0, 1)
 *   Scale       (460-484): vector fma(v, s, b);                       tail v*s + b
 *   GeluTanh, Gelu as unary_range above; Silu, Sigmoid and Exp have one form (.NET's Vector Exp against
 *   MathF.Exp: libm stands in for both). */
void orc_unary_kind(int kind, const float* x, float* y, int64_t n, float p0, float p1)
{
    const int64_t vec = n - n % 8;
    int64_t i = 0;
    switch (kind) {
    case U_SILU: unary_range(0, x, y, n); return;
    case U_GELU_TANH: unary_range(1, x, y, n); return;
    case U_GELU: unary_range(2, x, y, n); return;
    case U_HARD_SWISH:
        for (; i < vec; i++) y[i] = x[i] * net_min(net_max(fmaf(x[i], 1.0f / 6.0f, 0.5f), 0.0f), 1.0f);
        for (; i < n; i++) {
            float c = x[i] * (1.0f / 6.0f) + 0.5f;  /* Math.Clamp(v, 0, 1): v < 0 -> 0, v > 1 -> 1, else v */
            y[i] = x[i] * (c < 0.0f ? 0.0f : c > 1.0f ? 1.0f : c);
        }
        return;
    case U_HARD_SIGMOID:
        for (; i < vec; i++) y[i] = net_min(net_max(fmaf(x[i], p0, p1), 0.0f), 1.0f);
        for (; i < n; i++) {
            float c = x[i] * p0 + p1;
            y[i] = c < 0.0f ? 0.0f : c > 1.0f ? 1.0f : c;
        }
        return;
    case U_SCALE:
        for (; i < vec; i++) y[i] = fmaf(x[i], p0, p1);
        for (; i < n; i++) y[i] = x[i] * p0 + p1;
        return;
    case U_ERF: /* vector: the f64 rational (ErfV); tail ErfF, the same rational with separate mul/add */
        for (; i < vec; i++) y[i] = orc_erf_rational(x[i]);
        for (; i < n; i++) {
            const double A1 = -1.60960333262415e-02, A3 = -2.95459980854025e-03, A5 = -7.34990630326855e-04,
                         A7 = -5.69250639462346e-05, A9 = -2.10102402082508e-06, A11 = 2.77068142495902e-08,
                         A13 = -2.72614225801306e-10, B0 = -1.42647390514189e-02, B2 = -7.37332916720468e-03,
                         B4 = -1.68282697438203e-03, B6 = -2.13374055278905e-04, B8 = -1.45660718464996e-05;
            const double c = (double)3.832506856900711f;
            double v = x[i];
            v = v < -c ? -c : v > c ? c : v;
            double x2 = v * v;
            double pp = ((((((A13 * x2 + A11) * x2 + A9) * x2 + A7) * x2 + A5) * x2 + A3) * x2 + A1) * v;
            double q = ((((B8 * x2 + B6) * x2 + B4) * x2 + B2) * x2 + B0);
            y[i] = (float)(pp / q);
        }
        return;
    default: break;
    }
    for (; i < n; i++) {
        const float v = x[i];
        float r;
        switch (kind) {
        case U_NEG: r = -v; break;
        case U_EXP: r = expf(v); break;
        case U_LOG: r = logf(v); break;
        case U_SQRT: r = sqrtf(v); break;
        case U_RSQRT: r = 1.0f / sqrtf(v); break;
        case U_SIGMOID: r = 1.0f / (1.0f + expf(-v)); break;
        case U_TANH: r = tanhf(v); break;
        case U_SOFTPLUS: r = softplus(v); break;
        case U_RELU: r = v > 0 ? v : 0.0f; break;
        case U_ABS: r = fabsf(v); break;
        case U_SQUARE: r = v * v; break;
        case U_RECIP: r = 1.0f / v; break;
        case U_CLIP: r = net_min(net_max(v, p0), p1); break; /* Vector256.Min(Max(v, lo), hi) (:388-410) */
        case U_SIN: r = sinf(v); break;
        case U_COS: r = cosf(v); break;
        case U_TAN: r = tanf(v); break;
        case U_ASIN: r = asinf(v); break;
        case U_ACOS: r = acosf(v); break;
        case U_ATAN: r = atanf(v); break;
        case U_SINH: r = sinhf(v); break;
        case U_COSH: r = coshf(v); break;
        case U_ASINH: r = asinhf(v); break;
        case U_ACOSH: r = acoshf(v); break;
        case U_ATANH: r = atanhf(v); break;
        case U_FLOOR: r = floorf(v); break;
        case U_CEIL: r = ceilf(v); break;
        case U_ROUND: r = rintf(v); break; /* MidpointRounding.ToEven under the default rounding mode */
        case U_SIGN: r = v > 0 ? 1.0f : v < 0 ? -1.0f : v; break;
        case U_SOFTSIGN: r = v / (1.0f + fabsf(v)); break;
        case U_MISH: r = v * tanhf(softplus(v)); break;
        case U_ELU: r = v >= 0 ? v : p0 * (expf(v) - 1.0f); break;
        case U_CELU: r = net_max(0.0f, v) + net_min(0.0f, p0 * (expf(v / p0) - 1.0f)); break;
        case U_SELU: r = v > 0 ? p1 * v : p1 * p0 * (expf(v) - 1.0f); break;
        case U_LEAKY_RELU: r = v >= 0 ? v : p0 * v; break;
        case U_THRESHOLDED_RELU: r = v > p0 ? v : 0.0f; break;
        case U_NOT: r = v != 0 ? 0.0f : 1.0f; break;
        case U_IS_NAN: r = v != v ? 1.0f : 0.0f; break;
        default: r = isinf(v) ? 1.0f : 0.0f; break;
        }
        y[i] = r;
    }
}

/* BinaryKind (src/Sharplight.Cpu/BinaryKind.cs:4), then Mod with fmod = true. */
enum { B_ADD, B_SUB, B_MUL, B_DIV, B_MAX, B_MIN, B_POW, B_MOD, B_PRELU, B_EQ, B_NE, B_LT, B_LE, B_GT, B_GE, B_AND,
       B_OR, B_XOR, B_ATAN2, B_FMOD };

/* BinaryOp.OpS / OpS2 (BinaryOp.cs:309-357). */
static float binary_scalar(int k, float a, float b)
{
    switch (k) {
    case B_ADD: return a + b;
    case B_SUB: return a - b;
    case B_MUL: return a * b;
    case B_DIV: return a / b;
    case B_MAX: return net_max(a, b);
    case B_MIN: return net_min(a, b);
    case B_POW: return powf(a, b);
    case B_MOD:
    case B_FMOD: {
        float r = fmodf(a, b);
        if (k == B_MOD && r != 0 && (r < 0) != (b < 0)) r += b;
        return r;
    }
    case B_PRELU: return a < 0 ? a * b : a;
    case B_EQ: return a == b ? 1.0f : 0.0f;
    case B_NE: return a != b ? 1.0f : 0.0f;
    case B_LT: return a < b ? 1.0f : 0.0f;
    case B_LE: return a <= b ? 1.0f : 0.0f;
    case B_GT: return a > b ? 1.0f : 0.0f;
    case B_GE: return a >= b ? 1.0f : 0.0f;
    case B_AND: return a != 0 && b != 0 ? 1.0f : 0.0f;
    case B_OR: return a != 0 || b != 0 ? 1.0f : 0.0f;
    case B_XOR: return (a != 0) != (b != 0) ? 1.0f : 0.0f;
    default: return atan2f(a, b);
    }
}

/* BinaryOp.Apply (BinaryOp.cs:141-275) on one row of n outputs: Pow with a row-constant exponent (sb == 0)
 * takes the forms for 2, 1, 0.5 and 3 (:153-196); the vector loops compute what the scalar ops do. */
static void binary_row(int k, const float* a, int64_t sa, const float* b, int64_t sb, float* y, int64_t n)
{
    if (k == B_POW && sb == 0) {
        const float e = *b;
        for (int64_t i = 0; i < n; i++) {
            const float v = a[i * sa];
            y[i] = e == 2.0f ? v * v : e == 1.0f ? v : e == 0.5f ? sqrtf(v) : e == 3.0f ? v * v * v : powf(v, e);
        }
        return;
    }
    for (int64_t i = 0; i < n; i++) y[i] = binary_scalar(k, a[i * sa], b[i * sb]);
}

/* BinaryOp.Align (BinaryOp.cs:37-58): a's strides against y's rank; a dim of extent 1 or a missing
 * leading dim gets stride 0. a_dims/a_rank describe a dense operand. */
void orc_align(const int64_t* a_dims, int a_rank, int y_rank, int64_t* strides)
{
    int64_t dense[16];
    int64_t acc = 1;
    for (int k = a_rank - 1; k >= 0; k--) {
        dense[k] = acc;
        acc *= a_dims[k];
    }
    for (int k = 0; k < y_rank; k++) {
        const int ik = k - (y_rank - a_rank);
        strides[k] = ik < 0 || a_dims[ik] == 1 ? 0 : dense[ik];
    }
}

/* BinaryOp.Run + Body (BinaryOp.cs:60-139): y dense [dims], a and b by aligned strides. Rows of the
 * innermost dim (the trailing merge changes only the loop bounds, not the values); rank 0 is one element. */
void orc_binary(int k, const float* a, const int64_t* sa, const float* b, const int64_t* sb, float* y,
                const int64_t* dims, int rank)
{
    if (rank == 0) {
        binary_row(k, a, 0, b, 0, y, 1);
        return;
    }
    int64_t total = 1;
    for (int d = 0; d < rank; d++) total *= dims[d];
    if (total == 0) return;
    const int64_t l = dims[rank - 1];
    for (int64_t r = 0; r < total / l; r++) {
        int64_t ao = 0, bo = 0, rr = r;
        for (int d = rank - 2; d >= 0; d--) {
            const int64_t q = rr / dims[d], ix = rr - q * dims[d];
            rr = q;
            ao += ix * sa[d];
            bo += ix * sb[d];
        }
        binary_row(k, a + ao, sa[rank - 1], b + bo, sb[rank - 1], y + r * l, l);
    }
}

/* ------------------------------------------------------------------------------------------ */
/* rope                                                                                       */
/* ------------------------------------------------------------------------------------------ */

/* RopeOp.AxisOf (src/Sharplight.Cpu/RopeOp.cs:70-106): the position axis of pair section i under llama.cpp's
 * M-RoPE sector rules; 0 without sections (all of sections[0..2] zero). */
int orc_rope_axis_of(int i, const int32_t* sec, int interleaved)
{
    if (!sec || !(sec[0] > 0 || sec[1] > 0 || sec[2] > 0)) return 0;
    int sect_dims = sec[0] + sec[1] + sec[2] + sec[3];
    int sector = i % sect_dims;
    if (interleaved) {
        if (sector % 3 == 1 && sector < 3 * sec[1]) return 1;
        if (sector % 3 == 2 && sector < 3 * sec[2]) return 2;
        return sector % 3 == 0 && sector < 3 * sec[0] ? 0 : 3;
    }
    if (sector < sec[0]) return 0;
    if (sector < sec[0] + sec[1]) return 1;
    return sector < sec[0] + sec[1] + sec[2] ? 2 : 3;
}

/* RopeOp (src/Sharplight.Cpu/RopeOp.cs): inverse frequencies in f64 (ctor, :47-52); per pair the axes of its
 * first and second element (:54-66: with per-element sections element e takes the axis of pair section e/2);
 * per token the positions of 4 axes, a missing axis taking axis 0 when there is one axis, else 0 (:133-139);
 * theta = pos[axis] * invFreq (/ ff[i]) in f64, cos/sin narrowed to f32 then times attn_factor (:141-154);
 * neox pairs (i, i+half), normal pairs (2i, 2i+1): y0 = x0*c1 - x1*s1, y1 = x0*s2 + x1*c2 (:155-176);
 * elements from dims to D are copied (:177-180). pos [T, axes] dense. */
static void rope_tokens(const float* x, const int32_t* pos, int axes, const int32_t* sec, int interleaved,
                        int per_element, const float* ff, float* y, int64_t t0, int64_t t1, int64_t H, int64_t D,
                        int dims, int neox, float base, float freq_scale, float attn_factor)
{
    int half = dims / 2;
    size_t hn = (size_t)(half > 0 ? half : 1);
    double* inv = (double*)malloc(sizeof(double) * hn);
    float* cs = (float*)malloc(sizeof(float) * hn * 4);
    int* ax1 = (int*)malloc(sizeof(int) * hn);
    int* ax2 = (int*)malloc(sizeof(int) * hn);
    for (int i = 0; i < half; i++) {
        inv[i] = pow((double)base, -2.0 * i / dims) * (double)freq_scale;
        int first = neox ? i : 2 * i, second = neox ? i + half : 2 * i + 1;
        ax1[i] = orc_rope_axis_of(per_element ? first / 2 : i, sec, interleaved);
        ax2[i] = orc_rope_axis_of(per_element ? second / 2 : i, sec, interleaved);
    }
    for (int64_t t = t0; t < t1; t++) {
        double pp[4];
        for (int a = 0; a < 4; a++) pp[a] = a < axes ? (double)pos[t * axes + a] : (axes == 1 ? (double)pos[t * axes] : 0.0);
        for (int i = 0; i < half; i++) {
            double theta = pp[ax1[i]] * inv[i], theta2 = pp[ax2[i]] * inv[i];
            if (ff) {
                theta /= (double)ff[i];
                theta2 /= (double)ff[i];
            }
            cs[4 * i] = (float)cos(theta) * attn_factor;
            cs[4 * i + 1] = (float)sin(theta) * attn_factor;
            cs[4 * i + 2] = (float)cos(theta2) * attn_factor;
            cs[4 * i + 3] = (float)sin(theta2) * attn_factor;
        }
        for (int64_t h = 0; h < H; h++) {
            const float* xr = x + (t * H + h) * D;
            float* yr = y + (t * H + h) * D;
            for (int i = 0; i < half; i++) {
                int i0 = neox ? i : 2 * i;
                int i1 = neox ? i + half : 2 * i + 1;
                float x0 = xr[i0], x1 = xr[i1];
                yr[i0] = x0 * cs[4 * i] - x1 * cs[4 * i + 1];
                yr[i1] = x0 * cs[4 * i + 3] + x1 * cs[4 * i + 2];
            }
            for (int64_t i = dims; i < D; i++) yr[i] = xr[i];
        }
    }
    free(inv);
    free(cs);
    free(ax1);
    free(ax2);
}

void orc_rope(const float* x, const int32_t* pos, const float* ff, float* y, int64_t T, int64_t H, int64_t D, int dims,
              int neox, float base, float freq_scale, float attn_factor)
{
    rope_tokens(x, pos, 1, NULL, 0, 0, ff, y, 0, T, H, D, dims, neox, base, freq_scale, attn_factor);
}

void orc_rope_multi(const float* x, const int32_t* pos, int axes, const int32_t* sections, int interleaved,
                    int per_element, const float* ff, float* y, int64_t T, int64_t H, int64_t D, int dims, int neox,
                    float base, float freq_scale, float attn_factor)
{
    rope_tokens(x, pos, axes, sections, interleaved, per_element, ff, y, 0, T, H, D, dims, neox, base, freq_scale,
                attn_factor);
}

/* ------------------------------------------------------------------------------------------ */
/* dequant / gather                                                                           */
/* ------------------------------------------------------------------------------------------ */

/* Quant.BlockSize / BlockBytes (src/Sharplight.Cpu/Quant.cs:181-216) for the formats here. */
static int block_size(int fmt)
{
    switch (fmt) {  /* the reference's own formats (Quant.BlockSize, Quant.cs:181-198) */
    case ORC_Q1_0: case ORC_Q2_0_G128: case ORC_TERN1_G128: case ORC_Q2S_G128: case ORC_Q4Z_G128: case ORC_Q8Z_G128:
    case ORC_F8E4M3_B128: return 128;
    case ORC_TRELLIS_V4K8: case ORC_TRELLIS_V4K6: case ORC_TRELLIS_V4K7: case ORC_TRELLIS_V2K5: case ORC_TRELLIS_V2K6:
    case ORC_TRELLIS_V2K7: return 128;
    case ORC_Q2_0: case ORC_NVFP4_GS: case ORC_NF4_B64: case ORC_FP4_B64: return 64;
    case ORC_Q4Z_G32: case ORC_Q8Z_G32: case ORC_Q8A_G32: case ORC_F8E4M3_B32: return 32;
    case ORC_F8E4M3: case ORC_F8E5M2: return 1;
    default: break;
    }
    if (fmt == ORC_IQ4_NL || fmt == ORC_MXFP4) return 32;
    if (fmt == ORC_NVFP4) return 64;
    if (fmt >= ORC_Q2_K) return 256;
    return fmt >= ORC_Q8_0 ? 32 : 1;
}
static int block_bytes(int fmt)
{
    switch (fmt) {
    case ORC_F32: return 4;
    case ORC_F16: case ORC_BF16: return 2;
    case ORC_Q8_0: return 34;
    case ORC_Q4_0: return 18;
    case ORC_Q4_1: return 20;
    case ORC_Q5_0: return 22;
    case ORC_Q5_1: return 24;
    case ORC_Q2_K: return 84;
    case ORC_Q3_K: return 110;
    case ORC_Q4_K: return 144;
    case ORC_Q5_K: return 176;
    case ORC_Q6_K: return 210;
    case ORC_IQ4_NL: return 18;
    case ORC_IQ4_XS: return 136;
    case ORC_TQ1_0: return 54;
    case ORC_TQ2_0: return 66;
    case ORC_MXFP4: return 17;
    case ORC_NVFP4: return 36;
    case ORC_IQ2_XXS: return 66;
    case ORC_IQ2_XS: return 74;
    case ORC_IQ2_S: return 82;
    case ORC_IQ3_XXS: return 98;
    case ORC_IQ3_S: return 110;
    case ORC_IQ1_S: return 50;
    case ORC_IQ1_M: return 56;
    /* Quant.BlockBytes (Quant.cs:200-238) */
    case ORC_Q1_0: case ORC_Q2_0: return 18;
    case ORC_Q2_0_G128: return 34;
    case ORC_TERN1_G128: return 28;
    case ORC_NVFP4_GS: return 40;
    case ORC_Q4Z_G32: return 20;
    case ORC_Q4Z_G128: return 68;
    case ORC_Q8Z_G32: case ORC_NF4_B64: case ORC_FP4_B64: case ORC_Q8A_G32: case ORC_Q2S_G128: case ORC_F8E4M3_B32: return 36;
    case ORC_Q8Z_G128: case ORC_F8E4M3_B128: return 132;
    case ORC_F8E4M3: case ORC_F8E5M2: return 1;
    /* DataType.TrellisV4K8_G128 .. TrellisV2K7_G128 (DataType.cs:212-223): 2 + steps * bits / 8 */
    case ORC_TRELLIS_V4K8: return 34;
    case ORC_TRELLIS_V4K6: return 26;
    case ORC_TRELLIS_V4K7: return 30;
    case ORC_TRELLIS_V2K5: return 42;
    case ORC_TRELLIS_V2K6: return 50;
    case ORC_TRELLIS_V2K7: return 58;
    default: return -1;
    }
}

int64_t orc_row_bytes(int fmt, int64_t d)
{
    int bb = block_bytes(fmt);
    if (bb < 0 || d % block_size(fmt) != 0) return -1;
    return d / block_size(fmt) * bb;
}

static inline float rd_h(const uint8_t* p) { return orc_f16_to_f32((uint16_t)(p[0] | (p[1] << 8))); }

/* ---- K-quants and the 4-bit codebook formats ---- */

/* Quant.ScaleMin (Quant.cs:502-516): the 6-bit scale and minimum j (0..7) of the 12 packed bytes q. */
static void scale_min(int j, const uint8_t* q, int* sc, int* m)
{
    if (j < 4) {
        *sc = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *sc = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
        *m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

/* The IQ4_NL / IQ4_XS codebook (Quant.cs:409), the values ggml's non-linear 4-bit formats define. */
static const int8_t kIq4Values[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};

/* Quant.s_fp4Values (Quant.Fp4.cs:10): the E2M1 magnitudes doubled, codes 8..15 negative. */
static const int8_t kFp4Values[16] = {0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12};

/* Quant.E8M0Half (Quant.Fp4.cs:36-41): 2^(e-127) / 2, exponents 0 and 1 as f32 denormals. */
static float e8m0_half(uint8_t e)
{
    uint32_t bits = e < 2 ? 0x00200000u << e : (uint32_t)(e - 1) << 23;
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* Quant.BuildUe4m3 (Quant.Fp4.cs:14-33): a UE4M3 byte (exponent bits 3-6, bias 7; mantissa bits 0-2; bit 7
 * ignored) halved; 0 and 0x7F read as zero. */
static float ue4m3_half(uint8_t x)
{
    if (x == 0 || x == 0x7F) return 0.0f;
    const int e = (x >> 3) & 0xF, m = x & 7;
    const float raw = e == 0 ? ldexpf((float)m, -9) : ldexpf(1.0f + (float)m / 8.0f, e - 7);
    return raw * 0.5f;
}

/* Quant.BuildTrits (Quant.Ternary.cs:10-25): base-3 digit n of byte b, ((b * 3^n mod 256) * 3) >> 8, minus one. */
static int trit(uint8_t b, int n)
{
    static const int p3[5] = {1, 3, 9, 27, 81};
    return ((((int)b * p3[n]) & 0xFF) * 3 >> 8) - 1;
}

/* ksigns_iq2xs (IqSigns.cs): a 7-bit index i selects the signs of eight values, bit j set = value j
 * negative, the eighth sign the parity of the other seven: i | parity(i) << 7. */
static int ksign(uint32_t i) { return (int)(i | ((uint32_t)__builtin_parity(i) << 7)); }
static inline uint32_t rd_u32(const uint8_t* p) { uint32_t v; memcpy(&v, p, 4); return v; }
static inline uint32_t rd_u16(const uint8_t* p) { return (uint32_t)p[0] | ((uint32_t)p[1] << 8); }

/* Quant.StoreSigned8 / StoreSigned4x2 (Quant.Iq.cs:99-111): (grid byte * (+-1)) * scale, one rounding. */
static void signed8(const uint8_t* g8, int signs, float scale, float* dst)
{
    for (int j = 0; j < 8; j++) dst[j] = ((float)g8[j] * ((signs >> j) & 1 ? -1.0f : 1.0f)) * scale;
}

/* The grid IQ formats (Quant.Iq.cs:113-306), 256 values per block. */
static void iq_block(int fmt, const uint8_t* p, float* dst)
{
    uint8_t g[8];
    switch (fmt) {
    case ORC_IQ2_XXS: { /* {f16 d; u16 qs[32]}: per 32 values 4 grid indices, then 4 sign indices + scale */
        const float d = rd_h(p);
        for (int ib = 0; ib < 8; ib++, dst += 32) {
            const uint32_t idx = rd_u32(p + 2 + 8 * ib), ss = rd_u32(p + 6 + 8 * ib);
            const float db = d * (0.5f + (float)(ss >> 28)) * 0.25f;
            for (int l = 0; l < 4; l++) {
                memcpy(g, &kIq2xxsGrid[(idx >> (8 * l)) & 0xFF], 8);
                signed8(g, ksign((ss >> (7 * l)) & 127), db, dst + 8 * l);
            }
        }
        break;
    }
    case ORC_IQ2_XS: { /* {f16 d; u16 qs[32]; u8 scales[8]}: 9-bit grid index + 7-bit sign index */
        const float d = rd_h(p);
        for (int ib = 0; ib < 8; ib++, dst += 32) {
            const int sc = p[66 + ib];
            const float db0 = d * (0.5f + (float)(sc & 0xF)) * 0.25f, db1 = d * (0.5f + (float)(sc >> 4)) * 0.25f;
            for (int l = 0; l < 4; l++) {
                const uint32_t q = rd_u16(p + 2 + 2 * (4 * ib + l));
                memcpy(g, &kIq2xsGrid[q & 511], 8);
                signed8(g, ksign(q >> 9), l < 2 ? db0 : db1, dst + 8 * l);
            }
        }
        break;
    }
    case ORC_IQ2_S: { /* {f16 d; qs[64] (low index bits, then sign bytes); qh[8]; scales[8]} */
        const float d = rd_h(p);
        for (int ib = 0; ib < 8; ib++, dst += 32) {
            const int sc = p[74 + ib];
            const float db0 = d * (0.5f + (float)(sc & 0xF)) * 0.25f, db1 = d * (0.5f + (float)(sc >> 4)) * 0.25f;
            for (int l = 0; l < 4; l++) {
                const int index = p[2 + 4 * ib + l] | ((p[66 + ib] << (8 - 2 * l)) & 0x300);
                memcpy(g, &kIq2sGrid[index], 8);
                signed8(g, p[34 + 4 * ib + l], l < 2 ? db0 : db1, dst + 8 * l);
            }
        }
        break;
    }
    case ORC_IQ3_XXS: { /* {f16 d; qs[64] (8-bit indices of 4-value entries); 8 words: 4 sign indices + scale} */
        const float d = rd_h(p);
        for (int ib = 0; ib < 8; ib++, dst += 32) {
            const uint32_t w = rd_u32(p + 66 + 4 * ib);
            const float db = d * (0.5f + (float)(w >> 28)) * 0.5f;
            for (int l = 0; l < 4; l++) {
                memcpy(g, &kIq3xxsGrid[p[2 + 8 * ib + 2 * l]], 4);
                memcpy(g + 4, &kIq3xxsGrid[p[2 + 8 * ib + 2 * l + 1]], 4);
                signed8(g, ksign((w >> (7 * l)) & 127), db, dst + 8 * l);
            }
        }
        break;
    }
    case ORC_IQ3_S: { /* {f16 d; qs[64]; qh[8]; signs[32]; scales[4]}: 9-bit indices, scales 1 + 2s */
        const float d = rd_h(p);
        for (int ib = 0; ib < 8; ib++, dst += 32) {
            const int s4 = p[106 + ib / 2];
            const float db = d * (float)(1 + 2 * (ib % 2 == 0 ? (s4 & 0xF) : (s4 >> 4)));
            const int high = p[66 + ib];
            for (int l = 0; l < 4; l++) {
                const int lo = p[2 + 8 * ib + 2 * l] | ((high << (8 - 2 * l)) & 256);
                const int hi = p[2 + 8 * ib + 2 * l + 1] | ((high << (7 - 2 * l)) & 256);
                memcpy(g, &kIq3sGrid[lo], 4);
                memcpy(g + 4, &kIq3sGrid[hi], 4);
                signed8(g, p[74 + 4 * ib + l], db, dst + 8 * l);
            }
        }
        break;
    }
    case ORC_IQ1_S:
    case ORC_IQ1_M: {
        /* Quant.StoreIq1 (Quant.Iq.cs:246-251): (grid + delta) * scale, delta +-1/8 */
        int8_t e[8];
        if (fmt == ORC_IQ1_S) { /* {f16 d; qs[32]; u16 qh[8]} */
            const float d = rd_h(p);
            for (int ib = 0; ib < 8; ib++, dst += 32) {
                const uint32_t qh = rd_u16(p + 34 + 2 * ib);
                const float dl = d * (float)(2 * ((qh >> 12) & 7) + 1);
                const float delta = (qh & 0x8000) ? -0.125f : 0.125f;
                for (int l = 0; l < 4; l++) {
                    memcpy(e, &kIq1sGrid[p[2 + 4 * ib + l] | (((qh >> (3 * l)) & 7) << 8)], 8);
                    for (int j = 0; j < 8; j++) dst[8 * l + j] = ((float)e[j] + delta) * dl;
                }
            }
        } else { /* {qs[32]; qh[16]; u16 scales[4]}, the f16 super-scale in the scales' top nibbles */
            uint32_t sc[4];
            for (int i = 0; i < 4; i++) sc[i] = rd_u16(p + 48 + 2 * i);
            const uint32_t bits = (sc[0] >> 12) | ((sc[1] >> 8) & 0x00F0) | ((sc[2] >> 4) & 0x0F00) | (sc[3] & 0xF000);
            const float d = orc_f16_to_f32((uint16_t)bits);
            for (int ib = 0; ib < 8; ib++, dst += 32) {
                const float dl1 = d * (float)(2 * ((sc[ib / 2] >> (6 * (ib % 2))) & 7) + 1);
                const float dl2 = d * (float)(2 * ((sc[ib / 2] >> (6 * (ib % 2) + 3)) & 7) + 1);
                const uint8_t* qs = p + 4 * ib;
                const uint8_t* qh = p + 32 + 2 * ib;
                const int idx[4] = {qs[0] | ((qh[0] << 8) & 0x700), qs[1] | ((qh[0] << 4) & 0x700),
                                    qs[2] | ((qh[1] << 8) & 0x700), qs[3] | ((qh[1] << 4) & 0x700)};
                const int neg[4] = {qh[0] & 0x08, qh[0] & 0x80, qh[1] & 0x08, qh[1] & 0x80};
                for (int l = 0; l < 4; l++) {
                    memcpy(e, &kIq1sGrid[idx[l]], 8);
                    const float delta = neg[l] ? -0.125f : 0.125f, dl = l < 2 ? dl1 : dl2;
                    for (int j = 0; j < 8; j++) dst[8 * l + j] = ((float)e[j] + delta) * dl;
                }
            }
        }
        break;
    }
    default: break;
    }
}

/* One block of a K-quant or codebook format (256 values; IQ4_NL 32):
 *  Q2_K  (Quant.KQuants.cs:36-66): {scales[16] (lo: scale, hi: min), qs[64], f16 d, f16 dmin};
 *        value = q2 * (d * scale) - dmin * min, multiply and subtract unfused;
 *  Q3_K  (:68-107): {hmask[32], qs[64], scales[12] (6-bit, packed), f16 d}; value = (q2 + 4 hbit - 4) *
 *        (d * (scale - 32));
 *  Q4_K  (Quant.cs:518-545): {f16 d, f16 dmin, scales[12], qs[128]}; value = fma(q4, d*sc, -(dmin*m));
 *  Q5_K  (:547-582): {f16 d, f16 dmin, scales[12], qh[32], qs[128]}; the same with a fifth bit from qh;
 *  Q6_K  (:584-624): {ql[128], qh[64], int8 scales[16], f16 d}; value = fma(q6, s, -32 s), s = d * scale;
 *  IQ4_NL (:411-425): {f16 d, qs[16]}; value = d * codebook[nibble];
 *  IQ4_XS (:427-446): {f16 d, u16 scales_h, scales_l[4], qs[128]}; value = (d * (ls - 32)) * codebook[nibble]. */
/* Quant.E4m3ToFloat (Quant.Fp8.cs:37-49): bias 7, exponent 0 subnormal (m * 2^-9), exponent 15 with
 * mantissa 7 NaN (.NET's float.NaN, then negated for a set sign bit), no infinity. */
float orc_e4m3_value(uint8_t x)
{
    const int exp = (x >> 3) & 0xF, man = x & 7;
    float mag;
    if (exp == 0xF && man == 7) mag = u2f(0xFFC00000u);  /* float.NaN */
    else mag = exp == 0 ? ldexpf((float)man, -9) : ldexpf(1.0f + (float)man / 8.0f, exp - 7);
    return (x & 0x80) ? -mag : mag;
}

/* Quant.BuildE5m2 (Quant.Fp8.cs:62-72): the byte as the top half of an IEEE half. */
float orc_e5m2_value(uint8_t x) { return orc_f16_to_f32((uint16_t)(x << 8)); }

/* Nf4CodeBook / Fp4CodeBook (src/Sharplight.Core/Tensors/Grids/Nf4CodeBook.cs, Fp4CodeBook.cs): format data. */
static const float kNf4Book[16] = {
    -1.0f, -0.6961928009986877f, -0.5250730514526367f, -0.39491748809814453f, -0.28444138169288635f, -0.18477343022823334f,
    -0.09105003625154495f, 0.0f, 0.07958029955625534f, 0.16093020141124725f, 0.24611230194568634f, 0.33791524171829224f,
    0.44070982933044434f, 0.5626170039176941f, 0.7229568362236023f, 1.0f};
static const float kFp4Book[16] = {
    0.0f, 0.0052083334885537624f, 0.6666666865348816f, 1.0f, 0.3333333432674408f, 0.5f, 0.1666666716337204f, 0.25f,
    0.0f, -0.0052083334885537624f, -0.6666666865348816f, -1.0f, -0.3333333432674408f, -0.5f, -0.1666666716337204f, -0.25f};

static float rd_f32(const uint8_t* p) { float f; memcpy(&f, p, 4); return f; }

/* One block of the reference's own formats, restated from its decoders in their loop order. */
/* TrellisBlocks.State (src/Sharplight.Core/Tensors/TrellisBlocks.cs:61-73): step t's 16-bit state */
static uint32_t trellis_state(const uint8_t* qs, int v, int k, int t)
{
    const int steps = 128 / v;
    if (k == 8) return (uint32_t)qs[(t + steps - 1) % steps] << 8 | qs[t];
    const int bytes = steps * k / 8, off = (steps - 1 - t) * k, i0 = off >> 3;
    const uint32_t w = qs[i0] | (uint32_t)qs[(i0 + 1) % bytes] << 8 | (uint32_t)qs[(i0 + 2) % bytes] << 16;
    return (w >> (off & 7)) & 0xffffu;
}

/* TrellisBlocks.DecodeBlock (TrellisBlocks.cs:80-102): the state's low 15 bits times 0x9e3779b1 (mod 2^32);
 * point x >> 21 (and, 4 values per step, point (x >> 10) & 2047) of the f16 codebook, each value d * point */
static void trellis_block(int v, int k, const uint8_t* p, float* dst)
{
    const float d = rd_h(p);
    int o = 0;
    for (int t = 0; t < 128 / v; t++) {
        const uint32_t x = (trellis_state(p + 2, v, k, t) & 0x7fffu) * 0x9e3779b1u;
        uint32_t pt = x >> 21;
        dst[o++] = d * orc_f16_to_f32(kTrellisCodebook[2 * pt]);
        dst[o++] = d * orc_f16_to_f32(kTrellisCodebook[2 * pt + 1]);
        if (v == 4) {
            pt = (x >> 10) & 2047u;
            dst[o++] = d * orc_f16_to_f32(kTrellisCodebook[2 * pt]);
            dst[o++] = d * orc_f16_to_f32(kTrellisCodebook[2 * pt + 1]);
        }
    }
}

static void refblock(int fmt, const uint8_t* p, float* dst)
{
    switch (fmt) {
    case ORC_TRELLIS_V4K8: trellis_block(4, 8, p, dst); break;
    case ORC_TRELLIS_V4K6: trellis_block(4, 6, p, dst); break;
    case ORC_TRELLIS_V4K7: trellis_block(4, 7, p, dst); break;
    case ORC_TRELLIS_V2K5: trellis_block(2, 5, p, dst); break;
    case ORC_TRELLIS_V2K6: trellis_block(2, 6, p, dst); break;
    case ORC_TRELLIS_V2K7: trellis_block(2, 7, p, dst); break;
    case ORC_Q1_0: {  /* Quant.Q1_0 (Quant.cs:656-669): lut[byte][i] = bit i ? +1 : -1, times d */
        const float d = rd_h(p);
        for (int j = 0; j < 16; j++)
            for (int i = 0; i < 8; i++) dst[j * 8 + i] = (((p[2 + j] >> i) & 1) ? 1.0f : -1.0f) * d;
        break;
    }
    case ORC_Q2_0: case ORC_Q2_0_G128: {  /* Quant.Q2_0 (Quant.cs:673-686): lut[byte][i] = ((byte >> 2i) & 3) - 1 */
        const int qb = fmt == ORC_Q2_0 ? 16 : 32;
        const float d = rd_h(p);
        for (int j = 0; j < qb; j++)
            for (int i = 0; i < 4; i++) dst[j * 4 + i] = (float)(((p[2 + j] >> (2 * i)) & 3) - 1) * d;
        break;
    }
    case ORC_TERN1_G128: {  /* Quant.Tern1 (Quant.cs:689-718) */
        const float d = rd_h(p + 26);
        for (int m = 0; m < 16; m++)
            for (int n = 0; n < 5; n++) dst[n * 16 + m] = (float)trit(p[m], n) * d;
        for (int m = 0; m < 8; m++)
            for (int n = 0; n < 5; n++) dst[80 + n * 8 + m] = (float)trit(p[16 + m], n) * d;
        for (int h = 0; h < 2; h++)
            for (int n = 0; n < 4; n++) dst[120 + n * 2 + h] = (float)trit(p[24 + h], n) * d;
        break;
    }
    case ORC_NVFP4_GS: {  /* Quant.NVFP4_GS (Quant.Fp4.cs:86-107): d = ue4m3 * g, then fp4 * d */
        const float g = rd_f32(p);
        for (int sb = 0; sb < 4; sb++) {
            const float d = ue4m3_half(p[4 + sb]) * g;
            const uint8_t* q = p + 8 + 8 * sb;
            for (int j = 0; j < 8; j++) {
                dst[16 * sb + j] = (float)kFp4Values[q[j] & 0xF] * d;
                dst[16 * sb + j + 8] = (float)kFp4Values[q[j] >> 4] * d;
            }
        }
        break;
    }
    case ORC_Q4Z_G32: case ORC_Q4Z_G128: {  /* Quant.Q4Z (Quant.Grouped.cs:66-83), StoreU8x16Zeroed: (q - z) * d */
        const int group = fmt == ORC_Q4Z_G32 ? 32 : 128;
        const float d = rd_h(p), z = rd_h(p + 2);
        for (int run = 0; run < group / 32; run++)
            for (int j = 0; j < 16; j++) {
                const uint8_t q = p[4 + 16 * run + j];
                dst[32 * run + j] = ((float)(q & 0xF) - z) * d;
                dst[32 * run + 16 + j] = ((float)(q >> 4) - z) * d;
            }
        break;
    }
    case ORC_Q8Z_G32: case ORC_Q8Z_G128: {  /* Quant.Q8Z (Quant.Grouped.cs:86-98) */
        const int group = fmt == ORC_Q8Z_G32 ? 32 : 128;
        const float d = rd_h(p), z = rd_h(p + 2);
        for (int j = 0; j < group; j++) dst[j] = ((float)p[4 + j] - z) * d;
        break;
    }
    case ORC_NF4_B64: case ORC_FP4_B64: {  /* Quant.LookupB64 (Quant.Grouped.cs:107-127) */
        const float* book = fmt == ORC_NF4_B64 ? kNf4Book : kFp4Book;
        const float d = rd_f32(p);
        for (int run = 0; run < 2; run++)
            for (int j = 0; j < 16; j++) {
                const uint8_t q = p[4 + 16 * run + j];
                dst[32 * run + j] = book[q & 0xF] * d;
                dst[32 * run + j + 16] = book[q >> 4] * d;
            }
        break;
    }
    case ORC_Q8A_G32: {  /* Quant.Q8A_G32 (Quant.Absmax.cs:29-40): q * d * (1/127), left to right */
        const float d = rd_f32(p);
        for (int j = 0; j < 32; j++) dst[j] = (float)(int8_t)p[4 + j] * d * 7.874015718698502e-3f;
        break;
    }
    case ORC_Q2S_G128: {  /* Quant.Q2S_G128 (Quant.Absmax.cs:43-57) */
        const float d = rd_f32(p);
        for (int j = 0; j < 32; j++) {
            dst[j] = (float)(((p[4 + j] >> 6) & 3) - 1) * d;
            dst[32 + j] = (float)(((p[4 + j] >> 4) & 3) - 1) * d;
            dst[64 + j] = (float)(((p[4 + j] >> 2) & 3) - 1) * d;
            dst[96 + j] = (float)((p[4 + j] & 3) - 1) * d;
        }
        break;
    }
    case ORC_F8E4M3: dst[0] = orc_e4m3_value(p[0]) * 1.0f; break;  /* Quant.Lookup with scale 1 (Quant.Fp8.cs:125-137) */
    case ORC_F8E5M2: dst[0] = orc_e5m2_value(p[0]) * 1.0f; break;
    case ORC_F8E4M3_B32: case ORC_F8E4M3_B128: {  /* Quant.ScaledE4m3Blocks (Quant.Fp8.cs:112-122) */
        const int block = fmt == ORC_F8E4M3_B32 ? 32 : 128;
        const float d = rd_f32(p);
        for (int j = 0; j < block; j++) dst[j] = orc_e4m3_value(p[4 + j]) * d;
        break;
    }
    default: break;
    }
}

static void kblock(int fmt, const uint8_t* p, float* dst)
{
    switch (fmt) {
    case ORC_Q2_K: {
        const float d = rd_h(p + 80), dmin = rd_h(p + 82);
        for (int n = 0; n < 2; n++)
            for (int j = 0; j < 4; j++)
                for (int h = 0; h < 2; h++) {
                    const int sc = p[n * 8 + 2 * j + h];
                    const float dl = d * (float)(sc & 0xF), ml = dmin * (float)(sc >> 4);
                    for (int i = 0; i < 16; i++) {
                        const int q = (p[16 + 32 * n + 16 * h + i] >> (2 * j)) & 3;
                        const float prod = (float)q * dl;
                        dst[128 * n + 32 * j + 16 * h + i] = prod - ml;
                    }
                }
        break;
    }
    case ORC_Q3_K: {
        int8_t sc[16];
        for (int s = 0; s < 16; s++) {
            const int w = s / 4, b = s % 4;
            const uint8_t a = p[96 + 4 * (w & 1) + b];
            const int lo4 = w < 2 ? (a & 0xF) : (a >> 4);
            const int hi2 = (p[104 + b] >> (2 * w)) & 3;
            sc[s] = (int8_t)(lo4 | (hi2 << 4));
        }
        const float dall = rd_h(p + 108);
        for (int n = 0; n < 2; n++)
            for (int j = 0; j < 4; j++)
                for (int h = 0; h < 2; h++) {
                    const float dl = dall * (float)(sc[n * 8 + 2 * j + h] - 32);
                    for (int i = 0; i < 16; i++) {
                        const int low = (p[32 + 32 * n + 16 * h + i] >> (2 * j)) & 3;
                        const int high = (p[16 * h + i] >> (4 * n + j)) & 1;
                        const int v = low + 4 * high - 4;
                        dst[128 * n + 32 * j + 16 * h + i] = (float)v * dl;
                    }
                }
        break;
    }
    case ORC_Q4_K:
    case ORC_Q5_K: {
        const int k5 = fmt == ORC_Q5_K;
        const float d = rd_h(p), dmin = rd_h(p + 2);
        const uint8_t* scales = p + 4;
        const uint8_t* qh = p + 16;
        const uint8_t* qs = p + (k5 ? 48 : 16);
        for (int j = 0; j < 4; j++)
            for (int half = 0; half < 2; half++) {
                int sc, m;
                scale_min(2 * j + half, scales, &sc, &m);
                const float dl = d * (float)sc, mm = dmin * (float)m;
                for (int i = 0; i < 32; i++) {
                    int q = (qs[32 * j + i] >> (4 * half)) & 15;
                    if (k5) q |= ((qh[i] >> (2 * j + half)) & 1) << 4;
                    dst[64 * j + 32 * half + i] = fmaf((float)q, dl, -mm);
                }
            }
        break;
    }
    case ORC_Q6_K: {
        const float d = rd_h(p + 208);
        for (int n = 0; n < 2; n++)
            for (int r = 0; r < 128; r++) {
                const int qt = r / 32, i = r % 32, h = i / 16;
                const uint8_t l = p[64 * n + (qt & 1 ? 32 : 0) + i];
                const int lo = qt >= 2 ? l >> 4 : l & 15;
                const int hi = (p[128 + 32 * n + i] >> (2 * qt)) & 3;
                const float sc = d * (float)(int8_t)p[192 + 8 * n + h + 2 * qt];
                dst[128 * n + r] = fmaf((float)(lo | (hi << 4)), sc, -32.0f * sc);
            }
        break;
    }
    case ORC_IQ4_NL: {
        const float d = rd_h(p);
        for (int j = 0; j < 16; j++) {
            dst[j] = d * (float)kIq4Values[p[2 + j] & 0xF];
            dst[j + 16] = d * (float)kIq4Values[p[2 + j] >> 4];
        }
        break;
    }
    case ORC_IQ4_XS: {
        const float d = rd_h(p);
        const unsigned sh = p[2] | ((unsigned)p[3] << 8);
        for (int ib = 0; ib < 8; ib++) {
            const int ls = ((p[4 + ib / 2] >> (4 * (ib % 2))) & 0xF) | (int)(((sh >> (2 * ib)) & 3) << 4);
            const float dl = d * (float)(ls - 32);
            const uint8_t* qs = p + 8 + 16 * ib;
            for (int j = 0; j < 16; j++) {
                dst[32 * ib + j] = dl * (float)kIq4Values[qs[j] & 0xF];
                dst[32 * ib + j + 16] = dl * (float)kIq4Values[qs[j] >> 4];
            }
        }
        break;
    }
    case ORC_IQ2_XXS: case ORC_IQ2_XS: case ORC_IQ2_S: case ORC_IQ3_XXS: case ORC_IQ3_S: case ORC_IQ1_S:
    case ORC_IQ1_M:
        iq_block(fmt, p, dst);
        break;
    case ORC_TQ1_0: {  /* Quant.TQ1_0 (Quant.Ternary.cs:27-64): {qs[48], qh[4], f16 d} */
        const float d = rd_h(p + 52);
        for (int n = 0; n < 5; n++) {
            for (int m = 0; m < 32; m++) dst[n * 32 + m] = (float)trit(p[m], n) * d;
            for (int m = 0; m < 16; m++) dst[160 + n * 16 + m] = (float)trit(p[32 + m], n) * d;
        }
        for (int n = 0; n < 4; n++)
            for (int j = 0; j < 4; j++) dst[240 + n * 4 + j] = (float)trit(p[48 + j], n) * d;
        break;
    }
    case ORC_TQ2_0: {  /* Quant.TQ2_0 (Quant.Ternary.cs:66-86): {qs[64], f16 d} */
        const float d = rd_h(p + 64);
        for (int j = 0; j < 2; j++)
            for (int l = 0; l < 4; l++)
                for (int m = 0; m < 32; m++)
                    dst[128 * j + 32 * l + m] = (float)(((p[32 * j + m] >> (2 * l)) & 3) - 1) * d;
        break;
    }
    case ORC_MXFP4: {  /* Quant.MXFP4 (Quant.Fp4.cs:43-58): {u8 e, qs[16]} */
        const float d = e8m0_half(p[0]);
        for (int j = 0; j < 16; j++) {
            dst[j] = (float)kFp4Values[p[1 + j] & 0xF] * d;
            dst[j + 16] = (float)kFp4Values[p[1 + j] >> 4] * d;
        }
        break;
    }
    case ORC_NVFP4: {  /* Quant.NVFP4 (Quant.Fp4.cs:60-80): {u8 d[4], qs[32]}, four 16-value sub-blocks */
        for (int sb = 0; sb < 4; sb++) {
            const float d = ue4m3_half(p[sb]);
            const uint8_t* q = p + 4 + 8 * sb;
            for (int j = 0; j < 8; j++) {
                dst[16 * sb + j] = (float)kFp4Values[q[j] & 0xF] * d;
                dst[16 * sb + j + 8] = (float)kFp4Values[q[j] >> 4] * d;
            }
        }
        break;
    }
    default:
        refblock(fmt, p, dst);
        break;
    }
}

/* Quant.Dequantize (Quant.cs:242-368) with the block decoders Q4_0/Q8_0 (:384-405),
 * Q4_1/Q5_0/Q5_1 (:449-500) and Simd.StoreI8x16/StoreU8x16 (Simd.cs:699-753): value =
 * fma(q, d, offset), offset 0 (Q8_0), -8d (Q4_0), -16d (Q5_0), m (Q4_1, Q5_1). */
int orc_dequant(int fmt, const uint8_t* p, int64_t count, float* dst)
{
    switch (fmt) {
    case ORC_F32: memcpy(dst, p, (size_t)count * 4); return 0;
    case ORC_F16:
        for (int64_t i = 0; i < count; i++) dst[i] = rd_h(p + 2 * i);
        return 0;
    case ORC_BF16:
        for (int64_t i = 0; i < count; i++) dst[i] = orc_bf16_to_f32((uint16_t)(p[2 * i] | (p[2 * i + 1] << 8)));
        return 0;
    default: break;
    }
    if (block_bytes(fmt) < 0) return -1;
    if (fmt >= ORC_Q2_K) {
        const int bs = block_size(fmt), bb = block_bytes(fmt);
        if (count % bs) return -1;
        for (int64_t b = 0; b < count / bs; b++) kblock(fmt, p + b * bb, dst + b * bs);
        return 0;
    }
    if (count % 32) return -1;
    int64_t nb = count / 32;
    for (int64_t b = 0; b < nb; b++, dst += 32) {
        switch (fmt) {
        case ORC_Q8_0: {
            float d = rd_h(p);
            for (int j = 0; j < 32; j++) dst[j] = fmaf((float)(int8_t)p[2 + j], d, 0.0f);
            p += 34;
            break;
        }
        case ORC_Q4_0: {
            float d = rd_h(p), o = -8.0f * d;
            for (int j = 0; j < 16; j++) {
                dst[j] = fmaf((float)(p[2 + j] & 15), d, o);
                dst[j + 16] = fmaf((float)(p[2 + j] >> 4), d, o);
            }
            p += 18;
            break;
        }
        case ORC_Q4_1: {
            float d = rd_h(p), m = rd_h(p + 2);
            for (int j = 0; j < 16; j++) {
                dst[j] = fmaf((float)(p[4 + j] & 15), d, m);
                dst[j + 16] = fmaf((float)(p[4 + j] >> 4), d, m);
            }
            p += 20;
            break;
        }
        case ORC_Q5_0: {
            float d = rd_h(p), o = -16.0f * d;
            uint32_t qh = (uint32_t)p[2] | ((uint32_t)p[3] << 8) | ((uint32_t)p[4] << 16) | ((uint32_t)p[5] << 24);
            for (int j = 0; j < 16; j++) {
                uint32_t lo = (p[6 + j] & 15u) | (((qh >> j) & 1u) << 4);
                uint32_t hi = (p[6 + j] >> 4) | (((qh >> (j + 16)) & 1u) << 4);
                dst[j] = fmaf((float)lo, d, o);
                dst[j + 16] = fmaf((float)hi, d, o);
            }
            p += 22;
            break;
        }
        case ORC_Q5_1: {
            float d = rd_h(p), m = rd_h(p + 2);
            uint32_t qh = (uint32_t)p[4] | ((uint32_t)p[5] << 8) | ((uint32_t)p[6] << 16) | ((uint32_t)p[7] << 24);
            for (int j = 0; j < 16; j++) {
                uint32_t lo = (p[8 + j] & 15u) | (((qh >> j) & 1u) << 4);
                uint32_t hi = (p[8 + j] >> 4) | (((qh >> (j + 16)) & 1u) << 4);
                dst[j] = fmaf((float)lo, d, m);
                dst[j + 16] = fmaf((float)hi, d, m);
            }
            p += 24;
            break;
        }
        default: return -1;
        }
    }
    return 0;
}

/* GatherOp.Body (src/Sharplight.Cpu/GatherOp.cs:53-75): bounds check, then dequantize the row. */
static int gather_range(int fmt, const uint8_t* table, int64_t V, int64_t D, const int32_t* ids, int64_t i0, int64_t i1,
                        float* y, int64_t* bad)
{
    int64_t rb = orc_row_bytes(fmt, D);
    if (rb < 0) return -2;
    for (int64_t i = i0; i < i1; i++) {
        int64_t id = ids[i];
        if ((uint64_t)id >= (uint64_t)V) {
            if (bad) *bad = id;
            return -1;
        }
        if (orc_dequant(fmt, table + id * rb, D, y + i * D)) return -2;
    }
    return 0;
}

int orc_gather(int fmt, const uint8_t* table, int64_t V, int64_t D, const int32_t* ids, int64_t N, float* y,
               int64_t* bad_index)
{
    return gather_range(fmt, table, V, D, ids, 0, N, y, bad_index);
}

/* ------------------------------------------------------------------------------------------ */
/* KV cache writes                                                                            */
/* ------------------------------------------------------------------------------------------ */

/* Simd.FloatToHalf (src/Sharplight.Cpu/Simd.cs:521-525) is .NET's (Half)f, in the .NET runtime rather
 * than the reference: IEEE round to nearest even with gradual underflow and overflow to infinity; a NaN
 * keeps its sign and the top 10 bits of its payload with the quiet bit set (sign | 0x7E00 | mant >> 13).
 * The NaN rule is restated from the runtime's published source (parity unpinned for NaN payloads). */
uint16_t orc_f32_to_f16(float f)
{
    uint32_t b = f2u(f);
    uint32_t sign = (b >> 16) & 0x8000u;
    uint32_t exp = (b >> 23) & 0xFFu;
    uint32_t man = b & 0x7FFFFFu;
    if (exp == 0xFF) return (uint16_t)(man ? (sign | 0x7E00u | (man >> 13)) : (sign | 0x7C00u));
    int32_t e = (int32_t)exp - 127 + 15;  /* biased f16 exponent */
    if (e >= 31) return (uint16_t)(sign | 0x7C00u);
    uint32_t m = man | (exp ? 0x800000u : 0u);  /* 24-bit significand (f32 subnormals: no implicit 1) */
    int shift;                                   /* bits dropped from m */
    uint32_t base;
    if (e >= 1) {
        shift = 13;
        base = ((uint32_t)e << 10);
        m &= 0x7FFFFFu;  /* the implicit 1 is carried by the exponent field */
    } else {
        shift = 14 - e;  /* subnormal f16: value = m * 2^(exp-150) = q * 2^-24 */
        if (!exp) shift = 200;  /* f32 subnormals are far below the smallest f16 subnormal */
        base = 0;
    }
    if (shift > 31) return (uint16_t)sign;  /* rounds to zero (|f| < 2^-25 at most half an ulp) */
    uint32_t q = m >> shift;
    uint32_t rem = m & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1u))) q++;  /* may carry into the exponent: still correct */
    return (uint16_t)(sign | (base + q));
}

void orc_f32_to_f16_n(const float* x, uint16_t* y, int64_t n)
{
    for (int64_t i = 0; i < n; i++) y[i] = orc_f32_to_f16(x[i]);
}

/* Cache rows of tokens 0..T-1, as CacheWriteOp maps them (src/Sharplight.Cpu/CacheWriteOp.cs:103-155, no
 * compression): ROWS_PAST row = n_past + t; ROWS_SEQ row = slot * (ctx / slots) + position from sequence
 * rows seq[T, 4] = (slot, position, ., .); ROWS_PAGED row = table[slot, p / bs] * bs + p % bs
 * (KvPages.Row, KvPages.cs:28-32). The checks run first, over every token, as CacheWriteOp.Run does
 * (:103-127; KvPages.Check, KvPages.cs:38-49): 0, or -1 with the message the reference throws. */
int orc_cache_rows(int mode, int64_t T, int64_t ctx, int64_t n_past, const int32_t* seq, int64_t slots,
                   const int32_t* pages, int64_t page_slots, int64_t blocks_per_slot, int64_t block_size,
                   int64_t* rows, char* err, int64_t err_size)
{
    if (mode == ORC_ROWS_PAST) {
        if (n_past < 0 || n_past + T > ctx) {
            snprintf(err, (size_t)err_size, "KV cache overflow: n_past %lld + T %lld > context %lld.",
                     (long long)n_past, (long long)T, (long long)ctx);
            return -1;
        }
        for (int64_t t = 0; t < T; t++) rows[t] = n_past + t;
        return 0;
    }
    for (int64_t t = 0; t < T; t++) {
        int32_t slot = seq[t * 4], p = seq[t * 4 + 1];
        if (mode == ORC_ROWS_PAGED) {
            if ((uint64_t)(int64_t)slot >= (uint64_t)page_slots || p < 0 || p >= blocks_per_slot * block_size) {
                snprintf(err, (size_t)err_size, "Sequence slot %d / position %d outside the block table [%lld, %lld].",
                         slot, p, (long long)page_slots, (long long)blocks_per_slot);
                return -1;
            }
            int64_t block = pages[(int64_t)slot * blocks_per_slot + p / block_size];
            if (block < 0 || (block + 1) * block_size > ctx) {
                snprintf(err, (size_t)err_size, "Block %lld of slot %d (position %d) is outside the KV cache of %lld rows.",
                         (long long)block, slot, p, (long long)ctx);
                return -1;
            }
            rows[t] = block * block_size + p % block_size;
        } else {
            int64_t slot_ctx = ctx / (slots > 0 ? slots : 1);
            if ((uint64_t)(int64_t)slot >= (uint64_t)slots || (uint64_t)(int64_t)p >= (uint64_t)slot_ctx) {
                snprintf(err, (size_t)err_size, "KV cache overflow: sequence row %lld slot %d position %d (slot context %lld).",
                         (long long)t, slot, p, (long long)slot_ctx);
                return -1;
            }
            rows[t] = slot * slot_ctx + p;
        }
    }
    return 0;
}

/* CacheWriteOp.Body (CacheWriteOp.cs:129-175): token t's `inner` f32 values go to cache row rows[t] as
 * f32 (copied), f16 (FloatToHalf) or bf16 (FloatToBFloat). */
void orc_cache_write(int cache_type, void* cache, int64_t inner, const float* x, int64_t T, const int64_t* rows)
{
    for (int64_t t = 0; t < T; t++) {
        const float* src = x + t * inner;
        int64_t d = rows[t] * inner;
        if (cache_type == ORC_F32) {
            memcpy((float*)cache + d, src, (size_t)inner * 4);
        } else {
            uint16_t* dst = (uint16_t*)cache + d;
            for (int64_t i = 0; i < inner; i++)
                dst[i] = cache_type == ORC_F16 ? orc_f32_to_f16(src[i]) : orc_f32_to_bf16(src[i]);
        }
    }
}

/* ------------------------------------------------------------------------------------------ */
/* threading (CpuParallel.cs:34-78)                                                           */
/* ------------------------------------------------------------------------------------------ */

static int g_threads = 1;

void orc_set_threads(int threads) { g_threads = threads < 1 ? 1 : threads; }
int orc_get_threads(void) { return g_threads; }

/* CpuParallel.Chunks: 1 when total <= minChunk, else min(threads*4, total/minChunk). */
static int64_t chunks_for(int64_t total, int64_t min_chunk)
{
    if (total <= min_chunk) return 1;
    int64_t c = (int64_t)g_threads * 4;
    if (total / min_chunk < c) c = total / min_chunk;
    return c < 1 ? 1 : c;
}

typedef void (*chunk_fn)(void* ctx, int64_t c);

typedef struct {
    chunk_fn fn;
    void* ctx;
    int64_t n;
    int64_t next; /* guarded by mu */
    pthread_mutex_t mu;
} pfor_t;

static void* pfor_worker(void* arg)
{
    pfor_t* p = (pfor_t*)arg;
    for (;;) {
        pthread_mutex_lock(&p->mu);
        int64_t c = p->next++;
        pthread_mutex_unlock(&p->mu);
        if (c >= p->n) break;
        p->fn(p->ctx, c);
    }
    return NULL;
}

/* CpuParallel.For: chunk indices 0..n-1 handed to min(n, threads) workers. */
static void parallel_for(int64_t n, chunk_fn fn, void* ctx)
{
    if (n <= 0) return;
    int workers = g_threads < n ? g_threads : (int)n;
    if (workers <= 1) {
        for (int64_t c = 0; c < n; c++) fn(ctx, c);
        return;
    }
    pfor_t p;
    p.fn = fn;
    p.ctx = ctx;
    p.n = n;
    p.next = 0;
    pthread_mutex_init(&p.mu, NULL);
    pthread_t* th = (pthread_t*)malloc(sizeof(pthread_t) * (size_t)workers);
    for (int i = 1; i < workers; i++) pthread_create(&th[i], NULL, pfor_worker, &p);
    pfor_worker(&p);
    for (int i = 1; i < workers; i++) pthread_join(th[i], NULL);
    free(th);
    pthread_mutex_destroy(&p.mu);
}

typedef struct {
    const float *x, *w, *b;
    float* y;
    int64_t rows, n, per;
    float eps;
    int mode;
} row_ctx;

static void rms_chunk(void* v, int64_t c)
{
    row_ctx* r = (row_ctx*)v;
    int64_t s = c * r->per, e = s + r->per < r->rows ? s + r->per : r->rows;
    rmsnorm_rows(r->x, r->w, r->y, s, e, r->n, r->eps, r->mode);
}

static void ln_chunk(void* v, int64_t c)
{
    row_ctx* r = (row_ctx*)v;
    int64_t s = c * r->per, e = s + r->per < r->rows ? s + r->per : r->rows;
    layernorm_rows(r->x, r->w, r->b, r->y, s, e, r->n, r->eps);
}

/* RowOp.Run (RowOp.cs:37-49): chunks = min(rows, Chunks(rows*cols, 16384)). */
void orc_rmsnorm_mt(const float* x, const float* w, float* y, int64_t rows, int64_t n, float eps, int mode)
{
    if (rows == 0 || n == 0) return;
    int64_t ch = chunks_for(rows * n, 16384);
    if (ch > rows) ch = rows;
    row_ctx r = {x, w, NULL, y, rows, n, (rows + ch - 1) / ch, eps, mode};
    parallel_for(ch, rms_chunk, &r);
}

void orc_layernorm_mt(const float* x, const float* w, const float* b, float* y, int64_t rows, int64_t n, float eps)
{
    if (rows == 0 || n == 0) return;
    int64_t ch = chunks_for(rows * n, 16384);
    if (ch > rows) ch = rows;
    row_ctx r = {x, w, b, y, rows, n, (rows + ch - 1) / ch, eps, 0};
    parallel_for(ch, ln_chunk, &r);
}

typedef struct {
    const float *a, *b;
    float* y;
    int64_t n, per;
    int kind; /* 0 add, 1 mul, 2+ unary act (kind-2) */
} ew_ctx;

static void ew_chunk(void* v, int64_t c)
{
    ew_ctx* e = (ew_ctx*)v;
    int64_t s = c * e->per, t = s + e->per < e->n ? s + e->per : e->n;
    if (s >= t) return;
    if (e->kind == 0) orc_add(e->a + s, e->b + s, e->y + s, t - s);
    else if (e->kind == 1) orc_mul(e->a + s, e->b + s, e->y + s, t - s);
    else unary_range(e->kind - 2, e->a + s, e->y + s, t - s);
}

/* UnaryOp.Run / BinaryOp.Run on dense operands (UnaryOp.cs:30-48, BinaryOp.cs:60-100): flat
 * chunks of at least 32768 elements. */
static void ew_run(int kind, const float* a, const float* b, float* y, int64_t n)
{
    if (n == 0) return;
    int64_t ch = chunks_for(n, 32768);
    ew_ctx e = {a, b, y, n, (n + ch - 1) / ch, kind};
    parallel_for(ch, ew_chunk, &e);
}

void orc_add_mt(const float* a, const float* b, float* y, int64_t n) { ew_run(0, a, b, y, n); }
void orc_mul_mt(const float* a, const float* b, float* y, int64_t n) { ew_run(1, a, b, y, n); }
void orc_unary_mt(int act, const float* x, float* y, int64_t n) { ew_run(2 + act, x, NULL, y, n); }

typedef struct {
    const float* x;
    const int32_t* pos;
    const float* ff;
    float* y;
    int64_t T, H, D, per;
    int dims, neox;
    float base, fs, af;
} rope_ctx;

static void rope_chunk(void* v, int64_t c)
{
    rope_ctx* r = (rope_ctx*)v;
    int64_t s = c * r->per, e = s + r->per < r->T ? s + r->per : r->T;
    if (s < e) rope_tokens(r->x, r->pos, 1, NULL, 0, 0, r->ff, r->y, s, e, r->H, r->D, r->dims, r->neox, r->base, r->fs, r->af);
}

/* RopeOp.Run (RopeOp.cs:108-119): chunks = min(T, Chunks(T*H*D, 16384)). */
void orc_rope_mt(const float* x, const int32_t* pos, const float* ff, float* y, int64_t T, int64_t H, int64_t D, int dims,
                 int neox, float base, float freq_scale, float attn_factor)
{
    if (T == 0) return;
    int64_t ch = chunks_for(T * H * D, 16384);
    if (ch > T) ch = T;
    rope_ctx r = {x, pos, ff, y, T, H, D, (T + ch - 1) / ch, dims, neox, base, freq_scale, attn_factor};
    parallel_for(ch, rope_chunk, &r);
}

typedef struct {
    int fmt;
    const uint8_t* table;
    int64_t V, D, N, per;
    const int32_t* ids;
    float* y;
    int status;
    int64_t bad;
    pthread_mutex_t mu;
} gather_ctx;

static void gather_chunk(void* v, int64_t c)
{
    gather_ctx* g = (gather_ctx*)v;
    int64_t s = c * g->per, e = s + g->per < g->N ? s + g->per : g->N;
    int64_t bad = 0;
    int st = s < e ? gather_range(g->fmt, g->table, g->V, g->D, g->ids, s, e, g->y, &bad) : 0;
    if (st) {
        pthread_mutex_lock(&g->mu);
        if (!g->status) {
            g->status = st;
            g->bad = bad;
        }
        pthread_mutex_unlock(&g->mu);
    }
}

/* GatherOp.Run (GatherOp.cs:40-51): chunks = min(N, Chunks(N*D, 8192)). */
int orc_gather_mt(int fmt, const uint8_t* table, int64_t V, int64_t D, const int32_t* ids, int64_t N, float* y,
                  int64_t* bad_index)
{
    if (N == 0) return 0;
    int64_t ch = chunks_for(N * D, 8192);
    if (ch > N) ch = N;
    gather_ctx g;
    g.fmt = fmt;
    g.table = table;
    g.V = V;
    g.D = D;
    g.N = N;
    g.per = (N + ch - 1) / ch;
    g.ids = ids;
    g.y = y;
    g.status = 0;
    g.bad = 0;
    pthread_mutex_init(&g.mu, NULL);
    parallel_for(ch, gather_chunk, &g);
    pthread_mutex_destroy(&g.mu);
    if (g.status && bad_index) *bad_index = g.bad;
    return g.status;
}

typedef struct {
    int type;
    void* cache;
    int64_t inner, T, per;
    const float* x;
    const int64_t* rows;
} cache_ctx;

static void cache_chunk(void* v, int64_t c)
{
    cache_ctx* k = (cache_ctx*)v;
    int64_t s = c * k->per, e = s + k->per < k->T ? s + k->per : k->T;
    if (s < e) orc_cache_write(k->type, k->cache, k->inner, k->x + s * k->inner, e - s, k->rows + s);
}

/* CacheWriteOp.Run (CacheWriteOp.cs:122-126): chunks = min(rows, Chunks(rows*rowLen, 8192)), over tokens. */
void orc_cache_write_mt(int cache_type, void* cache, int64_t inner, const float* x, int64_t T, const int64_t* rows)
{
    if (T == 0) return;
    int64_t ch = chunks_for(T * inner, 8192);
    if (ch > T) ch = T;
    cache_ctx k = {cache_type, cache, inner, T, (T + ch - 1) / ch, x, rows};
    parallel_for(ch, cache_chunk, &k);
}

/* ------------------------------------------------------------------------------------------ */
/* E4M3 activation rows (norm-written copies for the fp8 GEMM)                               */
/* ------------------------------------------------------------------------------------------ */

/* e4m3_code (src/Sharplight.Shaders/Kernels/e4m3.slang:5-23): the E4M3 code of |v| <= 448 rounded to
 * nearest even; below 2^-6 a multiple of 2^-9 (round() of HLSL: halfway cases to even), above by adding
 * 0x7FFFF + lsb at bit 20 of the f32 bits; saturated at code 0x7E (448); the sign in bit 7. */
uint8_t orc_e4m3_code(float v)
{
    uint32_t sign = v < 0 ? 0x80u : 0u;
    float a = fabsf(v);
    uint32_t code;
    if (a < 0.015625f) {
        code = (uint32_t)nearbyintf(a * 512.0f); /* the default rounding mode: to nearest even */
    } else {
        uint32_t bits = f2u(a);
        bits += 0x7FFFFu + ((bits >> 20) & 1u);
        uint32_t c = (bits >> 20) - (120u << 3);
        code = c < 0x7Eu ? c : 0x7Eu;
    }
    return (uint8_t)(sign | code);
}

/* quantize_fp8 (Kernels/gemm_fp8.slang:36-55) on one row of K values (K % 128 == 0): per 128-value group
 * d = amax / 448 (e4m3_group_scale, e4m3.slang:25-31), codes of v * (d > 0 ? 1/d : 0) (e4m3_pack4,
 * :33-38); out = [K codes][K/128 f32 scales], the activation row layout of the fp8 GEMM. */
void orc_quantize_fp8_row(const float* x, int64_t K, uint8_t* out)
{
    float* scales = (float*)(out + K);
    for (int64_t g = 0; g < K / 128; g++) {
        const float* v = x + g * 128;
        float amax = 0.0f;
        for (int i = 0; i < 128; i++) {
            float m = fabsf(v[i]);
            if (m > amax) amax = m;
        }
        float d = amax / 448.0f;
        float id = d > 0 ? 1.0f / d : 0.0f;
        for (int i = 0; i < 128; i++) out[g * 128 + i] = orc_e4m3_code(v[i] * id);
        memcpy(&scales[g], &d, 4);
    }
}

void orc_quantize_fp8_rows(const float* x, int64_t rows, int64_t K, uint8_t* out)
{
    for (int64_t r = 0; r < rows; r++) orc_quantize_fp8_row(x + r * K, K, out + r * (K + K / 32));
}

typedef struct {
    const float* x;
    uint8_t* out;
    int64_t rows, K, per;
} fp8_ctx;

static void fp8_chunk(void* v, int64_t c)
{
    fp8_ctx* k = (fp8_ctx*)v;
    int64_t s = c * k->per, e = s + k->per < k->rows ? s + k->per : k->rows;
    if (s < e) orc_quantize_fp8_rows(k->x + s * k->K, e - s, k->K, k->out + s * (k->K + k->K / 32));
}

/* Row-chunked over the host threads, as the reference's CPU ops split rows (RowOp.cs chunking); only the
 * timing of the CPU baseline uses it. */
void orc_quantize_fp8_rows_mt(const float* x, int64_t rows, int64_t K, uint8_t* out)
{
    if (rows == 0) return;
    int64_t ch = chunks_for(rows * K, 16384);
    if (ch > rows) ch = rows;
    fp8_ctx k = {x, out, rows, K, (rows + ch - 1) / ch};
    parallel_for(ch, fp8_chunk, &k);
}

typedef struct {
    const float* x;
    uint16_t* y;
    int64_t n, per;
} f16_ctx;

static void f16_chunk(void* v, int64_t c)
{
    f16_ctx* k = (f16_ctx*)v;
    int64_t s = c * k->per, e = s + k->per < k->n ? s + k->per : k->n;
    if (s < e) orc_f32_to_f16_n(k->x + s, k->y + s, e - s);
}

/* orc_f32_to_f16_n split over the host threads (the CPU baseline's timing only). */
void orc_f32_to_f16_mt(const float* x, uint16_t* y, int64_t n)
{
    if (n == 0) return;
    int64_t ch = chunks_for(n, 16384);
    f16_ctx k = {x, y, n, (n + ch - 1) / ch};
    parallel_for(ch, f16_chunk, &k);
}

/* ------------------------------------------------------------------------------------------ */
/* Matvec: y = x . W^T for few activation rows (decode)                                       */
/* ------------------------------------------------------------------------------------------ */

/* Vector512.Sum: the runtime's horizontal add; restated as pairwise halving (lane i + lane i+8, then
 * +4, +2, +1). The order of the runtime's reduction is not in the reference, so this level of rounding
 * is parity unpinned; the matvec pins hold the results to the f64 dot within the f32 error bound. */
static float sum16(const float* v)
{
    float s[16];
    for (int i = 0; i < 16; i++) s[i] = v[i];
    for (int w = 8; w > 0; w >>= 1)
        for (int i = 0; i < w; i++) s[i] = s[i] + s[i + w];
    return s[0];
}

/* Simd.Dot4 on the AVX-512 path (Simd.cs:91-133,161-175): two 16-lane accumulators (a over the first, b
 * over the second half of each 32 elements, fma(w, x, acc)), a 16-element step into a, r = Sum(a + b),
 * then a scalar tail r += w * x. */
static void dot4(const float* x, const float* const* w, int64_t n, float* res)
{
    float a[4][16] = {{0}}, b[4][16] = {{0}};
    int64_t i = 0;
    for (; i + 32 <= n; i += 32)
        for (int r = 0; r < 4; r++)
            for (int l = 0; l < 16; l++) {
                a[r][l] = fmaf(w[r][i + l], x[i + l], a[r][l]);
                b[r][l] = fmaf(w[r][i + 16 + l], x[i + 16 + l], b[r][l]);
            }
    for (; i + 16 <= n; i += 16)
        for (int r = 0; r < 4; r++)
            for (int l = 0; l < 16; l++) a[r][l] = fmaf(w[r][i + l], x[i + l], a[r][l]);
    for (int r = 0; r < 4; r++) {
        float s[16];
        for (int l = 0; l < 16; l++) s[l] = a[r][l] + b[r][l];
        res[r] = sum16(s);
    }
    for (; i < n; i++)
        for (int r = 0; r < 4; r++) res[r] = res[r] + w[r][i] * x[i];
}

/* Simd.Dot4x2 on the AVX-512 path (Simd.cs:176-270): one 16-lane accumulator per (token, row), then the
 * scalar tail; res = [t0 r0..r3, t1 r0..r3]. */
static void dot4x2(const float* x0, const float* x1, const float* const* w, int64_t n, float* res)
{
    float a[4][16] = {{0}}, c[4][16] = {{0}};
    int64_t i = 0;
    for (; i + 16 <= n; i += 16)
        for (int r = 0; r < 4; r++)
            for (int l = 0; l < 16; l++) {
                a[r][l] = fmaf(w[r][i + l], x0[i + l], a[r][l]);
                c[r][l] = fmaf(w[r][i + l], x1[i + l], c[r][l]);
            }
    for (int r = 0; r < 4; r++) {
        res[r] = sum16(a[r]);
        res[4 + r] = sum16(c[r]);
    }
    for (; i < n; i++)
        for (int r = 0; r < 4; r++) {
            res[r] = res[r] + w[r][i] * x0[i];
            res[4 + r] = res[4 + r] + w[r][i] * x1[i];
        }
}

/* Quant.DotQ8_0x4 / DotQ4_0x4 (Quant.cs:738-803), the fused one-row path for Q8_0 / Q4_0: per block and
 * lane s = fma(q0, x0, q1 * x1) (Q4_0: fma(lo, x0, hi * x1) - 8 (x0 + x1)), acc = fma(s, d, acc); the
 * rows' results are Sum(acc). */
static float dot_fused_row(int fmt, const float* x, const uint8_t* row, int64_t nb)
{
    float acc[16] = {0};
    for (int64_t b = 0; b < nb; b++) {
        const float* x0 = x + b * 32;
        const float* x1 = x0 + 16;
        if (fmt == ORC_Q8_0) {
            const uint8_t* p = row + b * 34;
            const float d = rd_h(p);
            for (int l = 0; l < 16; l++) {
                const float s = fmaf((float)(int8_t)p[2 + l], x0[l], (float)(int8_t)p[18 + l] * x1[l]);
                acc[l] = fmaf(s, d, acc[l]);
            }
        } else {
            const uint8_t* p = row + b * 18;
            const float d = rd_h(p);
            for (int l = 0; l < 16; l++) {
                const float x8 = (x0[l] + x1[l]) * 8.0f;
                const float s = fmaf((float)(p[2 + l] & 15), x0[l], (float)(p[2 + l] >> 4) * x1[l]) - x8;
                acc[l] = fmaf(s, d, acc[l]);
            }
        }
    }
    return sum16(acc);
}

/* MatMulOp's float-row path (MatMulOp.cs:376-465), as the CPU provider runs decode: rows of W in groups
 * of four; with at most 4 activation rows and a fused kernel (Q8_0 / Q4_0) each row is one fused dot,
 * otherwise K is walked in 1024-value chunks -- each chunk of the four rows dequantized (Quant.Dequantize)
 * and dotted (Dot4x2 for pairs of rows when there are more than 4, Dot4 for the rest), the chunk results
 * added into f32 accumulators. y is [T, N] f32; x is [T, K] f32; W is N rows of row_bytes(fmt, K). */
static void matvec_groups(int fmt, const uint8_t* w, int64_t N, int64_t K, const float* x, int64_t T, float* y,
                          int64_t g0, int64_t g1)
{
    const int64_t rb = orc_row_bytes(fmt, K);
    const int fused = (fmt == ORC_Q8_0 || fmt == ORC_Q4_0) && T <= 4;
    float* wbuf = (float*)malloc(4 * 1024 * sizeof(float));
    float* acc = (float*)malloc((size_t)(T * 4 > 1 ? T * 4 : 1) * sizeof(float));
    for (int64_t g = g0; g < g1; g++) {
        const int64_t n0 = g * 4;
        const int nr = N - n0 < 4 ? (int)(N - n0) : 4;
        const uint8_t* rows[4];
        for (int r = 0; r < 4; r++) rows[r] = w + (n0 + r < N ? n0 + r : N - 1) * rb;
        if (fused) {
            for (int64_t t = 0; t < T; t++)
                for (int r = 0; r < nr; r++) y[t * N + n0 + r] = dot_fused_row(fmt, x + t * K, rows[r], K / 32);
            continue;
        }
        for (int64_t i = 0; i < T * 4; i++) acc[i] = 0.0f;
        for (int64_t kb = 0; kb < K; kb += 1024) {
            const int64_t len = K - kb < 1024 ? K - kb : 1024;
            const float* wp[4];
            for (int r = 0; r < 4; r++) {
                float* dst = wbuf + r * 1024;
                const int64_t off = fmt == ORC_F32 ? kb * 4 : fmt == ORC_F16 || fmt == ORC_BF16 ? kb * 2
                                                                     : kb / block_size(fmt) * block_bytes(fmt);
                orc_dequant(fmt, rows[r] + off, len, dst);
                wp[r] = dst;
            }
            float res[8];
            int64_t t = 0;
            for (; T > 4 && t + 2 <= T; t += 2) {
                dot4x2(x + t * K + kb, x + (t + 1) * K + kb, wp, len, res);
                for (int r = 0; r < 4; r++) {
                    acc[t * 4 + r] += res[r];
                    acc[(t + 1) * 4 + r] += res[4 + r];
                }
            }
            for (; t < T; t++) {
                dot4(x + t * K + kb, wp, len, res);
                for (int r = 0; r < 4; r++) acc[t * 4 + r] += res[r];
            }
        }
        for (int64_t t = 0; t < T; t++)
            for (int r = 0; r < nr; r++) y[t * N + n0 + r] = acc[t * 4 + r];
    }
    free(wbuf);
    free(acc);
}

int orc_matvec(int fmt, const uint8_t* w, int64_t N, int64_t K, const float* x, int64_t T, float* y)
{
    if (orc_row_bytes(fmt, K) <= 0 || (fmt >= ORC_Q8_0 && K % 32)) return -1;
    matvec_groups(fmt, w, N, K, x, T, y, 0, (N + 3) / 4);
    return 0;
}

typedef struct {
    int fmt;
    const uint8_t* w;
    int64_t N, K, T, groups, per;
    const float* x;
    float* y;
} mv_ctx;

static void mv_chunk(void* v, int64_t c)
{
    mv_ctx* k = (mv_ctx*)v;
    int64_t g0 = c * k->per, g1 = g0 + k->per < k->groups ? g0 + k->per : k->groups;
    if (g0 < g1) matvec_groups(k->fmt, k->w, k->N, k->K, k->x, k->T, k->y, g0, g1);
}

/* MatMulOp.Run's split (MatMulOp.cs:150-153): chunks = min(groups, threads * 8) over groups of 4 rows. */
int orc_matvec_mt(int fmt, const uint8_t* w, int64_t N, int64_t K, const float* x, int64_t T, float* y)
{
    if (orc_row_bytes(fmt, K) <= 0 || (fmt >= ORC_Q8_0 && K % 32)) return -1;
    const int64_t groups = (N + 3) / 4;
    int64_t ch = groups < (int64_t)g_threads * 8 ? groups : (int64_t)g_threads * 8;
    if (ch < 1) return 0;
    mv_ctx k = {fmt, w, N, K, T, groups, (groups + ch - 1) / ch, x, y};
    parallel_for(ch, mv_chunk, &k);
    return 0;
}

/* ==== Integer-dot matmul: q8 activations x decoded weight codes (IntDot.cs, IntDot.Decode.cs, IntDot.Kernels.cs)
 * The CPU provider's few-row MatMul when integer dots are enabled (MatMulOp.cs:144-146, 173-213). A quantized
 * activation row here is three arrays: q int8 [K], d f32 [K/32] (one block scale per 32 values, the values of
 * Q8Row.LaneScales without their fourfold repetition) and gs f32 [K/16] (Q8Row.GroupSums: d * sum(q) per 16). */

/* .NET's saturating float -> int conversion (NaN -> 0), the cast of IntDot.QuantizeBlockScalar. */
static int32_t sat_i32(float v)
{
    if (v != v) return 0;
    if (v >= 2147483648.0f) return INT32_MAX;
    if (v <= -2147483648.0f) return INT32_MIN;
    return (int32_t)v;
}

/* IntDot.QuantizeBlockScalar (IntDot.cs:92-126), one 32-value block: amax by MathF.Max (NaN-propagating),
 * d = amax / 127, id = 1 / d (0 for d == 0), q = (int)(x * id + copysign(0.5, x * id)) -- round half away from
 * zero through an f32 addition, so x * id = 0.49999997 rounds to 1 -- and the two 16-value group sums d * s. */
static void q8_block(const float* x, int8_t* q, float* d, float* gs)
{
    float amax = 0.0f;
    for (int i = 0; i < 32; i++) {
        const float a = fabsf(x[i]);
        amax = (a != a || amax != amax) ? NAN : (a > amax ? a : amax);
    }
    const float dd = amax / 127.0f;
    const float id = dd != 0.0f ? 1.0f / dd : 0.0f;
    int s0 = 0, s1 = 0;
    for (int i = 0; i < 32; i++) {
        const float v = x[i] * id;
        const int32_t r = sat_i32(v + copysignf(0.5f, v));
        q[i] = (int8_t)(uint8_t)(uint32_t)r;
        if (i < 16) s0 += r;
        else s1 += r;
    }
    *d = dd;
    gs[0] = dd * (float)s0;
    gs[1] = dd * (float)s1;
}

int orc_q8_quantize(const float* x, int64_t rows, int64_t K, int8_t* q, float* d, float* gs)
{
    if (K % 32) return -1;
    for (int64_t r = 0; r < rows; r++)
        for (int64_t b = 0; b < K / 32; b++)
            q8_block(x + r * K + 32 * b, q + r * K + 32 * b, d + r * (K / 32) + b, gs + r * (K / 16) + 2 * b);
    return 0;
}

/* IntDot.Decode (IntDot.Decode.cs:17-293): K values of a weight row -> unsigned codes u [K] and a multiplier a
 * and an offset b per 16 values, value = a * u + b. Formats: IntDot.Supports (IntDot.cs:36-38). */
int orc_intdot_decode(int fmt, const uint8_t* p, int64_t K, uint8_t* u, float* a, float* b)
{
    static const uint8_t iq4u[16] = {1, 24, 45, 63, 79, 93, 106, 118, 129, 141, 153, 166, 181, 197, 217, 241};
    static const uint8_t fp4u[16] = {16, 17, 18, 19, 20, 22, 24, 28, 16, 15, 14, 13, 12, 10, 8, 4};
#define SETB(g, m, o) (a[2 * (g)] = a[2 * (g) + 1] = (m), b[2 * (g)] = b[2 * (g) + 1] = (o))
    switch (fmt) {
    case ORC_Q8_0:
        for (int64_t blk = 0; blk < K / 32; blk++, p += 34) {
            const float dd = rd_h(p);
            for (int i = 0; i < 32; i++) u[32 * blk + i] = (uint8_t)(p[2 + i] ^ 0x80);
            SETB(blk, dd, -128.0f * dd);
        }
        return 0;
    case ORC_Q4_0:
    case ORC_Q4_1: {
        const int m = fmt == ORC_Q4_1, bytes = m ? 20 : 18, qo = m ? 4 : 2;
        for (int64_t blk = 0; blk < K / 32; blk++, p += bytes) {
            const float dd = rd_h(p);
            for (int i = 0; i < 16; i++) {
                u[32 * blk + i] = p[qo + i] & 0xF;
                u[32 * blk + 16 + i] = p[qo + i] >> 4;
            }
            SETB(blk, dd, m ? rd_h(p + 2) : -8.0f * dd);
        }
        return 0;
    }
    case ORC_Q5_0:
    case ORC_Q5_1: {
        const int m = fmt == ORC_Q5_1, bytes = m ? 24 : 22, ho = m ? 4 : 2;
        for (int64_t blk = 0; blk < K / 32; blk++, p += bytes) {
            const float dd = rd_h(p);
            const uint32_t qh = (uint32_t)p[ho] | ((uint32_t)p[ho + 1] << 8) | ((uint32_t)p[ho + 2] << 16) |
                                ((uint32_t)p[ho + 3] << 24);
            for (int i = 0; i < 16; i++) {
                u[32 * blk + i] = (uint8_t)((p[ho + 4 + i] & 0xF) | (((qh >> i) & 1) << 4));
                u[32 * blk + 16 + i] = (uint8_t)((p[ho + 4 + i] >> 4) | (((qh >> (16 + i)) & 1) << 4));
            }
            SETB(blk, dd, m ? rd_h(p + 2) : -16.0f * dd);
        }
        return 0;
    }
    case ORC_Q4_K:
    case ORC_Q5_K: {
        const int five = fmt == ORC_Q5_K, bytes = five ? 176 : 144;
        for (int64_t blk = 0; blk < K / 256; blk++, p += bytes) {
            const float dd = rd_h(p), dmin = rd_h(p + 2);
            const uint8_t* qs = p + (five ? 48 : 16);
            uint8_t* ub = u + 256 * blk;
            for (int j = 0; j < 4; j++)
                for (int i = 0; i < 32; i++) {
                    const uint8_t c = qs[32 * j + i];
                    int lo = c & 0xF, hi = c >> 4;
                    if (five) {
                        const uint8_t h = p[16 + i];
                        lo |= ((h >> (2 * j)) & 1) << 4;
                        hi |= ((h >> (2 * j + 1)) & 1) << 4;
                    }
                    ub[64 * j + i] = (uint8_t)lo;
                    ub[64 * j + 32 + i] = (uint8_t)hi;
                }
            for (int j = 0; j < 8; j++) {
                int sc, mn;
                scale_min(j, p + 4, &sc, &mn);
                SETB(8 * blk + j, dd * (float)sc, -dmin * (float)mn);
            }
        }
        return 0;
    }
    case ORC_Q6_K:
        for (int64_t blk = 0; blk < K / 256; blk++, p += 210) {
            const float dd = rd_h(p + 208);
            uint8_t* ub = u + 256 * blk;
            for (int n = 0; n < 2; n++) {
                const uint8_t* ql = p + 64 * n;
                const uint8_t* qh = p + 128 + 32 * n;
                for (int i = 0; i < 32; i++) {
                    ub[128 * n + i] = (uint8_t)((ql[i] & 0xF) | ((qh[i] & 3) << 4));
                    ub[128 * n + 32 + i] = (uint8_t)((ql[32 + i] & 0xF) | (((qh[i] >> 2) & 3) << 4));
                    ub[128 * n + 64 + i] = (uint8_t)((ql[i] >> 4) | (((qh[i] >> 4) & 3) << 4));
                    ub[128 * n + 96 + i] = (uint8_t)((ql[32 + i] >> 4) | (((qh[i] >> 6) & 3) << 4));
                }
            }
            for (int g = 0; g < 16; g++) {
                const float s = dd * (float)(int8_t)p[192 + g];
                a[16 * blk + g] = s;
                b[16 * blk + g] = -32.0f * s;
            }
        }
        return 0;
    case ORC_IQ4_NL:
        for (int64_t blk = 0; blk < K / 32; blk++, p += 18) {
            const float dd = rd_h(p);
            for (int i = 0; i < 16; i++) {
                u[32 * blk + i] = iq4u[p[2 + i] & 0xF];
                u[32 * blk + 16 + i] = iq4u[p[2 + i] >> 4];
            }
            SETB(blk, dd, -128.0f * dd);
        }
        return 0;
    case ORC_IQ4_XS:
        for (int64_t blk = 0; blk < K / 256; blk++, p += 136) {
            const float dd = rd_h(p);
            const uint32_t sh = (uint32_t)p[2] | ((uint32_t)p[3] << 8);
            for (int ib = 0; ib < 8; ib++) {
                const int ls = ((p[4 + ib / 2] >> (4 * (ib % 2))) & 0xF) | (int)(((sh >> (2 * ib)) & 3) << 4);
                const float dl = dd * (float)(ls - 32);
                for (int i = 0; i < 16; i++) {
                    u[256 * blk + 32 * ib + i] = iq4u[p[8 + 16 * ib + i] & 0xF];
                    u[256 * blk + 32 * ib + 16 + i] = iq4u[p[8 + 16 * ib + i] >> 4];
                }
                SETB(8 * blk + ib, dl, -128.0f * dl);
            }
        }
        return 0;
    case ORC_MXFP4:
        for (int64_t blk = 0; blk < K / 32; blk++, p += 17) {
            const float dd = e8m0_half(p[0]);
            for (int i = 0; i < 16; i++) {
                u[32 * blk + i] = fp4u[p[1 + i] & 0xF];
                u[32 * blk + 16 + i] = fp4u[p[1 + i] >> 4];
            }
            SETB(blk, dd, -16.0f * dd);
        }
        return 0;
    default:
        return -1;
    }
#undef SETB
}

/* IntDot.DotScalar (IntDot.Kernels.cs:12-29): per 16 values the exact integer sum s = sum(u q), then
 * acc += a * d * s + b * gs in f32, group by group. */
float orc_intdot_dot(const uint8_t* u, const float* a, const float* b, const int8_t* q, const float* d, const float* gs,
                     int64_t K)
{
    float acc = 0.0f;
    for (int64_t g = 0; g < K / 16; g++) {
        int32_t s = 0;
        for (int i = 0; i < 16; i++) s += (int32_t)u[16 * g + i] * (int32_t)q[16 * g + i];
        const float t1 = (a[g] * d[g / 2]) * (float)s;
        const float t2 = b[g] * gs[g];
        acc += t1 + t2;
    }
    return acc;
}

/* sum over groups of |a d s| + |b gs|: the magnitude of what the dot adds, for tolerance bounds */
static double intdot_abs(const uint8_t* u, const float* a, const float* b, const int8_t* q, const float* d,
                         const float* gs, int64_t K)
{
    double acc = 0.0;
    for (int64_t g = 0; g < K / 16; g++) {
        int64_t s = 0;
        for (int i = 0; i < 16; i++) s += (int64_t)u[16 * g + i] * (int64_t)q[16 * g + i];
        acc += fabs((double)a[g] * (double)d[g / 2] * (double)s) + fabs((double)b[g] * (double)gs[g]);
    }
    return acc;
}

int orc_intdot_supported(int fmt)
{
    return fmt == ORC_Q8_0 || fmt == ORC_Q4_0 || fmt == ORC_Q4_1 || fmt == ORC_Q5_0 || fmt == ORC_Q5_1 ||
           fmt == ORC_Q4_K || fmt == ORC_Q5_K || fmt == ORC_Q6_K || fmt == ORC_IQ4_NL || fmt == ORC_IQ4_XS ||
           fmt == ORC_MXFP4;
}

typedef struct {
    int fmt;
    const uint8_t* w;
    int64_t N, K, T, per, rowb;
    const int8_t* q;
    const float *d, *gs;
    float* y;
    double* yabs;
} iv_ctx;

static void iv_rows(void* v, int64_t c)
{
    iv_ctx* k = (iv_ctx*)v;
    const int64_t n0 = c * k->per, n1 = n0 + k->per < k->N ? n0 + k->per : k->N;
    if (n0 >= n1) return;
    uint8_t* u = (uint8_t*)malloc((size_t)k->K);
    float* a = (float*)malloc((size_t)(k->K / 16) * 4);
    float* b = (float*)malloc((size_t)(k->K / 16) * 4);
    for (int64_t n = n0; n < n1; n++) {
        orc_intdot_decode(k->fmt, k->w + n * k->rowb, k->K, u, a, b);
        for (int64_t t = 0; t < k->T; t++) {
            const int8_t* q = k->q + t * k->K;
            const float* d = k->d + t * (k->K / 32);
            const float* gs = k->gs + t * (k->K / 16);
            if (k->y) k->y[t * k->N + n] = orc_intdot_dot(u, a, b, q, d, gs, k->K);
            if (k->yabs) k->yabs[t * k->N + n] = intdot_abs(u, a, b, q, d, gs, k->K);
        }
    }
    free(u);
    free(a);
    free(b);
}

/* MatMulOp.RunIntDot (MatMulOp.cs:173-213): quantize the T activation rows, then every weight row decoded once
 * and dotted with each of them; threaded over chunks = clamp(N / 16, 1, threads * 4) row ranges. yabs (may be
 * null): sum |a d s| + |b gs| per output. y may be null when only yabs is wanted. */
static int matvec_q8_impl(int fmt, const uint8_t* w, int64_t N, int64_t K, const float* x, int64_t T, float* y,
                          double* yabs, int threaded)
{
    const int super = fmt == ORC_Q4_K || fmt == ORC_Q5_K || fmt == ORC_Q6_K || fmt == ORC_IQ4_XS;
    if (!orc_intdot_supported(fmt) || K % (super ? 256 : 32)) return -1;
    int8_t* q = (int8_t*)malloc((size_t)(T * K) + 1);
    float* d = (float*)malloc((size_t)(T * (K / 32)) * 4 + 4);
    float* gs = (float*)malloc((size_t)(T * (K / 16)) * 4 + 4);
    orc_q8_quantize(x, T, K, q, d, gs);
    int64_t chunks = threaded ? N / 16 : 1;
    if (chunks < 1) chunks = 1;
    if (threaded && chunks > (int64_t)g_threads * 4) chunks = (int64_t)g_threads * 4;
    iv_ctx k = {fmt, w, N, K, T, (N + chunks - 1) / chunks, orc_row_bytes(fmt, K), q, d, gs, y, yabs};
    if (threaded) parallel_for(chunks, iv_rows, &k);
    else iv_rows(&k, 0);
    free(q);
    free(d);
    free(gs);
    return 0;
}

int orc_matvec_q8(int fmt, const uint8_t* w, int64_t N, int64_t K, const float* x, int64_t T, float* y, double* yabs)
{
    return matvec_q8_impl(fmt, w, N, K, x, T, y, yabs, 0);
}

int orc_matvec_q8_mt(int fmt, const uint8_t* w, int64_t N, int64_t K, const float* x, int64_t T, float* y)
{
    return matvec_q8_impl(fmt, w, N, K, x, T, y, NULL, 1);
}
