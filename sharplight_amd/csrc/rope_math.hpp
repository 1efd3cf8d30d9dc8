// f64 sine/cosine used for rotary angles; host- and device-callable so the host tests can check it
// against libm.
#pragma once

#include <hip/hip_runtime.h>

#include <cmath>

namespace slhip {

// sin and cos of an f64 angle as f32: Cody-Waite reduction by pi/2 in f64 (pi/2 split in two f64 parts,
// the products fused, so the reduction is exact to ~1e-16 for |theta| < 2^40; this is the part that needs
// f64: at theta ~ 3e4 an f32 argument would already be off by ~1e-3), then the reduced angle split as
// r = rh + rl (rh = (float)r) and Taylor series of sin/cos of rh to r^9 / r^10 evaluated in f32
// (truncation < 2e-9 on |r| <= pi/4), corrected to first order by rl. Within ~1 f32 ulp of
// (float)sin/cos(theta) of a correctly rounded f64 libm (checked on 8.3M angles, tests/rope_math_check.cpp),
// with a third of the f64 instructions of an all-f64 evaluation.
__host__ __device__ inline void sincos_f64_to_f32(double theta, float* s_out, float* c_out)
{
    const double kTwoOverPi = 0.63661977236758134308;
    const double kPio2Hi = 1.5707963267948966;
    const double kPio2Lo = 6.123233995736766e-17;
    const double k = rint(theta * kTwoOverPi);
    double r = fma(-k, kPio2Hi, theta);
    r = fma(-k, kPio2Lo, r);
    const float rh = static_cast<float>(r);
    const float rl = static_cast<float>(r - static_cast<double>(rh));
    const float r2 = rh * rh;
    // sin rh = rh + rh^3 (-1/3! + rh^2/5! - rh^4/7! + rh^6/9!)
    float ps = 1.0f / 362880.0f;
    ps = fmaf(ps, r2, -1.0f / 5040.0f);
    ps = fmaf(ps, r2, 1.0f / 120.0f);
    ps = fmaf(ps, r2, -1.0f / 6.0f);
    float sn = fmaf(ps * r2, rh, rh);
    // cos rh = 1 + rh^2 (-1/2! + rh^2/4! - rh^4/6! + rh^6/8! - rh^8/10!)
    float pc = -1.0f / 3628800.0f;
    pc = fmaf(pc, r2, 1.0f / 40320.0f);
    pc = fmaf(pc, r2, -1.0f / 720.0f);
    pc = fmaf(pc, r2, 1.0f / 24.0f);
    pc = fmaf(pc, r2, -0.5f);
    float cn = fmaf(pc, r2, 1.0f);
    // sin(rh + rl) ~ sin rh + rl cos rh, cos(rh + rl) ~ cos rh - rl sin rh (rl <= 2^-25 |rh|)
    const float s1 = fmaf(rl, cn, sn);
    const float c1 = fmaf(-rl, sn, cn);
    sn = s1;
    cn = c1;
    const int q = static_cast<int>(static_cast<long long>(k) & 3);
    const float s = (q & 1) ? cn : sn;
    const float c = (q & 1) ? sn : cn;
    *s_out = (q & 2) ? -s : s;
    *c_out = ((q + 1) & 2) ? -c : c;
}

}  // namespace slhip
