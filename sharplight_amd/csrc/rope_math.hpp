// f64 sine/cosine used for rotary angles; host- and device-callable so the host tests can check it
// against libm.
#pragma once

#include <hip/hip_runtime.h>

#include <cmath>

namespace slhip {

// sin and cos of an f64 angle: Cody-Waite reduction by pi/2 (pi/2 split in two f64 parts, the products
// fused so the reduction is exact to ~1e-16 for |theta| < 2^40), then the Taylor series of sin and cos on
// |r| <= pi/4 up to r^17 / r^18 (truncation < 1e-19), in f64 Horner form. Narrowed to f32 the result
// matches (float)cos(theta) of a correctly rounded libm except when the f64 value lies within ~1e-16 of an
// f32 rounding boundary.
__host__ __device__ inline void sincos_f64(double theta, double* s_out, double* c_out)
{
    const double kTwoOverPi = 0.63661977236758134308;
    const double kPio2Hi = 1.5707963267948966;     // pi/2 rounded to f64
    const double kPio2Lo = 6.123233995736766e-17;  // pi/2 - kPio2Hi
    const double k = rint(theta * kTwoOverPi);
    double r = fma(-k, kPio2Hi, theta);
    r = fma(-k, kPio2Lo, r);
    const double r2 = r * r;
    // sin r = r + r^3 (-1/3! + r^2/5! - r^4/7! + ... + r^14/17!)
    double ps = 1.0 / 355687428096000.0;  // 1/17!
    ps = fma(ps, r2, -1.0 / 1307674368000.0);
    ps = fma(ps, r2, 1.0 / 6227020800.0);
    ps = fma(ps, r2, -1.0 / 39916800.0);
    ps = fma(ps, r2, 1.0 / 362880.0);
    ps = fma(ps, r2, -1.0 / 5040.0);
    ps = fma(ps, r2, 1.0 / 120.0);
    ps = fma(ps, r2, -1.0 / 6.0);
    const double sn = fma(ps * r2, r, r);
    // cos r = 1 + r^2 (-1/2! + r^2/4! - r^4/6! + ... - r^16/18!)
    double pc = -1.0 / 6402373705728000.0;  // -1/18!
    pc = fma(pc, r2, 1.0 / 20922789888000.0);
    pc = fma(pc, r2, -1.0 / 87178291200.0);
    pc = fma(pc, r2, 1.0 / 479001600.0);
    pc = fma(pc, r2, -1.0 / 3628800.0);
    pc = fma(pc, r2, 1.0 / 40320.0);
    pc = fma(pc, r2, -1.0 / 720.0);
    pc = fma(pc, r2, 1.0 / 24.0);
    pc = fma(pc, r2, -0.5);
    const double cn = fma(pc, r2, 1.0);
    const int q = static_cast<int>(static_cast<long long>(k) & 3);
    const double s = (q & 1) ? cn : sn;
    const double c = (q & 1) ? sn : cn;
    *s_out = (q & 2) ? -s : s;
    *c_out = ((q + 1) & 2) ? -c : c;
}

}  // namespace slhip
