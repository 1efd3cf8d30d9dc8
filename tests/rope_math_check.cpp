// Host check of the rope kernels' sin/cos (sharplight_amd/csrc/rope_math.hpp) against f64 libm narrowed
// to f32: prints the ulp histogram and the worst case over rotary angles pos * base^(-2i/dims) for three
// bases and three head sizes, positions 0..65535, plus 2M uniform angles in [-2e5, 2e5].
#include "../sharplight_amd/csrc/rope_math.hpp"

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>

static int ulp_diff(float a, float b)
{
    int32_t x, y;
    memcpy(&x, &a, 4);
    memcpy(&y, &b, 4);
    if ((x < 0) != (y < 0)) return a == b ? 0 : 1 << 30;
    return abs(x - y);
}

int main()
{
    long n = 0, exact = 0;
    int worst = 0;
    double worst_theta = 0;
    auto check = [&](double th) {
        float s, c;
        slhip::sincos_f64_to_f32(th, &s, &c);
        const int u = std::max(ulp_diff(s, static_cast<float>(sin(th))), ulp_diff(c, static_cast<float>(cos(th))));
        if (u > worst) {
            worst = u;
            worst_theta = th;
        }
        exact += u == 0;
        n++;
    };
    for (double base : {1e6, 1e4, 5e5})
        for (int dims : {64, 128, 256})
            for (int p = 0; p < 65536; p += 7)
                for (int i = 0; i < dims / 2; i++) check(p * pow(base, -2.0 * i / dims));
    std::mt19937_64 g(5);
    std::uniform_real_distribution<double> u(-2e5, 2e5);
    for (int k = 0; k < 2000000; k++) check(u(g));
    printf("angles %ld exact %ld worst_ulp %d at %.17g\n", n, exact, worst, worst_theta);
    return 0;
}
