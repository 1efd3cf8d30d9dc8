// Exhaustive check of recip_nr / recip_ieee (sharplight_amd/csrc/common.hpp), the reciprocal the row-norm
// scales use: for every positive f32 s in [2^-125, 2^125], recip_nr(s) (hardware reciprocal plus one Newton
// step) must equal the IEEE quotient 1.0f / s bit for bit; over all 2^32 bit patterns recip_ieee(s) must equal
// it (NaNs compared as NaN). The bare hardware reciprocal is counted too and must differ somewhere, so a
// checker that compares nothing cannot pass.
// Prints: "checked <n> nr_mismatches <a> ieee_mismatches <b> bare_mismatches <c> first <bits>"; exit status 0
// when a == 0 and b == 0 and c > 0.
#include "../sharplight_amd/csrc/common.hpp"

#include <cstdio>

using namespace slhip;

__global__ void check(unsigned long long* counts, uint32_t* first, uint32_t base)
{
    const uint64_t gid = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const uint32_t u0 = base + static_cast<uint32_t>(gid * 4);
    int nr_bad = 0, ieee_bad = 0, bare_bad = 0;
    for (int i = 0; i < 4; i++) {
        const uint32_t u = u0 + i;
        const float s = __uint_as_float(u);
        const float q = 1.0f / s;
        const float r = recip_ieee(s);
        const bool same = __float_as_uint(r) == __float_as_uint(q) || (r != r && q != q);
        if (!same) {
            ieee_bad++;
            atomicMin(first, u);
        }
        const float a = fabsf(s);
        if (a >= 0x1p-125f && a <= 0x1p125f) {
            if (__float_as_uint(recip_nr(s)) != __float_as_uint(q)) {
                nr_bad++;
                atomicMin(first, u);
            }
            bare_bad += __float_as_uint(__builtin_amdgcn_rcpf(s)) != __float_as_uint(q);
        }
    }
    if (nr_bad) atomicAdd(&counts[0], static_cast<unsigned long long>(nr_bad));
    if (ieee_bad) atomicAdd(&counts[1], static_cast<unsigned long long>(ieee_bad));
    if (bare_bad) atomicAdd(&counts[2], static_cast<unsigned long long>(bare_bad));
}

int main()
{
    unsigned long long* counts = nullptr;
    uint32_t* first = nullptr;
    if (hipMalloc(&counts, 3 * sizeof(unsigned long long)) != hipSuccess || hipMalloc(&first, 4) != hipSuccess) return 2;
    hipMemset(counts, 0, 3 * sizeof(unsigned long long));
    hipMemset(first, 0xFF, 4);
    // 2^32 patterns: 2^30 threads of 4, in 4 launches of 2^28 threads
    for (uint64_t part = 0; part < 4; part++) {
        check<<<dim3(1u << 20), 256>>>(counts, first, static_cast<uint32_t>(part << 30));
        if (hipDeviceSynchronize() != hipSuccess) return 3;
    }
    unsigned long long h[3];
    uint32_t f;
    hipMemcpy(h, counts, sizeof h, hipMemcpyDeviceToHost);
    hipMemcpy(&f, first, 4, hipMemcpyDeviceToHost);
    printf("checked %llu nr_mismatches %llu ieee_mismatches %llu bare_mismatches %llu first 0x%08x\n", 1ull << 32, h[0],
           h[1], h[2], f);
    return h[0] == 0 && h[1] == 0 && h[2] > 0 ? 0 : 1;
}
