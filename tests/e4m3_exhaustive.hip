// Exhaustive checks of the kernels' E4M3 arithmetic (sharplight_amd/csrc/common.hpp):
//  1. e4m3_code / e4m3_pack4 (gfx950's v_cvt_pk_fp8_f32 of fma(v, id, +0) clamped to [-448, 448]) against an
//     integer restatement of the reference's rule (e4m3_code, src/Sharplight.Shaders/Kernels/e4m3.slang:5-23)
//     over all 2^32 f32 bit patterns; it also counts the differences of the bare hardware conversion, which
//     must be nonzero (-0, NaN and the infinities differ), so a checker that compares nothing cannot pass;
//  2. e4m3_group_scale (d = m/448 and id = 1/d by fma-corrected products) against IEEE division for every
//     non-negative, non-NaN f32 amax m.
// Prints: "checked <n> mismatches <m> first <bits> bare_mismatches <b> scale_checked <n2> scale_mismatches
// <m2> first <bits>"; exit status 0 when m == 0 and m2 == 0.
#include "../sharplight_amd/csrc/common.hpp"

#include <cstdio>

using namespace slhip;

// The rule as the reference states it: integer rounding of the f32 bits, nearest-even multiples of 2^-9
// below 2^-6.
__device__ uint32_t rule_code(float v)
{
    const uint32_t sign = v < 0.0f ? 0x80u : 0u;
    const float a = fabsf(v);
    if (a < 0.015625f) return sign | static_cast<uint32_t>(__builtin_rintf(a * 512.0f));
    uint32_t bits = __float_as_uint(a);
    bits += 0x7FFFFu + ((bits >> 20) & 1u);
    const uint32_t c = (bits >> 20) - (120u << 3);
    return sign | (c < 0x7Eu ? c : 0x7Eu);
}

__global__ void check(unsigned long long* counts, uint32_t* first, uint32_t base)
{
    const uint64_t gid = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const uint32_t u0 = base + static_cast<uint32_t>(gid * 4);
    float v[4];
    for (int i = 0; i < 4; i++) v[i] = __uint_as_float(u0 + i);
    const uint32_t packed = e4m3_pack4(v, 1.0f);
    const uint32_t bare = static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(v[0], v[1], 0, false)) & 0xFFFFu;
    int bad = 0, bare_bad = 0;
    for (int i = 0; i < 4; i++) {
        const uint32_t r = rule_code(v[i]);
        const bool b = ((packed >> (8 * i)) & 0xFFu) != r || e4m3_code(v[i]) != r;
        if (b) atomicMin(first, u0 + i);
        bad += b;
        if (i < 2) bare_bad += ((bare >> (8 * i)) & 0xFFu) != r;
    }
    if (bad) atomicAdd(&counts[0], static_cast<unsigned long long>(bad));
    if (bare_bad) atomicAdd(&counts[1], static_cast<unsigned long long>(bare_bad));
}

__global__ void check_scale(unsigned long long* counts, uint32_t* first)
{
    const uint32_t u = blockIdx.x * blockDim.x + threadIdx.x;  // 0 .. 0x7F800000 (+0 .. +inf)
    if (u > 0x7F800000u) return;
    const float m = __uint_as_float(u);
    float d, id;
    e4m3_group_scale(m, d, id);
    const float d_ref = m / 448.0f;
    const float id_ref = d_ref > 0.0f ? 1.0f / d_ref : 0.0f;
    if (__float_as_uint(d) != __float_as_uint(d_ref) || __float_as_uint(id) != __float_as_uint(id_ref)) {
        atomicAdd(&counts[2], 1ull);
        atomicMin(first + 1, u);
    }
}

int main()
{
    unsigned long long* counts = nullptr;
    uint32_t* first = nullptr;
    if (hipMalloc(&counts, 24) != hipSuccess || hipMalloc(&first, 8) != hipSuccess) return 2;
    if (hipMemset(counts, 0, 24) != hipSuccess || hipMemset(first, 0xFF, 8) != hipSuccess) return 2;
    // 2^32 values: 4 launches of 2^28 threads, 4 values each
    for (uint32_t q = 0; q < 4; q++) check<<<(1u << 28) / 256, 256>>>(counts, first, q << 30);
    check_scale<<<(0x7F800000u / 256) + 1, 256>>>(counts, first);
    if (hipDeviceSynchronize() != hipSuccess) return 2;
    unsigned long long c[3];
    uint32_t f[2];
    if (hipMemcpy(c, counts, 24, hipMemcpyDeviceToHost) != hipSuccess ||
        hipMemcpy(f, first, 8, hipMemcpyDeviceToHost) != hipSuccess)
        return 2;
    printf("checked 4294967296 mismatches %llu first 0x%08x bare_mismatches %llu scale_checked %u scale_mismatches "
           "%llu first 0x%08x\n", c[0], f[0], c[1], 0x7F800001u, c[2], f[1]);
    (void)hipFree(counts);
    (void)hipFree(first);
    return c[0] == 0 && c[2] == 0 ? 0 : 1;
}
