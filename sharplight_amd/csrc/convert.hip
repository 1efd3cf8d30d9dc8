// Element type conversion between f32, f16 and bf16 activations (the CPU provider's Cast of
// activations; f32 -> bf16 rounding is Simd.FloatToBFloat, src/Sharplight.Cpu/Simd.cs:530-540).
//
// Layout: a wave converts 512 consecutive elements per step as two groups of 4 per lane -- elements
// [4l, 4l+4) and [256+4l, 256+4l+4) -- so that every load and store instruction of the wave covers one
// contiguous span (512 B or 1 KiB) whatever the two element sizes are; between two 2-byte types a lane takes 8
// contiguous elements, one 16-byte access each way. (Giving each lane 8 contiguous
// elements instead would make the wider side's two 16-byte accesses per lane land 32 bytes apart, and a
// store instruction would then half-fill every 64-byte segment it touches: measured 1.6x the write traffic
// and 35% less bandwidth on MI355X.) The last, partial chunk is converted one element per lane by its wave,
// within the same launch.
#include "common.hpp"

namespace slhip {

// Loads / stores 4 consecutive elements of dtype DT (16 bytes for f32, 8 bytes for f16/bf16).
template <int DT> __device__ __forceinline__ void load4(const char* p, float* f)
{
    if (DT == SLHIP_F32) {
        Vec<SLHIP_F32>::unpack(load_nt(p), f);
    } else {
        const u32x2 v = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(p));
        if (DT == SLHIP_BF16) {
            f[0] = bf16_lo(v.x); f[1] = bf16_hi(v.x); f[2] = bf16_lo(v.y); f[3] = bf16_hi(v.y);
        } else {
            f[0] = f16_lo(v.x); f[1] = f16_hi(v.x); f[2] = f16_lo(v.y); f[3] = f16_hi(v.y);
        }
    }
}

template <int DI, int DO>
__global__ __launch_bounds__(256) void convert_vec(const void* x, void* y, int64_t n)
{
    const int64_t chunk = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);  // 512 elements each
    const int64_t chunks = (n + 511) / 512;
    if (chunk >= chunks) return;
    const int lane = threadIdx.x & 63;
    if (chunk * 512 + 512 > n) {  // the last, partial chunk (wave-uniform): one element per lane and step
        for (int64_t i = chunk * 512 + lane; i < n; i += 64) Vec<DO>::store1(y, i, Vec<DI>::load1(x, i));
        return;
    }
    if constexpr (DI != SLHIP_F32 && DO != SLHIP_F32) {
        // Both sides 2 bytes wide: 8 consecutive elements per lane, one 16-byte load and one 16-byte store
        // (8-byte accesses measured ~10% slower at 84 MB).
        const int64_t e = chunk * 512 + 8 * lane;
        float f[8];
        Vec<DI>::unpack(load_nt(static_cast<const char*>(x) + e * 2), f);
        store_packed<DO, 8>(static_cast<char*>(y) + e * 2, f);
        return;
    }
    const int64_t e0 = chunk * 512 + 4 * lane;
    float f0[4], f1[4];
    load4<DI>(static_cast<const char*>(x) + e0 * Vec<DI>::BYTES, f0);
    load4<DI>(static_cast<const char*>(x) + (e0 + 256) * Vec<DI>::BYTES, f1);
    store_packed<DO, 4>(static_cast<char*>(y) + e0 * Vec<DO>::BYTES, f0);
    store_packed<DO, 4>(static_cast<char*>(y) + (e0 + 256) * Vec<DO>::BYTES, f1);
}

template <int DI, int DO>
__global__ __launch_bounds__(256) void convert_scalar(const void* x, void* y, int64_t n)
{
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n; i += static_cast<int64_t>(gridDim.x) * 256)
        Vec<DO>::store1(y, i, Vec<DI>::load1(x, i));
}

template <int DI, int DO>
static int run(const void* x, void* y, int64_t n, hipStream_t st)
{
    if (aligned16(x) && aligned16(y)) {  // one launch, the partial last chunk included
        const int64_t blocks = ((n + 511) / 512 + 3) / 4;
        if (blocks > 0x7FFFFFFF) return fail(SLHIP_ERR_UNSUPPORTED, "convert: %lld elements", static_cast<long long>(n));
        convert_vec<DI, DO><<<static_cast<unsigned>(blocks), 256, 0, st>>>(x, y, n);
        return check_launch("convert_vec");
    }
    const int64_t blocks = (n + 255) / 256;
    convert_scalar<DI, DO><<<static_cast<unsigned>(blocks < 8192 ? blocks : 8192), 256, 0, st>>>(x, y, n);
    return check_launch("convert_scalar");
}

template <int DI>
static int by_out(int dout, const void* x, void* y, int64_t n, hipStream_t st)
{
    switch (dout) {
    case SLHIP_F32: return run<DI, SLHIP_F32>(x, y, n, st);
    case SLHIP_F16: return run<DI, SLHIP_F16>(x, y, n, st);
    case SLHIP_BF16: return run<DI, SLHIP_BF16>(x, y, n, st);
    default: return fail(SLHIP_ERR_UNSUPPORTED, "convert: dtype %d not supported", dout);
    }
}

}  // namespace slhip

using namespace slhip;

extern "C" SLHIP_API int slhip_convert(int dtype_in, int dtype_out, const void* x, void* y, int64_t n,
                                       slhip_stream stream)
{
    if (n < 0) return fail(SLHIP_ERR_INVALID, "convert: negative size");
    if (n == 0) return SLHIP_OK;
    if (!x || !y) return fail(SLHIP_ERR_INVALID, "convert: null tensor");
    hipStream_t st = to_stream(stream);
    switch (dtype_in) {
    case SLHIP_F32: return by_out<SLHIP_F32>(dtype_out, x, y, n, st);
    case SLHIP_F16: return by_out<SLHIP_F16>(dtype_out, x, y, n, st);
    case SLHIP_BF16: return by_out<SLHIP_BF16>(dtype_out, x, y, n, st);
    default: return fail(SLHIP_ERR_UNSUPPORTED, "convert: dtype %d not supported", dtype_in);
    }
}
