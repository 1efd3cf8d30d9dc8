// Element type conversion between f32, f16 and bf16 activations (the CPU provider's Cast of
// activations; f32 -> bf16 rounding is Simd.FloatToBFloat, src/Sharplight.Cpu/Simd.cs:530-540).
// Streaming kernel: 8 elements per lane per step (16-byte loads of the 2-byte types, 2x16-byte of f32).
#include "common.hpp"

namespace slhip {

template <int DI, int DO>
__device__ __forceinline__ void cvt8(const void* x, void* y, int64_t i8)
{
    float f[8];
    if (DI == SLHIP_F32) {
        const char* p = static_cast<const char*>(x) + 32 * i8;
        Vec<SLHIP_F32>::unpack(load_nt(p), f);
        Vec<SLHIP_F32>::unpack(load_nt(p + 16), f + 4);
    } else {
        Vec<DI>::unpack(load_nt(static_cast<const char*>(x) + 16 * i8), f);
    }
    store_packed<DO, 8>(static_cast<char*>(y) + i8 * 8 * Vec<DO>::BYTES, f);
}

template <int DI, int DO>
__global__ __launch_bounds__(256) void convert_vec(const void* x, void* y, int64_t n8)
{
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n8; i += static_cast<int64_t>(gridDim.x) * 256)
        cvt8<DI, DO>(x, y, i);
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
    const bool vec = n % 8 == 0 && aligned16(x) && aligned16(y);
    const int64_t work = vec ? n / 8 : n;
    const int64_t blocks = (work + 255) / 256;
    const unsigned grid = static_cast<unsigned>(blocks < 8192 ? blocks : 8192);
    if (vec) convert_vec<DI, DO><<<grid, 256, 0, st>>>(x, y, n / 8);
    else convert_scalar<DI, DO><<<grid, 256, 0, st>>>(x, y, n);
    return check_launch("convert");
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
