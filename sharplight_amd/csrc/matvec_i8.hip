// Integer-dot decode matvec: activations quantized to int8 per 32 values, weight codes multiplied with them in
// exact int32 sums, the block scales applied once per 16 or 32 values in f32 -- the numerics of the reference's
// few-row MatMul when integer dots are enabled (src/Sharplight.Cpu/MatMulOp.cs:144-146,173-213; IntDot.cs,
// IntDot.Decode.cs, IntDot.Kernels.cs:12-29) and of the Vulkan lowerer's int-dot matvec (GraphLowerer.IntDot.cs,
// Kernels/mmvq.slang), which both quantize x to q8 unless the MatMul carries f32_activations.
//
// Quantized activation rows (slhip_quantize_q8), 1.5 K bytes per row, K a multiple of 32:
//   q  int8 [K]            round-half-away(x / d), per 32-value block d = amax / 127 (IntDot.QuantizeBlockScalar)
//   s  f32x4 [K / 32]      {d, d * sum(q[0..15]), d * sum(q[16..31]), 0} per block (Q8Row.LaneScales /
//                          GroupSums: the CPU provider keeps d four times per block and the sums per 16 values)
// The quantization is bit for bit the reference's (the f32 operations in its order, .NET's saturating casts).
//
// The dot: a weight row is read as 32-value units (a block of the 32-value formats, a sub-block of the
// 256-value ones), each decoded to 32 int8 codes and a multiplier a and offset b per 16 values, so that
// w = a * code + b (IntDot.Decode's u, a, b; Q8_0 and the codebook formats keep their signed codes with b = 0,
// the reference's unsigned codes minus 128 or 16 -- the same exact integers). Per unit and token:
//   s0 = sum of the first 16 code * q products, s1 the second (v_dot4c_i32_i8: exact int32),
//   y += a0 * (d * s0) + a1 * (d * s1) + b0 * gs0 + b1 * gs1
// (a0 = a1, b0 = b1 for the formats with one scale per 32 values: a * (d * (s0 + s1)) + b * (gs0 + gs1)).
// The f32 sums run in another order than the CPU provider's group-by-group loop (whose own ISA tiers differ in
// their order too), so the result agrees with it within f32 accumulation of the terms, not bit for bit.
//
// Schedule (matvec_i8): persistent blocks of 4 waves; a wave takes a weight row (a gate/up row pair for the
// dual form) at a time, copies its image to the wave's LDS region with 16-byte loads (narrower for rows that
// are not 16-byte multiples) and issues the next row's loads before computing the current one; the block's TT
// quantized activation rows are staged in LDS once. Each lane takes whole 32-value units (lane, lane + 64, ...).
#include "matvec_i8.hpp"

#include <stdlib.h>

#include <mutex>

namespace slhip {

__device__ __forceinline__ int32_t sat_i32(float v)
{
    // .NET's saturating float -> int conversion: NaN -> 0, out of range -> the nearest end
    return v != v ? 0 : v >= 2147483648.0f ? INT_MAX : v <= -2147483648.0f ? INT_MIN : static_cast<int32_t>(v);
}

// One lane per four values, eight lanes per 32-value block (K % 32 == 0, so a block never spans two rows and a
// group of eight lanes is wholly inside or wholly past the end). IntDot.QuantizeBlockScalar (IntDot.cs:92-126):
// amax (NaN propagating), d = amax / 127, id = d != 0 ? 1 / d : 0, q = (int)(x id + copysign(0.5, x id)),
// group sums d * s per 16 values.
template <int DT>
__global__ __launch_bounds__(256) void quantize_q8(const void* x, int64_t xs, int64_t T, int64_t K, uint8_t* xq)
{
    const int64_t per_row = K / 4;
    const int64_t total = T * per_row;
    const int64_t i0 = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    const bool live = i0 < total;
    const int64_t i = live ? i0 : total - 1;
    const int64_t t = i / per_row, k4 = i - t * per_row;
    float v[4];
    if (DT == SLHIP_F32) {
        const float4 f = reinterpret_cast<const float4*>(static_cast<const float*>(x) + t * xs)[k4];
        v[0] = f.x; v[1] = f.y; v[2] = f.z; v[3] = f.w;
    } else {
        const uint2 b = reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(x) + t * xs)[k4];
        v[0] = bf16_lo(b.x); v[1] = bf16_hi(b.x); v[2] = bf16_lo(b.y); v[3] = bf16_hi(b.y);
    }
    float m = 0.0f;
    int nan = 0;
#pragma unroll
    for (int e = 0; e < 4; e++) {
        m = fmaxf(m, fabsf(v[e]));
        nan |= v[e] != v[e];
    }
#pragma unroll
    for (int o = 1; o < 8; o <<= 1) {
        m = fmaxf(m, __shfl_xor(m, o));
        nan |= __shfl_xor(nan, o);
    }
    const float amax = nan ? __builtin_nanf("") : m;
    const float d = __fdiv_rn(amax, 127.0f);
    const float id = d != 0.0f ? __fdiv_rn(1.0f, d) : 0.0f;
    int32_t r[4];
    int s = 0;
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const float p = __fmul_rn(v[e], id);
        r[e] = sat_i32(__fadd_rn(p, copysignf(0.5f, p)));
        s += r[e];
    }
    s += __shfl_xor(s, 1);
    s += __shfl_xor(s, 2);  // the sum of the lane's 16-value group (lanes 0-3 or 4-7 of the block)
    const int s_hi = __shfl_xor(s, 4);
    if (!live) return;
    uint8_t* row = xq + t * (K + K / 2);
    reinterpret_cast<uint32_t*>(row)[k4] = (static_cast<uint32_t>(r[0]) & 0xFFu) |
                                           ((static_cast<uint32_t>(r[1]) & 0xFFu) << 8) |
                                           ((static_cast<uint32_t>(r[2]) & 0xFFu) << 16) |
                                           (static_cast<uint32_t>(r[3]) << 24);
    if ((k4 & 7) == 0)
        reinterpret_cast<float4*>(row + K)[k4 >> 3] =
            make_float4(d, __fmul_rn(d, static_cast<float>(s)), __fmul_rn(d, static_cast<float>(s_hi)), 0.0f);
}

bool matvec_q8_supported(int fmt) { return i8_geom(fmt).bs != 0; }

bool matvec_q8_fits(int fmt, int64_t K, bool dual)
{
    const I8Geom g = i8_geom(fmt);
    if (g.bs == 0 || K <= 0 || K % g.bs != 0 || (K / g.bs * g.bb) % 2 != 0) return false;
    return i8_lds(1, K, K / g.bs * g.bb, dual) <= kI8MaxLds;
}

int quantize_q8_common(int dtype_x, const void* x, int64_t x_stride, int64_t T, int64_t K, void* xq, hipStream_t st)
{
    if (T < 0 || K < 0) return fail(SLHIP_ERR_INVALID, "quantize_q8: negative shape");
    if (T == 0 || K == 0) return SLHIP_OK;
    if (K % 32 != 0) return fail(SLHIP_ERR_UNSUPPORTED, "quantize_q8: K = %lld must be a multiple of 32", static_cast<long long>(K));
    if (!x || !xq) return fail(SLHIP_ERR_INVALID, "quantize_q8: null pointer");
    if (dtype_x != SLHIP_F32 && dtype_x != SLHIP_BF16) return fail(SLHIP_ERR_UNSUPPORTED, "quantize_q8: x is f32 or bf16");
    if (x_stride < K) return fail(SLHIP_ERR_INVALID, "quantize_q8: the row stride is smaller than the row");
    if (!aligned16(x) || !aligned16(xq) || x_stride % 4 != 0)
        return fail(SLHIP_ERR_UNSUPPORTED, "quantize_q8: x and xq must be 16-byte aligned, the stride a multiple of 4");
    if (T * K / 4 > 0x7FFFFFFFLL * 256) return fail(SLHIP_ERR_UNSUPPORTED, "quantize_q8: shape too large");
    const int64_t groups = T * (K / 4);
    const dim3 grid(static_cast<unsigned>((groups + 255) / 256));
    if (dtype_x == SLHIP_F32)
        quantize_q8<SLHIP_F32><<<grid, 256, 0, st>>>(x, x_stride, T, K, static_cast<uint8_t*>(xq));
    else
        quantize_q8<SLHIP_BF16><<<grid, 256, 0, st>>>(x, x_stride, T, K, static_cast<uint8_t*>(xq));
    return check_launch("quantize_q8");
}

int matvec_q8_common(int fmt, int dtype_y, const void* xq, int64_t T, int64_t K, const void* wg, const void* wu,
                     int64_t N, void* y, int64_t y_stride, const float* bias, int act, bool dual, hipStream_t st)
{
    const char* name = dual ? "dual_matvec_q8" : "matvec_q8";
    if (T < 0 || K < 0 || N < 0) return fail(SLHIP_ERR_INVALID, "%s: negative shape", name);
    if (T == 0 || N == 0) return SLHIP_OK;
    if (K == 0) return fail(SLHIP_ERR_INVALID, "%s: K must be positive", name);
    if (!xq || !wg || !y || (dual && !wu)) return fail(SLHIP_ERR_INVALID, "%s: null pointer", name);
    if (dual && (act < SLHIP_ACT_SILU || act > SLHIP_ACT_GELU_ERF)) return fail(SLHIP_ERR_INVALID, "%s: bad activation %d", name, act);
    if (dtype_y != SLHIP_F32 && dtype_y != SLHIP_BF16) return fail(SLHIP_ERR_UNSUPPORTED, "%s: outputs are f32 or bf16", name);
    if (y_stride < N) return fail(SLHIP_ERR_INVALID, "%s: the output row stride is smaller than the row", name);
    const I8Geom g = i8_geom(fmt);
    if (g.bs == 0) return fail(SLHIP_ERR_UNSUPPORTED, "%s: weight format %d has no integer-dot decoder", name, fmt);
    if (K % g.bs != 0)
        return fail(SLHIP_ERR_UNSUPPORTED, "%s: K = %lld must be a multiple of %d for this format", name,
                    static_cast<long long>(K), g.bs);
    if ((K / g.bs * g.bb) % 2 != 0)
        return fail(SLHIP_ERR_UNSUPPORTED, "%s: rows of an odd number of bytes (%lld) are not supported", name,
                    static_cast<long long>(K / g.bs * g.bb));
    if (!aligned16(xq) || !aligned16(wg) || (dual && !aligned16(wu)))
        return fail(SLHIP_ERR_UNSUPPORTED, "%s: the quantized rows and the weights must be 16-byte aligned", name);
    if (N > 0x7FFFFFFF || T > 0x7FFFFFFF) return fail(SLHIP_ERR_UNSUPPORTED, "%s: shape too large", name);
    I8Args a{static_cast<const uint8_t*>(xq), static_cast<const char*>(wg), static_cast<const char*>(wu),
             K / g.bs * g.bb, y, y_stride, T, K, N, 0, dtype_y, act, dual ? nullptr : bias};
    switch (fmt) {
    case SLHIP_FMT_Q8_0:
    case SLHIP_FMT_Q4_0:
    case SLHIP_FMT_Q4_1: return run_i8_part0(fmt, a, dual, st);
    case SLHIP_FMT_Q5_0:
    case SLHIP_FMT_Q5_1:
    case SLHIP_FMT_IQ4_NL: return run_i8_part1(fmt, a, dual, st);
    case SLHIP_FMT_MXFP4:
    case SLHIP_FMT_IQ4_XS:
    case SLHIP_FMT_Q6_K: return run_i8_part2(fmt, a, dual, st);
    default: return run_i8_part3(fmt, a, dual, st);
    }
}

// The decode FFN's gate/up projections in one call: x quantized into `work` (at least T q8 rows), then the
// dual integer-dot matvec. The no-allocation variant below runs the same two kernels on a file-scope device
// array instead of `work`.
int dual_int8_common(int act, int fmt, int dtype_x, int dtype_y, const void* x, int64_t x_stride, int64_t T, int64_t K,
                     const void* wg, const void* wu, int64_t N, void* y, int64_t y_stride, void* work, int64_t work_bytes,
                     hipStream_t st)
{
    if (T < 0 || K < 0) return fail(SLHIP_ERR_INVALID, "dual_matvec_int8: negative shape");
    if (T == 0 || N == 0) return SLHIP_OK;
    const int64_t need = T * (K + K / 2);
    if (!work || work_bytes < need)
        return fail(SLHIP_ERR_INVALID, "dual_matvec_int8: the workspace holds %lld bytes, %lld needed",
                    static_cast<long long>(work ? work_bytes : 0), static_cast<long long>(need));
    const int r = quantize_q8_common(dtype_x, x, x_stride, T, K, work, st);
    if (r != SLHIP_OK) return r;
    return matvec_q8_common(fmt, dtype_y, work, T, K, wg, wu, N, y, y_stride, nullptr, act, true, st);
}

// The no-allocation variant's workspace: 1 MiB per device (T * 1.5 K bytes, e.g. 32 rows of K = 16384 or 170 of
// K = 4096), held by every GPU the library runs on until the process ends. Host code reaches it only through the
// device address hipGetSymbolAddress gives, once per device.
constexpr int64_t kStaticWorkBytes = int64_t{1} << 20;
static __device__ __align__(256) uint8_t scratch[kStaticWorkBytes];

constexpr int kMaxDevices = 64;
static void* g_scratch_ptr[kMaxDevices];
static std::mutex g_scratch_mu;

static int static_work(void** out)
{
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
        return fail(SLHIP_ERR_HIP, "dual_matvec_int8_noalloc: no current device");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) return fail(SLHIP_ERR_HIP, "dual_matvec_int8_noalloc: workspace address: %s", hipGetErrorString(e));
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return SLHIP_OK;
}

}  // namespace slhip

using namespace slhip;

extern "C" SLHIP_API int slhip_dual_matvec_int8(int act, int fmt, int dtype_x, int dtype_y, const void* x,
                                                int64_t x_stride, int64_t T, int64_t K, const void* w_gate,
                                                const void* w_up, int64_t N, void* y, int64_t y_stride, void* work,
                                                int64_t work_bytes, slhip_stream stream)
{
    return dual_int8_common(act, fmt, dtype_x, dtype_y, x, x_stride, T, K, w_gate, w_up, N, y, y_stride, work,
                            work_bytes, to_stream(stream));
}

extern "C" SLHIP_API int slhip_dual_matvec_int8_noalloc(int act, int fmt, int dtype_x, int dtype_y, const void* x,
                                                        int64_t x_stride, int64_t T, int64_t K, const void* w_gate,
                                                        const void* w_up, int64_t N, void* y, int64_t y_stride,
                                                        slhip_stream stream)
{
    if (T > 0 && K > 0 && T * (K + K / 2) > kStaticWorkBytes)
        return fail(SLHIP_ERR_UNSUPPORTED,
                    "dual_matvec_int8_noalloc: %lld rows of K = %lld need %lld bytes of workspace, above the static %lld",
                    static_cast<long long>(T), static_cast<long long>(K), static_cast<long long>(T * (K + K / 2)),
                    static_cast<long long>(kStaticWorkBytes));
    if (T <= 0 || N <= 0)  // the shape checks (and the empty no-op) of the workspace form
        return dual_int8_common(act, fmt, dtype_x, dtype_y, x, x_stride, T, K, w_gate, w_up, N, y, y_stride, nullptr, 0,
                                to_stream(stream));
    void* work = nullptr;
    const int r = static_work(&work);
    if (r != SLHIP_OK) return r;
    return dual_int8_common(act, fmt, dtype_x, dtype_y, x, x_stride, T, K, w_gate, w_up, N, y, y_stride, work,
                            kStaticWorkBytes, to_stream(stream));
}

extern "C" SLHIP_API int64_t slhip_q8_row_bytes(int64_t K) { return K < 0 ? 0 : K + K / 2; }

extern "C" SLHIP_API int slhip_quantize_q8(int dtype_x, const void* x, int64_t x_stride, int64_t T, int64_t K, void* xq,
                                           slhip_stream stream)
{
    return quantize_q8_common(dtype_x, x, x_stride, T, K, xq, to_stream(stream));
}

extern "C" SLHIP_API int slhip_matvec_q8(int fmt, int dtype_y, const void* xq, int64_t T, int64_t K, const void* w,
                                         int64_t N, void* y, int64_t y_stride, const float* bias, slhip_stream stream)
{
    return matvec_q8_common(fmt, dtype_y, xq, T, K, w, nullptr, N, y, y_stride, bias, 0, false, to_stream(stream));
}

extern "C" SLHIP_API int slhip_dual_matvec_q8(int act, int fmt, int dtype_y, const void* xq, int64_t T, int64_t K,
                                              const void* w_gate, const void* w_up, int64_t N, void* y, int64_t y_stride,
                                              slhip_stream stream)
{
    return matvec_q8_common(fmt, dtype_y, xq, T, K, w_gate, w_up, N, y, y_stride, nullptr, act, true, to_stream(stream));
}
