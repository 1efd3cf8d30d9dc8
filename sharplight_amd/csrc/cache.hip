// KV-cache write: token t's `inner` values go to the cache row the token maps to, converted to the cache's
// element type -- the CacheWrite op without an absorbed producer (src/Sharplight.Cpu/CacheWriteOp.cs:129-175:
// f32 copied, f16 by FloatToHalf, bf16 by FloatToBFloat). Row maps: n_past + t, multi-sequence rows and a
// paged block table (cache_row, common.hpp).
//
// Layout (vector path): grid (token, 512-element chunk), one wave each; a lane converts elements
// [4l, 4l+4) and [256+4l, 256+4l+4) of its chunk, so every load and store instruction covers one
// contiguous span. Lanes past a partial chunk's end redo its last group (identical bytes), keeping every
// memory operation unconditional. The token's row (scalar loads of its sequence row and block table
// entry) is resolved while the data loads are in flight; a row outside the cache is skipped and reported
// through the device error record.
#include "common.hpp"

namespace slhip {

struct CacheWriteArgs {
    const void* x;
    int64_t xs;     // x row stride (elements)
    int64_t T, inner;
    void* cache;
    CacheRowsDev rows;
    uint32_t* err;
};

// 4 consecutive elements of dtype DT (16 bytes for f32, 8 bytes for f16/bf16).
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
__global__ __launch_bounds__(64) void cache_write_vec(CacheWriteArgs a)
{
    const int64_t t = blockIdx.x;
    const int lane = threadIdx.x;
    const int64_t base = static_cast<int64_t>(blockIdx.y) * 512;
    const int64_t e0 = base + 4 * lane < a.inner - 4 ? base + 4 * lane : a.inner - 4;
    const int64_t e1 = base + 256 + 4 * lane < a.inner - 4 ? base + 256 + 4 * lane : a.inner - 4;
    const char* xr = static_cast<const char*>(a.x) + t * a.xs * Vec<DI>::BYTES;
    float f0[4], f1[4];
    load4<DI>(xr + e0 * Vec<DI>::BYTES, f0);
    load4<DI>(xr + e1 * Vec<DI>::BYTES, f1);
    const CacheRow cr = cache_row(a.rows, t);
    if (cr.row >= 0) {  // wave-uniform
        char* yr = static_cast<char*>(a.cache) + cr.row * a.inner * Vec<DO>::BYTES;
        store_packed<DO, 4>(yr + e0 * Vec<DO>::BYTES, f0);
        store_packed<DO, 4>(yr + e1 * Vec<DO>::BYTES, f1);
    } else if (lane == 0 && blockIdx.y == 0) {
        raise_cache_error(a.err, cr, t);
    }
}

// General path (any alignment or inner): one block per token, one element per thread and step.
template <int DI, int DO>
__global__ __launch_bounds__(256) void cache_write_scalar(CacheWriteArgs a)
{
    const int64_t t = blockIdx.x;
    const CacheRow cr = cache_row(a.rows, t);
    if (cr.row < 0) {
        if (threadIdx.x == 0) raise_cache_error(a.err, cr, t);
        return;
    }
    const void* xr = static_cast<const char*>(a.x) + t * a.xs * Vec<DI>::BYTES;
    void* yr = static_cast<char*>(a.cache) + cr.row * a.inner * Vec<DO>::BYTES;
    for (int64_t i = threadIdx.x; i < a.inner; i += 256) Vec<DO>::store1(yr, i, Vec<DI>::load1(xr, i));
}

template <int DI, int DO>
static int run(const CacheWriteArgs& a, hipStream_t st)
{
    constexpr int LA = DI == SLHIP_F32 ? 16 : 8;  // load alignment of 4 elements
    constexpr int SA = DO == SLHIP_F32 ? 16 : 8;  // store alignment
    const bool vec = a.inner % 4 == 0 && a.inner >= 4 && reinterpret_cast<uintptr_t>(a.x) % LA == 0 &&
                     (a.xs * Vec<DI>::BYTES) % LA == 0 && reinterpret_cast<uintptr_t>(a.cache) % SA == 0 &&
                     (a.inner * Vec<DO>::BYTES) % SA == 0;
    if (vec) {
        const int64_t chunks = (a.inner + 511) / 512;
        if (chunks > 65535) return fail(SLHIP_ERR_UNSUPPORTED, "cache_write: rows of %lld values", static_cast<long long>(a.inner));
        cache_write_vec<DI, DO><<<dim3(static_cast<unsigned>(a.T), static_cast<unsigned>(chunks)), 64, 0, st>>>(a);
        return check_launch("cache_write_vec");
    }
    cache_write_scalar<DI, DO><<<dim3(static_cast<unsigned>(a.T)), 256, 0, st>>>(a);
    return check_launch("cache_write_scalar");
}

template <int DI>
static int by_cache(int dc, const CacheWriteArgs& a, hipStream_t st)
{
    switch (dc) {
    case SLHIP_F32: return run<DI, SLHIP_F32>(a, st);
    case SLHIP_F16: return run<DI, SLHIP_F16>(a, st);
    case SLHIP_BF16: return run<DI, SLHIP_BF16>(a, st);
    default: return fail(SLHIP_ERR_UNSUPPORTED, "cache_write: cache dtype %d not supported", dc);
    }
}

}  // namespace slhip

using namespace slhip;

extern "C" SLHIP_API int slhip_cache_write(int dtype_in, int dtype_cache, const void* x, int64_t x_stride, int64_t T,
                                           int64_t inner, void* cache, const slhip_cache_rows* rows, slhip_stream stream)
{
    if (T < 0 || inner < 0) return fail(SLHIP_ERR_INVALID, "cache_write: negative shape");
    if (T == 0 || inner == 0) return SLHIP_OK;
    if (!x || !cache) return fail(SLHIP_ERR_INVALID, "cache_write: x and cache are required");
    if (x_stride < inner) return fail(SLHIP_ERR_INVALID, "cache_write: x row stride is smaller than the row");
    if (T > 0x7FFFFFFF) return fail(SLHIP_ERR_UNSUPPORTED, "cache_write: more than 2^31-1 tokens");
    CacheWriteArgs a{x, x_stride, T, inner, cache, {}, nullptr};
    int e = make_cache_rows(rows, T, &a.rows);
    if (e) return e;
    e = error_word(&a.err);
    if (e) return e;
    hipStream_t st = to_stream(stream);
    if (dtype_in == SLHIP_F32) return by_cache<SLHIP_F32>(dtype_cache, a, st);
    if (dtype_in == SLHIP_BF16) return by_cache<SLHIP_BF16>(dtype_cache, a, st);
    return fail(SLHIP_ERR_UNSUPPORTED, "cache_write: input dtype %d not supported", dtype_in);
}
