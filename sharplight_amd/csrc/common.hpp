// Shared device helpers and host plumbing of libsharplight_hip (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/sharplight_hip.h"

namespace slhip {

// ---- host side: error reporting -------------------------------------------------------------------

// Records a formatted message as this thread's last error and returns `status`.
int fail(int status, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
// Maps a HIP error to SLHIP_ERR_HIP with the call site; SLHIP_OK for hipSuccess.
int hip_fail(hipError_t e, const char* what);
// Checks the launch that was just enqueued.
int check_launch(const char* kernel);

#define SLHIP_CHECK_HIP(call)                                                                                          \
    do {                                                                                                               \
        hipError_t e_ = (call);                                                                                        \
        if (e_ != hipSuccess) return ::slhip::hip_fail(e_, #call);                                                     \
    } while (0)

// The current device's error record, eight 32-bit words that kernels raise (raise_error) and
// slhip_stream_sync reports: [0] code (0 = none), [1..6] the code's values. A device variable of the
// library: nothing is allocated for it.
int error_word(uint32_t** word);

// Whether slhip_matvec / slhip_dual_matvec can stage rows of K values of `fmt` (matvec.hip).
bool matvec_fits(int fmt, int64_t K, bool dual);

// KV-cache destination rows (slhip_cache_rows) as kernels take them.
struct CacheRowsDev {
    int mode;
    int64_t ctx, n_past;
    const int32_t* seq;
    int64_t slots, slot_ctx;
    const int32_t* pages;
    int64_t page_slots, bps, bs;
};
// Validates `in` for a launch of T tokens (PAST overflow is refused here, as CacheWriteOp.Run throws for
// it, src/Sharplight.Cpu/CacheWriteOp.cs:118-121) and fills `out`.
int make_cache_rows(const slhip_cache_rows* in, int64_t T, CacheRowsDev* out);

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

inline hipStream_t to_stream(slhip_stream s) { return reinterpret_cast<hipStream_t>(s); }

// ---- device side: streaming 16-byte accesses --------------------------------------------------------

// Every activation byte of these ops is touched exactly once, so inputs are loaded and outputs stored
// with the nontemporal cache policy: the lines do not displace reusable data (weights, norm gammas) and
// a plain copy measures ~8% faster on MI355X this way than with default-policy accesses.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint4 load_nt(const void* p)
{
    u32x4 v = __builtin_nontemporal_load(static_cast<const u32x4*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ void store_nt(void* p, const uint4& v)
{
    u32x4 t = {v.x, v.y, v.z, v.w};
    __builtin_nontemporal_store(t, static_cast<u32x4*>(p));
}

__device__ __forceinline__ void store_nt(void* p, const uint2& v)
{
    u32x2 t = {v.x, v.y};
    __builtin_nontemporal_store(t, static_cast<u32x2*>(p));
}

__device__ __forceinline__ void store_nt(void* p, uint32_t v) { __builtin_nontemporal_store(v, static_cast<uint32_t*>(p)); }

// ---- device side: conversions ----------------------------------------------------------------------

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }

// f32 -> bf16 with the reference's rounding (Simd.FloatToBFloat, src/Sharplight.Cpu/Simd.cs:530-540):
// round to nearest even (adding 0x7FFF + lsb); a NaN keeps its top half with the quiet bit set; f32
// subnormals round like normals. gfx950's v_cvt_pk_bf16_f32 gives exactly these bits for every f32 input
// (checked on all 2^16 top halves with tie, near-tie and NaN-payload low halves, and by the bit-exact
// conversion tests), at one instruction per pair instead of about five per value.
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f)
{
    return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi)
{
    const f32x2_t v = {lo, hi};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

__device__ __forceinline__ float f16_lo(uint32_t w)
{
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w & 0xFFFFu)));
}
__device__ __forceinline__ float f16_hi(uint32_t w)
{
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w >> 16)));
}
__device__ __forceinline__ uint32_t pack_f16x2(float lo, float hi)
{
    uint32_t a = __builtin_bit_cast(uint16_t, static_cast<_Float16>(lo));
    uint32_t b = __builtin_bit_cast(uint16_t, static_cast<_Float16>(hi));
    return a | (b << 16);
}

// ---- device side: element-type traits for 16-byte vectors -----------------------------------------

// A 16-byte vector of an activation dtype, unpacked to / packed from f32 lanes.
template <int DT> struct Vec;

template <> struct Vec<SLHIP_F32> {
    static constexpr int N = 4;  // elements per 16 bytes
    static constexpr int BYTES = 4;
    __device__ static __forceinline__ void unpack(const uint4& v, float* f)
    {
        f[0] = __uint_as_float(v.x);
        f[1] = __uint_as_float(v.y);
        f[2] = __uint_as_float(v.z);
        f[3] = __uint_as_float(v.w);
    }
    // Packs N floats into N*BYTES bytes (16).
    __device__ static __forceinline__ uint4 pack(const float* f)
    {
        return make_uint4(__float_as_uint(f[0]), __float_as_uint(f[1]), __float_as_uint(f[2]), __float_as_uint(f[3]));
    }
    __device__ static __forceinline__ float load1(const void* p, int64_t i) { return static_cast<const float*>(p)[i]; }
    __device__ static __forceinline__ void store1(void* p, int64_t i, float v) { static_cast<float*>(p)[i] = v; }
};

template <> struct Vec<SLHIP_BF16> {
    static constexpr int N = 8;
    static constexpr int BYTES = 2;
    __device__ static __forceinline__ void unpack(const uint4& v, float* f)
    {
        f[0] = bf16_lo(v.x); f[1] = bf16_hi(v.x);
        f[2] = bf16_lo(v.y); f[3] = bf16_hi(v.y);
        f[4] = bf16_lo(v.z); f[5] = bf16_hi(v.z);
        f[6] = bf16_lo(v.w); f[7] = bf16_hi(v.w);
    }
    __device__ static __forceinline__ uint4 pack(const float* f)
    {
        return make_uint4(pack_bf16x2(f[0], f[1]), pack_bf16x2(f[2], f[3]), pack_bf16x2(f[4], f[5]),
                          pack_bf16x2(f[6], f[7]));
    }
    __device__ static __forceinline__ float load1(const void* p, int64_t i)
    {
        return __uint_as_float(static_cast<uint32_t>(static_cast<const uint16_t*>(p)[i]) << 16);
    }
    __device__ static __forceinline__ void store1(void* p, int64_t i, float v)
    {
        static_cast<uint16_t*>(p)[i] = static_cast<uint16_t>(f32_to_bf16_bits(v));
    }
};

template <> struct Vec<SLHIP_F16> {
    static constexpr int N = 8;
    static constexpr int BYTES = 2;
    __device__ static __forceinline__ void unpack(const uint4& v, float* f)
    {
        f[0] = f16_lo(v.x); f[1] = f16_hi(v.x);
        f[2] = f16_lo(v.y); f[3] = f16_hi(v.y);
        f[4] = f16_lo(v.z); f[5] = f16_hi(v.z);
        f[6] = f16_lo(v.w); f[7] = f16_hi(v.w);
    }
    __device__ static __forceinline__ uint4 pack(const float* f)
    {
        return make_uint4(pack_f16x2(f[0], f[1]), pack_f16x2(f[2], f[3]), pack_f16x2(f[4], f[5]),
                          pack_f16x2(f[6], f[7]));
    }
    __device__ static __forceinline__ float load1(const void* p, int64_t i)
    {
        return static_cast<float>(static_cast<const _Float16*>(p)[i]);
    }
    __device__ static __forceinline__ void store1(void* p, int64_t i, float v)
    {
        static_cast<_Float16*>(p)[i] = static_cast<_Float16>(v);
    }
};

// Stores M f32 values as dtype DT at byte address p (M*BYTES bytes, which is 16 or a multiple of 8), with
// the streaming (nontemporal) policy.
template <int DT, int M> __device__ __forceinline__ void store_packed(void* p, const float* f);

template <> __device__ __forceinline__ void store_packed<SLHIP_F32, 4>(void* p, const float* f)
{
    store_nt(p, Vec<SLHIP_F32>::pack(f));
}
template <> __device__ __forceinline__ void store_packed<SLHIP_F32, 8>(void* p, const float* f)
{
    store_nt(p, Vec<SLHIP_F32>::pack(f));
    store_nt(static_cast<char*>(p) + 16, Vec<SLHIP_F32>::pack(f + 4));
}
template <> __device__ __forceinline__ void store_packed<SLHIP_BF16, 8>(void* p, const float* f)
{
    store_nt(p, Vec<SLHIP_BF16>::pack(f));
}
template <> __device__ __forceinline__ void store_packed<SLHIP_BF16, 4>(void* p, const float* f)
{
    store_nt(p, make_uint2(pack_bf16x2(f[0], f[1]), pack_bf16x2(f[2], f[3])));
}
template <> __device__ __forceinline__ void store_packed<SLHIP_F16, 8>(void* p, const float* f)
{
    store_nt(p, Vec<SLHIP_F16>::pack(f));
}
template <> __device__ __forceinline__ void store_packed<SLHIP_F16, 4>(void* p, const float* f)
{
    store_nt(p, make_uint2(pack_f16x2(f[0], f[1]), pack_f16x2(f[2], f[3])));
}

// ---- device side: wavefront reductions ------------------------------------------------------------

template <int CTRL> __device__ __forceinline__ float dpp_f32(float v)
{
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, false));
}

// Sum over groups of W consecutive lanes (W a power of two <= 64); every lane of the group ends with the
// same value (the same pairs, quads, ... summed in the same order for every lane). Within a 16-lane row the
// steps are DPP moves (quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror, row_mirror: once the
// lanes of a quad (of 8 lanes) agree, the mirror pairs each with the other quad (half)), with no LDS round
// trip; across rows a lane exchange.
template <int W> __device__ __forceinline__ float group_sum(float v)
{
    static_assert(W >= 1 && W <= 64 && (W & (W - 1)) == 0, "group of 1..64 lanes");
    if constexpr (W >= 2) v += dpp_f32<0xB1>(v);
    if constexpr (W >= 4) v += dpp_f32<0x4E>(v);
    if constexpr (W >= 8) v += dpp_f32<0x141>(v);
    if constexpr (W >= 16) v += dpp_f32<0x140>(v);
    if constexpr (W >= 32) v += __shfl_xor(v, 16, 64);
    if constexpr (W >= 64) v += __shfl_xor(v, 32, 64);
    return v;
}

// The hardware reciprocal with one Newton step: r = fma(fma(-s, y, 1), y, y), y = rcp(s).
__device__ __forceinline__ float recip_nr(float s)
{
    const float y = __builtin_amdgcn_rcpf(s);
    return fmaf(fmaf(-s, y, 1.0f), y, y);
}

// 1/s rounded as IEEE division: recip_nr where it equals the quotient -- s in [2^-125, 2^125], checked for
// every f32 there on the device by tests/recip_exhaustive.hip -- and the division elsewhere.
__device__ __forceinline__ float recip_ieee(float s)
{
    const float r = recip_nr(s);
    return (s >= 0x1p-125f && s <= 0x1p125f) ? r : 1.0f / s;
}

// Sum over the whole wave, returned wave-uniform: the row sums by DPP as above, then row_bcast:15 and
// row_bcast:31 carry rows 0..2 into row 3, whose last lane holds the total ((r0 + r1) + (r2 + r3)).
__device__ __forceinline__ float wave_sum(float v)
{
    v += dpp_f32<0xB1>(v);
    v += dpp_f32<0x4E>(v);
    v += dpp_f32<0x141>(v);
    v += dpp_f32<0x140>(v);
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x142, 0xA, 0xF, false));  // row_bcast:15
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x143, 0xC, 0xF, false));  // row_bcast:31
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Max over groups of W consecutive lanes; every lane of the group ends with the same value.
template <int W> __device__ __forceinline__ float group_max(float v)
{
#pragma unroll
    for (int o = W / 2; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

// Max over groups of W (2..32) consecutive lanes with DPP lane moves (no LDS round trip): swaps within
// quads, then the mirror of each 8 and of each 16 lanes -- each step combines two disjoint halves, so
// every lane ends with the group's max -- and one exchange across 16 lanes for W = 32.
template <int CTRL> __device__ __forceinline__ float dpp_max_step(float v)
{
    return fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, false)));
}

template <int W> __device__ __forceinline__ float group_max_dpp(float v)
{
    static_assert(W >= 2 && W <= 32 && (W & (W - 1)) == 0, "group of 2..32 lanes");
    v = dpp_max_step<0xB1>(v);                       // quad_perm [1,0,3,2]
    if constexpr (W >= 4) v = dpp_max_step<0x4E>(v);  // quad_perm [2,3,0,1]
    if constexpr (W >= 8) v = dpp_max_step<0x141>(v);  // row_half_mirror
    if constexpr (W >= 16) v = dpp_max_step<0x140>(v);  // row_mirror
    if constexpr (W >= 32) v = fmaxf(v, __shfl_xor(v, 16, 64));
    return v;
}

// Max over groups of W (2..32) consecutive lanes of non-negative, non-NaN floats, with DPP lane moves
// (no LDS round trip): swaps within quads, then the mirror of each 8 and of each 16 lanes -- each step
// combines two disjoint halves, so every lane ends with the group's max -- and one exchange across 16
// lanes for W = 32. For such values the order of the bit patterns as unsigned integers is the order of
// the values, so the steps are integer maxima (a float max would first quiet possible signalling NaNs).
template <int CTRL> __device__ __forceinline__ uint32_t dpp_umax_step(uint32_t v)
{
    return max(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), CTRL, 0xF, 0xF, false)));
}

template <int W> __device__ __forceinline__ float group_max_nonneg(float x)
{
    static_assert(W >= 2 && W <= 32 && (W & (W - 1)) == 0, "group of 2..32 lanes");
    uint32_t v = __float_as_uint(x);
    v = dpp_umax_step<0xB1>(v);                       // quad_perm [1,0,3,2]
    if constexpr (W >= 4) v = dpp_umax_step<0x4E>(v);  // quad_perm [2,3,0,1]
    if constexpr (W >= 8) v = dpp_umax_step<0x141>(v);  // row_half_mirror
    if constexpr (W >= 16) v = dpp_umax_step<0x140>(v);  // row_mirror
    if constexpr (W >= 32) v = max(v, static_cast<uint32_t>(__shfl_xor(static_cast<int>(v), 16, 64)));
    return __uint_as_float(v);
}

// ---- device side: E4M3 activation rows -------------------------------------------------------------

// E4M3 codes with the reference's rule (e4m3_code, src/Sharplight.Shaders/Kernels/e4m3.slang:5-23): round
// to nearest even on the E4M3 grid (multiples of 2^-9 below 2^-6), saturate at code 0x7E (448), and set
// the sign bit only for v < 0 -- so -0 gives code 0x00, NaN 0x7E and +-inf 0x7E / 0xFE. gfx950's
// v_cvt_pk_fp8_f32 (OCP E4M3, round to nearest even) returns these codes for every finite |v| <= 448
// except -0. So the value is formed as fma(v, id, +0) -- v * id rounded once, with -0 turned into +0 --
// and clamped to [-448, 448] (fminf first: it returns 448 for NaN). Over all 2^32 f32 inputs this equals
// the integer rule bit for bit (tests/e4m3_exhaustive.hip).
__device__ __forceinline__ float e4m3_operand(float v, float id)
{
    return fmaxf(fminf(fmaf(v, id, 0.0f), 448.0f), -448.0f);
}

// The 4 codes of v[0..3] * id, packed little-endian (e4m3_pack4, e4m3.slang:33-38).
__device__ __forceinline__ uint32_t e4m3_pack4(const float* v, float id)
{
    int r = __builtin_amdgcn_cvt_pk_fp8_f32(e4m3_operand(v[0], id), e4m3_operand(v[1], id), 0, false);
    r = __builtin_amdgcn_cvt_pk_fp8_f32(e4m3_operand(v[2], id), e4m3_operand(v[3], id), r, true);
    return static_cast<uint32_t>(r);
}

__device__ __forceinline__ uint32_t e4m3_code(float v)
{
    return static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(e4m3_operand(v, 1.0f), 0.0f, 0, false)) & 0xFFu;
}

// The group scale of quantize_fp8 from the group's amax m (>= 0, not NaN): d = m / 448 and
// id = d > 0 ? 1 / d : 0 (e4m3_group_scale / e4m3_pack4, e4m3.slang:25-38), both correctly rounded. For
// m = 0 and m in [2^-116, FLT_MAX] -- every amax of real activations -- a product with the rounded
// reciprocal of 448 corrected by one fma gives d exactly, and the hardware reciprocal of d corrected by
// one Newton step gives 1/d exactly (the division's results are normal there); elsewhere the lanes take
// IEEE division. Checked against IEEE division for every non-negative f32 m (tests/e4m3_exhaustive.hip).
__device__ __forceinline__ void e4m3_group_scale(float m, float& d, float& id)
{
    constexpr float kInv448 = 1.0f / 448.0f;
    const float q = m * kInv448;
    d = fmaf(fmaf(-q, 448.0f, m), kInv448, q);
    const float y = __builtin_amdgcn_rcpf(d);
    const float r = fmaf(fmaf(-d, y, 1.0f), y, y);
    id = d > 0.0f ? r : 0.0f;
    const uint32_t u = __float_as_uint(m);  // [2^-116, FLT_MAX] as bit patterns: [0x05800000, 0x7F7FFFFF]
    if (u - 0x05800000u > 0x7F7FFFFFu - 0x05800000u && u != 0) {
        d = m / 448.0f;
        id = d > 0.0f ? 1.0f / d : 0.0f;
    }
}

// ---- device side: errors raised by kernels -----------------------------------------------------------

enum : uint32_t { kErrGatherIndex = 1, kErrCacheSeq = 2, kErrCachePageTable = 3, kErrCacheBlock = 4 };

// Records an error in the device's error record unless one is already there (the first error wins).
__device__ __forceinline__ void raise_error(uint32_t* err, uint32_t code, uint32_t a, uint32_t b, uint32_t c,
                                            uint32_t d, uint32_t e, uint32_t f)
{
    if (atomicCAS(err, 0u, code) == 0u) {
        err[1] = a;
        err[2] = b;
        err[3] = c;
        err[4] = d;
        err[5] = e;
        err[6] = f;
    }
}

// The cache row of token t (CacheWriteOp.Body, src/Sharplight.Cpu/CacheWriteOp.cs:129-155; KvPages.Row,
// KvPages.cs:28-32), or row -1 with the error the reference would throw (CacheWriteOp.cs:103-117,
// KvPages.Check, KvPages.cs:38-49) in code/values. Wave-uniform t: the sequence row and block table
// entry are scalar loads.
struct CacheRow {
    int64_t row;
    uint32_t code;
    int32_t slot, pos;
    int64_t v1, v2;
};

__device__ __forceinline__ CacheRow cache_row(const CacheRowsDev& r, int64_t t)
{
    CacheRow o{-1, 0, 0, 0, 0, 0};
    if (r.mode == SLHIP_ROWS_PAST) {
        o.row = r.n_past + t;  // checked against ctx on the host
        return o;
    }
    const int32_t slot = r.seq[t * 4], pos = r.seq[t * 4 + 1];
    o.slot = slot;
    o.pos = pos;
    if (r.mode == SLHIP_ROWS_SEQ) {
        if (static_cast<uint64_t>(static_cast<int64_t>(slot)) >= static_cast<uint64_t>(r.slots) ||
            static_cast<uint64_t>(static_cast<int64_t>(pos)) >= static_cast<uint64_t>(r.slot_ctx)) {
            o.code = kErrCacheSeq;
            o.v1 = r.slot_ctx;
            return o;
        }
        o.row = slot * r.slot_ctx + pos;
        return o;
    }
    if (static_cast<uint64_t>(static_cast<int64_t>(slot)) >= static_cast<uint64_t>(r.page_slots) || pos < 0 ||
        pos >= r.bps * r.bs) {
        o.code = kErrCachePageTable;
        o.v1 = r.page_slots;
        o.v2 = r.bps;
        return o;
    }
    const int64_t block = r.pages[static_cast<int64_t>(slot) * r.bps + pos / r.bs];
    if (block < 0 || (block + 1) * r.bs > r.ctx) {
        o.code = kErrCacheBlock;
        o.v1 = block;
        o.v2 = r.ctx;
        return o;
    }
    o.row = block * r.bs + pos % r.bs;
    return o;
}

__device__ __forceinline__ void raise_cache_error(uint32_t* err, const CacheRow& c, int64_t t)
{
    raise_error(err, c.code, static_cast<uint32_t>(t), static_cast<uint32_t>(c.slot), static_cast<uint32_t>(c.pos),
                static_cast<uint32_t>(static_cast<uint64_t>(c.v1)), static_cast<uint32_t>(static_cast<uint64_t>(c.v1) >> 32),
                static_cast<uint32_t>(c.v2));
}

// Makes this wave's LDS writes visible to its own later LDS reads, for kernels whose waves work on
// independent items and never wait for each other.
__device__ __forceinline__ void wave_lds_sync()
{
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// The index of the calling thread's wave in its block, as a wave-uniform (scalar) value.
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

}  // namespace slhip
