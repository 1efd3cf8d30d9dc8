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

// Device word that gather kernels raise on an out-of-range id: [0] flag, [1] the id (low 32 bits),
// [2] the id (high 32 bits). One per device, allocated on first use.
int index_error_word(uint32_t** word);

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

// Butterfly sum over groups of W consecutive lanes (W a power of two <= 64); every lane of the group
// ends with the same value, summed in the same order.
template <int W> __device__ __forceinline__ float group_sum(float v)
{
#pragma unroll
    for (int o = W / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

__device__ __forceinline__ float wave_sum(float v) { return group_sum<64>(v); }

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
