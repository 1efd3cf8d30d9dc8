#pragma once
// The per-element pieces of the fused elementwise groups, shared by the op-code interpreter (ewgroup.hip) and
// the kernels generated per group at run time (their source includes this header): four values of an input,
// of an output, a node's rounding, and a node's arithmetic on four values.
#include "common.hpp"
#include "ew_ops.hpp"

namespace slhip {

typedef float f4v __attribute__((ext_vector_type(4)));

// Four values of an input of mode MODE and type DT at row r, columns c .. c + 3 (c + 3 < cols, or the
// clamped last vector).
template <int MODE, int DT>
__device__ __forceinline__ f4v fetch4_t(const void* data, int64_t r, int64_t c, int64_t cols)
{
    f4v v;
    if constexpr (MODE == SLHIP_EWI_COL || MODE == SLHIP_EWI_SCALAR) {
        const int64_t off = MODE == SLHIP_EWI_COL ? r : 0;
        float x;
        if constexpr (DT == SLHIP_F32) x = static_cast<const float*>(data)[off];
        else if constexpr (DT == SLHIP_BF16) x = __uint_as_float(static_cast<uint32_t>(static_cast<const uint16_t*>(data)[off]) << 16);
        else x = static_cast<float>(static_cast<const _Float16*>(data)[off]);
        v[0] = v[1] = v[2] = v[3] = x;
        return v;
    } else {
        const int64_t off = MODE == SLHIP_EWI_ROW ? c : r * cols + c;
        if constexpr (DT == SLHIP_F32) {
            const float4 f = *reinterpret_cast<const float4*>(static_cast<const float*>(data) + off);
            v[0] = f.x; v[1] = f.y; v[2] = f.z; v[3] = f.w;
        } else {
            const uint2 b = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(data) + off);
            if constexpr (DT == SLHIP_BF16) {
                v[0] = bf16_lo(b.x); v[1] = bf16_hi(b.x); v[2] = bf16_lo(b.y); v[3] = bf16_hi(b.y);
            } else {
                v[0] = f16_lo(b.x); v[1] = f16_hi(b.x); v[2] = f16_lo(b.y); v[3] = f16_hi(b.y);
            }
        }
        return v;
    }
}

// Four values stored as DT at element offset off.
template <int DT>
__device__ __forceinline__ void store4_t(void* p, int64_t off, f4v v)
{
    if constexpr (DT == SLHIP_F32) {
        *reinterpret_cast<float4*>(static_cast<float*>(p) + off) = make_float4(v[0], v[1], v[2], v[3]);
    } else if constexpr (DT == SLHIP_BF16) {
        *reinterpret_cast<uint2*>(static_cast<uint16_t*>(p) + off) =
            make_uint2(f32_to_bf16_bits(v[0]) | (f32_to_bf16_bits(v[1]) << 16), f32_to_bf16_bits(v[2]) | (f32_to_bf16_bits(v[3]) << 16));
    } else {
        *reinterpret_cast<uint2*>(static_cast<uint16_t*>(p) + off) = make_uint2(pack_f16x2(v[0], v[1]), pack_f16x2(v[2], v[3]));
    }
}

// A value rounded to a node's output type (the unfused graph stores it in that type).
__device__ __forceinline__ float round_to(int dt, float v)
{
    if (dt == SLHIP_BF16) return __uint_as_float(f32_to_bf16_bits(v) << 16);
    if (dt == SLHIP_F16) return static_cast<float>(static_cast<_Float16>(v));
    return v;
}

__device__ __forceinline__ f4v round4(int dt, f4v v)
{
    f4v r;
#pragma unroll
    for (int e = 0; e < 4; e++) r[e] = round_to(dt, v[e]);
    return r;
}

__device__ __forceinline__ f4v bin4(int op, f4v x, f4v y, bool pow_special)
{
    f4v r;
#pragma unroll
    for (int e = 0; e < 4; e++) r[e] = binary_op(op, x[e], y[e], pow_special);
    return r;
}

__device__ __forceinline__ f4v un4(int op, f4v x, float p0, float p1)
{
    f4v r;
#pragma unroll
    for (int e = 0; e < 4; e++) r[e] = unary_op(op, x[e], p0, p1);
    return r;
}

// Sum of squares of four values, in the order the row norms of the groups use.
__device__ __forceinline__ float sumsq4(f4v v) { return fmaf(v[0], v[0], v[1] * v[1]) + fmaf(v[2], v[2], v[3] * v[3]); }

// The arguments of a generated group kernel (the program's pointers; its shape and ops are compiled in).
struct EwgJitArgs {
    const void* in[SLHIP_EW_MAX_INPUTS];
    void* out[SLHIP_EW_MAX_OUTPUTS];
    const float* w;  // the norm's weight, or null
    void* y;         // the tail's output
    int64_t rows;
};

}  // namespace slhip
