#pragma once
// Pieces shared by the matvec kernels (matvec.hip) and the several-token block-format kernel on the bf16
// matrix cores (matvec_mq.hpp): the launch arguments, x split into bf16 parts, the per-format stage geometry
// and the block formats' codes as exact bf16 operands.
#include "act.hpp"
#include "common.hpp"
#include "quant.hpp"

#include <type_traits>

namespace slhip {

struct MatvecArgs {
    const void* x;  // [T, K] activations, row stride xs elements
    int64_t xs;
    const char* wg;  // N rows of wrow bytes
    const char* wu;  // the second matrix of a dual matvec, else null
    int64_t wrow;
    void* y;  // [T, N], row stride ys elements
    int64_t ys;
    int64_t T, K, N;
    int64_t t0;  // first activation row of this launch
    int xt, yt;  // SLHIP_F32 / SLHIP_BF16
    int act;     // dual: SLHIP_ACT_*
    const float* bias;  // single matvec: [N] f32 added to each output row (FoldMatMulBiases), or null
};

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ bf16x8_t as_bf16x8(const uint4& v) { return __builtin_bit_cast(bf16x8_t, v); }

// split3 for finite x: the same parts without the guard.
__device__ __forceinline__ void split3_finite(const float* x, uint4& h, uint4& m, uint4& l)
{
    uint32_t hw[4], mw[4], lw[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float a0 = x[2 * i], a1 = x[2 * i + 1];
        hw[i] = pack_bf16x2(a0, a1);
        const float r0 = a0 - bf16_lo(hw[i]), r1 = a1 - bf16_hi(hw[i]);
        mw[i] = pack_bf16x2(r0, r1);
        lw[i] = pack_bf16x2(r0 - bf16_lo(mw[i]), r1 - bf16_hi(mw[i]));
    }
    h = make_uint4(hw[0], hw[1], hw[2], hw[3]);
    m = make_uint4(mw[0], mw[1], mw[2], mw[3]);
    l = make_uint4(lw[0], lw[1], lw[2], lw[3]);
}

// x[0..7] (f32) as three bf16 vectors with h + m + l == x; a non-finite x keeps only h (inf - inf would
// otherwise make the remainders NaN).
__device__ __forceinline__ void split3(const float* x, uint4& h, uint4& m, uint4& l)
{
    uint32_t hw[4], mw[4], lw[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float a0 = x[2 * i], a1 = x[2 * i + 1];
        hw[i] = pack_bf16x2(a0, a1);
        float r0 = a0 - bf16_lo(hw[i]), r1 = a1 - bf16_hi(hw[i]);
        r0 = r0 == r0 ? r0 : 0.0f;
        r1 = r1 == r1 ? r1 : 0.0f;
        mw[i] = pack_bf16x2(r0, r1);
        lw[i] = pack_bf16x2(r0 - bf16_lo(mw[i]), r1 - bf16_hi(mw[i]));
    }
    h = make_uint4(hw[0], hw[1], hw[2], hw[3]);
    m = make_uint4(mw[0], mw[1], mw[2], mw[3]);
    l = make_uint4(lw[0], lw[1], lw[2], lw[3]);
}

template <int FMT> struct MqGeom;
constexpr int kMqWaves = 8;
// SKB: 32-value blocks per stage, RB: bytes of one row per stage, UB: bytes per staging load
template <> struct MqGeom<SLHIP_FMT_Q4_0> { static constexpr int SKB = 32, RB = 32 * 18, UB = 16; };
template <> struct MqGeom<SLHIP_FMT_Q8_0> { static constexpr int SKB = 16, RB = 16 * 34, UB = 16; };
template <> struct MqGeom<SLHIP_FMT_Q4_1> { static constexpr int SKB = 32, RB = 32 * 20, UB = 16; };
template <> struct MqGeom<SLHIP_FMT_Q5_0> { static constexpr int SKB = 32, RB = 32 * 22, UB = 16; };
template <> struct MqGeom<SLHIP_FMT_Q5_1> { static constexpr int SKB = 32, RB = 32 * 24, UB = 16; };
template <> struct MqGeom<SLHIP_FMT_Q4_K> { static constexpr int SKB = 32, RB = 4 * 144, UB = 16; };  // 4 super-blocks
template <> struct MqGeom<SLHIP_FMT_Q5_K> { static constexpr int SKB = 32, RB = 4 * 176, UB = 16; };
template <> struct MqGeom<SLHIP_FMT_Q6_K> { static constexpr int SKB = 16, RB = 2 * 210, UB = 4; };   // 420 bytes
template <> struct MqGeom<SLHIP_FMT_Q2_K> { static constexpr int SKB = 32, RB = 4 * 84, UB = 16; };   // 336 bytes
template <> struct MqGeom<SLHIP_FMT_Q3_K> { static constexpr int SKB = 32, RB = 4 * 110, UB = 8; };   // 440 bytes

// Eight codes of lane group g (values 8g .. 8g + 7 of the block) as four bf16 pairs, the format's offset
// applied (Q4_0 q - 8, Q5_0 q - 16: exact); row: the row's stage bytes (4-byte aligned), off: the block's
// first byte in it. Layouts of Quant.cs:242-405: {f16 d, [f16 m], [u32 qh], qs}, value v the low (v < 16) or
// high nibble of qs[v % 16], plus 16 when bit v of qh is set (Q5_0, Q5_1); Q8_0 int8 codes.
template <int FMT>
__device__ __forceinline__ uint4 mq_codes(const uint8_t* row, int off, int g)
{
    using F = Fmt<FMT>;
    constexpr bool NIB = FMT != SLHIP_FMT_Q8_0;
    // the eight code bytes at off + QS + (nibble formats: 8 (g & 1); Q8_0: 8 g), 2-byte aligned: three
    // aligned words and a funnel shift (the row pointer is used as it is, so the reads stay LDS reads)
    const int q = off + F::QS + (NIB ? 8 * (g & 1) : 8 * g);
    auto words = [&](int p, uint32_t& a, uint32_t& b) {
        const uint32_t* w = reinterpret_cast<const uint32_t*>(row) + (p >> 2);
        const uint32_t sh = static_cast<uint32_t>(p & 3) * 8;
        const uint32_t w0 = w[0], w1 = w[1], w2 = w[2];
        a = __builtin_amdgcn_alignbit(w1, w0, sh);
        b = __builtin_amdgcn_alignbit(w2, w1, sh);
    };
    uint32_t lo, hi;
    words(q, lo, hi);
    float f[8];
    if constexpr (NIB) {  // low nibbles (g < 2: values 0-15) or high (values 16-31)
        const uint32_t s = 4 * static_cast<uint32_t>(g >> 1);
        lo = (lo >> s) & 0x0F0F0F0Fu;
        hi = (hi >> s) & 0x0F0F0F0Fu;
        if constexpr (F::QH >= 0) {  // bits 8g .. 8g + 7 of qh, one per value, to bit 4 of its byte
            uint32_t qh, unused;
            words(off + F::QH, qh, unused);
            const uint32_t hb = (qh >> (8 * g)) & 0xFFu;
            // spread the 8 bits to bit 4 of 8 bytes: bit e -> byte e
            const uint32_t b0 = hb & 0x0Fu, b1 = hb >> 4;
            auto spread = [](uint32_t n) {  // 4 bits -> bit 4 of 4 bytes
                return ((n & 1u) << 4) | ((n & 2u) << 11) | ((n & 4u) << 18) | ((n & 8u) << 25);
            };
            lo |= spread(b0);
            hi |= spread(b1);
        }
#pragma unroll
        for (int e = 0; e < 4; e++) {
            f[e] = static_cast<float>((lo >> (8 * e)) & 0xFFu) + static_cast<float>(F::OFF);
            f[4 + e] = static_cast<float>((hi >> (8 * e)) & 0xFFu) + static_cast<float>(F::OFF);
        }
    } else {  // int8 codes: q + 128 as an unsigned byte, then exact f32 arithmetic
        lo ^= 0x80808080u;
        hi ^= 0x80808080u;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            f[e] = static_cast<float>((lo >> (8 * e)) & 0xFFu) - 128.0f;
            f[4 + e] = static_cast<float>((hi >> (8 * e)) & 0xFFu) - 128.0f;
        }
    }
    return make_uint4(pack_bf16x2(f[0], f[1]), pack_bf16x2(f[2], f[3]), pack_bf16x2(f[4], f[5]), pack_bf16x2(f[6], f[7]));
}

// Eight Q4_K codes of lane group g (values 8g .. 8g + 7 of sub-block j: the low (j even) or high nibbles of
// bytes 32 (j / 2) + 8g .. of the super-block's 128 code bytes, Quant.cs:518-545) as four bf16 pairs; sbo: the
// super-block's first byte in the staged row (a multiple of 16), so the eight bytes are one aligned 8-byte read.
// Q5_K (FIVE): the codes after a 32-byte qh at byte 16, and value l of sub-block j adds 16 when bit j of qh[l]
// is set (ggml's Q5_K layout, the same scale packing as Q4_K).
template <bool FIVE = false>
__device__ __forceinline__ uint4 q4k_codes(const uint8_t* row, int sbo, int j, int g)
{
    const uint2 w = *reinterpret_cast<const uint2*>(row + sbo + (FIVE ? 48 : 16) + 32 * (j >> 1) + 8 * g);
    const uint32_t sh = 4 * static_cast<uint32_t>(j & 1);
    uint32_t lo = (w.x >> sh) & 0x0F0F0F0Fu, hi = (w.y >> sh) & 0x0F0F0F0Fu;
    if constexpr (FIVE) {
        const uint2 h = *reinterpret_cast<const uint2*>(row + sbo + 16 + 8 * g);
        lo |= ((h.x >> j) & 0x01010101u) << 4;
        hi |= ((h.y >> j) & 0x01010101u) << 4;
    }
    float f[8];
#pragma unroll
    for (int e = 0; e < 4; e++) {
        f[e] = static_cast<float>((lo >> (8 * e)) & 0xFFu);
        f[4 + e] = static_cast<float>((hi >> (8 * e)) & 0xFFu);
    }
    return make_uint4(pack_bf16x2(f[0], f[1]), pack_bf16x2(f[2], f[3]), pack_bf16x2(f[4], f[5]), pack_bf16x2(f[6], f[7]));
}

// Eight bytes at LDS byte q of a 4-byte aligned row, q 2-byte aligned: three aligned words and a funnel shift.
__device__ __forceinline__ uint2 lds_bytes8(const uint8_t* row, int q)
{
    const uint32_t* w = reinterpret_cast<const uint32_t*>(row) + (q >> 2);
    const uint32_t sh = static_cast<uint32_t>(q & 3) * 8;
    const uint32_t w0 = w[0], w1 = w[1], w2 = w[2];
    return make_uint2(__builtin_amdgcn_alignbit(w1, w0, sh), __builtin_amdgcn_alignbit(w2, w1, sh));
}

// Eight Q2_K / Q3_K codes of lane group g for the 32-value block u = 4n + j of a super-block, as four bf16
// pairs (Quant.KQuants.cs:36-107, ggml's layouts): value 128n + 32j + 8g + e has the 2-bit field 2j of byte
// 32n + 8g + e of qs (Q2_K: qs at 16; Q3_K: qs at 32, plus 4 when bit 4n + j of hmask byte 8g + e is set,
// minus 4). Lane groups 0-1 hold the block's first 16-value scale group, 2-3 the second.
template <bool Q3>
__device__ __forceinline__ uint4 q23k_codes(const uint8_t* row, int sbo, int u, int g)
{
    const int n = u >> 2, j = u & 3;
    const uint2 l = lds_bytes8(row, sbo + (Q3 ? 32 : 16) + 32 * n + 8 * g);
    const uint32_t sh = 2 * static_cast<uint32_t>(j);
    uint32_t q0 = (l.x >> sh) & 0x03030303u, q1 = (l.y >> sh) & 0x03030303u;
    if constexpr (Q3) {
        const uint2 h = lds_bytes8(row, sbo + 8 * g);
        const uint32_t hs = static_cast<uint32_t>(4 * n + j);
        q0 |= ((h.x >> hs) & 0x01010101u) << 2;
        q1 |= ((h.y >> hs) & 0x01010101u) << 2;
    }
    constexpr float OFF = Q3 ? -4.0f : 0.0f;
    float f[8];
#pragma unroll
    for (int e = 0; e < 4; e++) {
        f[e] = static_cast<float>((q0 >> (8 * e)) & 0xFFu) + OFF;
        f[4 + e] = static_cast<float>((q1 >> (8 * e)) & 0xFFu) + OFF;
    }
    return make_uint4(pack_bf16x2(f[0], f[1]), pack_bf16x2(f[2], f[3]), pack_bf16x2(f[4], f[5]), pack_bf16x2(f[6], f[7]));
}

// The same eight Q2_K / Q3_K codes multiplied by the integer scale of their 16-value group (lane groups 0-1: the
// block's first group, 2-3 its second), with the super-block's d: d * (code * scale) is the weight, and
// code * scale is an exact bf16 integer (Q3_K |(q - 4) * (s - 32)| <= 128, Q2_K q * s <= 45), so that both
// groups of a block take one MFMA chain (Quant.KQuants.cs:36-107: Q3_K scales are 6-bit fields, 4 low bits at
// byte 96 + (i % 8), 2 high bits at byte 104 + i % 4, minus 32; Q2_K's are the low nibbles of bytes 0..15).
template <bool Q3>
__device__ __forceinline__ uint4 q23k_codes_scaled(const uint8_t* row, int sbo, int u, int g, float& d)
{
    auto u16 = [&](int o) { return static_cast<uint32_t>(*reinterpret_cast<const uint16_t*>(row + o)); };
    float sc;
    if constexpr (Q3) {
        d = static_cast<float>(*reinterpret_cast<const _Float16*>(row + sbo + 108));
        const int s0 = 2 * u, w = s0 >> 2, b0 = s0 & 3;
        const uint32_t a = u16(sbo + 96 + 4 * (w & 1) + b0);
        const uint32_t h = u16(sbo + 104 + b0);
        const uint32_t lo = w < 2 ? (a & 0x0F0Fu) : ((a >> 4) & 0x0F0Fu);
        const uint32_t s2 = lo | (((h >> (2 * w)) & 0x0303u) << 4);
        sc = static_cast<float>(static_cast<int>(g < 2 ? (s2 & 0xFFu) : (s2 >> 8)) - 32);
    } else {
        d = static_cast<float>(*reinterpret_cast<const _Float16*>(row + sbo + 80));
        const uint32_t v = u16(sbo + 2 * u);
        sc = static_cast<float>(g < 2 ? (v & 0xFu) : ((v >> 8) & 0xFu));
    }
    const int n = u >> 2, j = u & 3;
    const uint2 l = lds_bytes8(row, sbo + (Q3 ? 32 : 16) + 32 * n + 8 * g);
    const uint32_t sh = 2 * static_cast<uint32_t>(j);
    uint32_t q0 = (l.x >> sh) & 0x03030303u, q1 = (l.y >> sh) & 0x03030303u;
    if constexpr (Q3) {
        const uint2 hm = lds_bytes8(row, sbo + 8 * g);
        const uint32_t hs = static_cast<uint32_t>(4 * n + j);
        q0 |= ((hm.x >> hs) & 0x01010101u) << 2;
        q1 |= ((hm.y >> hs) & 0x01010101u) << 2;
    }
    constexpr float OFF = Q3 ? -4.0f : 0.0f;
    float f[8];
#pragma unroll
    for (int e = 0; e < 4; e++) {
        f[e] = (static_cast<float>((q0 >> (8 * e)) & 0xFFu) + OFF) * sc;
        f[4 + e] = (static_cast<float>((q1 >> (8 * e)) & 0xFFu) + OFF) * sc;
    }
    return make_uint4(pack_bf16x2(f[0], f[1]), pack_bf16x2(f[2], f[3]), pack_bf16x2(f[4], f[5]), pack_bf16x2(f[6], f[7]));
}

// Eight Q6_K codes q - 32 of lane group g: values l = 8g .. 8g + 7 of the 32-value block u = 4 hf + k of a
// super-block {ql[128], qh[64], sc[16], f16 d}: q = (low (k < 2) or high nibble of ql[64 hf + 32 (k & 1) + l]) |
// (bits 2k, 2k + 1 of qh[32 hf + l]) << 4 (ggml's Q6_K layout, Quant.KQuants.cs:36-107), as four bf16 pairs
// (exact: -32 .. 31). sbo: the super-block's first byte in the staged row (2-byte aligned), so each 8-byte
// run is three aligned words and a funnel shift.
__device__ __forceinline__ uint4 q6k_codes(const uint8_t* row, int sbo, int u, int g)
{
    const int hf = u >> 2, k = u & 3;
    auto bytes8 = [&](int q) {
        const uint32_t* w = reinterpret_cast<const uint32_t*>(row) + (q >> 2);
        const uint32_t sh = static_cast<uint32_t>(q & 3) * 8;
        const uint32_t w0 = w[0], w1 = w[1], w2 = w[2];
        return make_uint2(__builtin_amdgcn_alignbit(w1, w0, sh), __builtin_amdgcn_alignbit(w2, w1, sh));
    };
    const uint2 l = bytes8(sbo + 64 * hf + 32 * (k & 1) + 8 * g);
    const uint2 h = bytes8(sbo + 128 + 32 * hf + 8 * g);
    const uint32_t ls = 4 * static_cast<uint32_t>(k >> 1), hs = 2 * static_cast<uint32_t>(k);
    const uint32_t q0 = ((l.x >> ls) & 0x0F0F0F0Fu) | (((h.x >> hs) & 0x03030303u) << 4);
    const uint32_t q1 = ((l.y >> ls) & 0x0F0F0F0Fu) | (((h.y >> hs) & 0x03030303u) << 4);
    float f[8];
#pragma unroll
    for (int e = 0; e < 4; e++) {
        f[e] = static_cast<float>((q0 >> (8 * e)) & 0xFFu) - 32.0f;
        f[4 + e] = static_cast<float>((q1 >> (8 * e)) & 0xFFu) - 32.0f;
    }
    return make_uint4(pack_bf16x2(f[0], f[1]), pack_bf16x2(f[2], f[3]), pack_bf16x2(f[4], f[5]), pack_bf16x2(f[6], f[7]));
}

// x[0..7] (f32) as two bf16 vectors h + m: h = bf16(x), m = bf16(x - h); a non-finite x keeps only h.
__device__ __forceinline__ void split2(const float* x, uint4& h, uint4& m)
{
    uint32_t hw[4], mw[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float a0 = x[2 * i], a1 = x[2 * i + 1];
        hw[i] = pack_bf16x2(a0, a1);
        float r0 = a0 - bf16_lo(hw[i]), r1 = a1 - bf16_hi(hw[i]);
        r0 = r0 == r0 ? r0 : 0.0f;
        r1 = r1 == r1 ? r1 : 0.0f;
        mw[i] = pack_bf16x2(r0, r1);
    }
    h = make_uint4(hw[0], hw[1], hw[2], hw[3]);
    m = make_uint4(mw[0], mw[1], mw[2], mw[3]);
}

}  // namespace slhip
