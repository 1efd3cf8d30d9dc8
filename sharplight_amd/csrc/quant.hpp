// GGUF legacy block formats decoded from a row image staged in LDS (the embedding gather and the quantized
// matvec). Decoders as the reference CPU provider's (Quant.Dequantize, src/Sharplight.Cpu/Quant.cs:242-405;
// Simd.StoreI8x16/StoreU8x16, Simd.cs:699-753): value = fma(q, d, offset) with the block's f16 scale d and
//   Q8_0: q int8, offset 0       Q4_0: q nibble, offset -8d    Q5_0: q 5-bit, offset -16d
//   Q4_1: q nibble, offset m     Q5_1: q 5-bit, offset m
// Every product is exact in f32. Blocks are 34, 18, 20, 22 or 24 bytes (only 2-byte aligned), so the
// readers below assemble words at even LDS byte offsets.
#pragma once

#include "common.hpp"

namespace slhip {

template <int FMT> struct Fmt;
template <> struct Fmt<SLHIP_FMT_Q8_0> { static constexpr int BB = 34, QS = 2, QH = -1; static constexpr bool M = false; static constexpr int OFF = 0; };
template <> struct Fmt<SLHIP_FMT_Q4_0> { static constexpr int BB = 18, QS = 2, QH = -1; static constexpr bool M = false; static constexpr int OFF = -8; };
template <> struct Fmt<SLHIP_FMT_Q4_1> { static constexpr int BB = 20, QS = 4, QH = -1; static constexpr bool M = true; static constexpr int OFF = 0; };
template <> struct Fmt<SLHIP_FMT_Q5_0> { static constexpr int BB = 22, QS = 6, QH = 2; static constexpr bool M = false; static constexpr int OFF = -16; };
template <> struct Fmt<SLHIP_FMT_Q5_1> { static constexpr int BB = 24, QS = 8, QH = 4; static constexpr bool M = true; static constexpr int OFF = 0; };

__device__ __forceinline__ uint32_t lds_u16(const uint32_t* s, int off)
{
    uint32_t w = s[off >> 2];
    return (off & 2) ? (w >> 16) : (w & 0xFFFFu);
}

// 4 bytes at an even LDS byte offset.
__device__ __forceinline__ uint32_t lds_u32(const uint32_t* s, int off)
{
    const int i = off >> 2;
    const uint32_t sh = (off & 3) * 8;
    return __builtin_amdgcn_alignbit(s[i + 1], s[i], sh);
}

// 8 bytes at an even LDS byte offset, as two little-endian words.
__device__ __forceinline__ uint2 lds_u64(const uint32_t* s, int off)
{
    const int i = off >> 2;
    const uint32_t sh = (off & 3) * 8;
    const uint32_t w0 = s[i], w1 = s[i + 1], w2 = s[i + 2];
    return make_uint2(__builtin_amdgcn_alignbit(w1, w0, sh), __builtin_amdgcn_alignbit(w2, w1, sh));
}

__device__ __forceinline__ float half_at(const uint32_t* s, int off)
{
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(lds_u16(s, off))));
}

// A whole block of a row image in LDS for a dot product: its scale d, additive term (OFF * d, or m) and the
// raw code words -- Q8_0: 8 words of int8 codes; Q4_x: 4 words of nibble pairs; Q5_x: the same plus the 32
// fifth bits in hi.
template <int FMT> struct BlockWords {
    float d, add;
    uint32_t w[FMT == SLHIP_FMT_Q8_0 ? 8 : 4];
    uint32_t hi;
};

template <int FMT>
__device__ __forceinline__ BlockWords<FMT> block_words(const uint32_t* s, int b)
{
    using F = Fmt<FMT>;
    BlockWords<FMT> r;
    const int o = b * F::BB;
    r.d = half_at(s, o);
    r.add = FMT == SLHIP_FMT_Q8_0 ? 0.0f : F::M ? half_at(s, o + 2) : static_cast<float>(F::OFF) * r.d;
    constexpr int NW = FMT == SLHIP_FMT_Q8_0 ? 8 : 4;
    // NW + 1 aligned words cover the NW words at the (even) byte offset o + QS
    const int q0 = o + F::QS;
    const int i0 = q0 >> 2;
    const uint32_t sh = (q0 & 3) * 8;
    uint32_t raw[NW + 1];
#pragma unroll
    for (int k = 0; k <= NW; k++) raw[k] = s[i0 + k];
#pragma unroll
    for (int k = 0; k < NW; k++) r.w[k] = __builtin_amdgcn_alignbit(raw[k + 1], raw[k], sh);
    r.hi = F::QH >= 0 ? lds_u32(s, o + (F::QH >= 0 ? F::QH : 0)) : 0u;
    return r;
}

// The codes of values 8j .. 8j+7 of a block as floats (j = 0..3).
template <int FMT>
__device__ __forceinline__ void block_codes8(const BlockWords<FMT>& bw, int j, float* q)
{
    using F = Fmt<FMT>;
    if (FMT == SLHIP_FMT_Q8_0) {
#pragma unroll
        for (int e = 0; e < 8; e++)
            q[e] = static_cast<float>(static_cast<int8_t>(bw.w[2 * j + (e >> 2)] >> (8 * (e & 3))));
        return;
    }
    // value k < 16: low nibble of byte k; k >= 16: high nibble of byte k - 16
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const uint32_t word = bw.w[2 * (j & 1) + h];
        uint32_t nib = (j >= 2 ? word >> 4 : word) & 0x0F0F0F0Fu;
        if (F::QH < 0) asm("" : "+v"(nib));  // see codes(): keeps one byte conversion per value
#pragma unroll
        for (int e = 0; e < 4; e++) {
            uint32_t v = (nib >> (8 * e)) & 0xFFu;
            if (F::QH >= 0) v |= ((bw.hi >> (8 * j + 4 * h + e)) & 1u) << 4;
            q[4 * h + e] = static_cast<float>(v);
        }
    }
}

// Decodes N (4 or 8) consecutive values starting at value j0 (a multiple of N) of the chunk in LDS.
// The codes of N (4 or 8) consecutive values starting at value j0 (a multiple of N) of the row image in LDS,
// as floats, with their block's scale d and additive term (OFF * d, or m): value = fma(q, d, add).
template <int FMT, int N>
__device__ __forceinline__ void codes(const uint32_t* s, int j0, float* q, float& d, float& add)
{
    using F = Fmt<FMT>;
    const int o = (j0 >> 5) * F::BB;  // the value's block
    const int k0 = j0 & 31;           // first value index within the block
    d = half_at(s, o);
    uint32_t b[2];
    if (FMT == SLHIP_FMT_Q8_0) {
        add = 0.0f;
        if (N == 8) {
            const uint2 w = lds_u64(s, o + F::QS + k0);
            b[0] = w.x;
            b[1] = w.y;
        } else {
            b[0] = lds_u32(s, o + F::QS + k0);
        }
#pragma unroll
        for (int e = 0; e < N; e++) q[e] = static_cast<float>(static_cast<int8_t>(b[e >> 2] >> (8 * (e & 3))));
        return;
    }
    // Nibble blocks: value k < 16 is the low nibble of qs[k], k >= 16 the high nibble of qs[k - 16]; the
    // 5-bit formats take bit k of the 32-bit qh as the fifth bit.
    add = F::M ? half_at(s, o + 2) : static_cast<float>(F::OFF) * d;
    const int kk = k0 & 15;
    const int shift = k0 >= 16 ? 4 : 0;
    if (N == 8) {
        const uint2 w = lds_u64(s, o + F::QS + kk);
        b[0] = w.x;
        b[1] = w.y;
    } else {
        b[0] = lds_u32(s, o + F::QS + kk);
    }
    uint32_t qh = 0;
    if (F::QH >= 0) qh = lds_u32(s, o + F::QH) >> k0;
    // Four nibbles at once: rotating the word by the nibble shift and masking leaves one value per byte,
    // which converts with a single byte-to-float instruction (the rotate keeps the compiler from folding
    // the mask back into one bit-field extract per value).
    // The empty asm hides that the masked bytes' high nibbles are zero: knowing it, the compiler would turn
    // each byte conversion back into a bit-field extract plus a conversion.
    uint32_t nib[2];
#pragma unroll
    for (int h = 0; h < N / 4; h++) {
        nib[h] = __builtin_amdgcn_alignbit(b[h], b[h], shift) & 0x0F0F0F0Fu;
        if (F::QH < 0) asm("" : "+v"(nib[h]));
    }
#pragma unroll
    for (int e = 0; e < N; e++) {
        uint32_t v = (nib[e >> 2] >> (8 * (e & 3))) & 0xFFu;
        if (F::QH >= 0) v |= ((qh >> e) & 1u) << 4;
        q[e] = static_cast<float>(v);
    }
}

// Decodes N (4 or 8) consecutive values starting at value j0 (a multiple of N) of the row image in LDS.
template <int FMT, int N>
__device__ __forceinline__ void decode(const uint32_t* s, int j0, float* f)
{
    float q[N], d, add;
    codes<FMT, N>(s, j0, q, d, add);
#pragma unroll
    for (int e = 0; e < N; e++) f[e] = __fmaf_rn(q[e], d, add);
}

}  // namespace slhip
