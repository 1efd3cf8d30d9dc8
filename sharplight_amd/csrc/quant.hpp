// GGUF block formats decoded from a row image staged in LDS (the embedding gather and the quantized
// matvec). Decoders as the reference CPU provider's (Quant.Dequantize, src/Sharplight.Cpu/Quant.cs:242-405;
// Simd.StoreI8x16/StoreU8x16, Simd.cs:699-753): value = fma(q, d, offset) with the block's f16 scale d and
//   Q8_0: q int8, offset 0       Q4_0: q nibble, offset -8d    Q5_0: q 5-bit, offset -16d
//   Q4_1: q nibble, offset m     Q5_1: q 5-bit, offset m
// Every product is exact in f32. Blocks are 34, 18, 20, 22 or 24 bytes (only 2-byte aligned), so the
// readers below assemble words at even LDS byte offsets.
#pragma once

#include "common.hpp"

// plain device globals: as constant-address-space arrays, per-lane lookups were turned into scalar loads
#define SLHIP_GRID_QUAL static __device__ __attribute__((aligned(16)))
#include "iq_grids.h"
#include "trellis_codebook.h"

namespace slhip {

// BB: bytes per block; BS: values per block; QS / QH: byte offsets of the codes and of the fifth bits;
// M: an f16 minimum follows d; OFF: the offset in units of d. K: the block is decoded by decode_k.
template <int FMT> struct Fmt;
template <> struct Fmt<SLHIP_FMT_Q8_0> { static constexpr int BB = 34, BS = 32, QS = 2, QH = -1; static constexpr bool M = false, K = false; static constexpr int OFF = 0; };
template <> struct Fmt<SLHIP_FMT_Q4_0> { static constexpr int BB = 18, BS = 32, QS = 2, QH = -1; static constexpr bool M = false, K = false; static constexpr int OFF = -8; };
template <> struct Fmt<SLHIP_FMT_Q4_1> { static constexpr int BB = 20, BS = 32, QS = 4, QH = -1; static constexpr bool M = true, K = false; static constexpr int OFF = 0; };
template <> struct Fmt<SLHIP_FMT_Q5_0> { static constexpr int BB = 22, BS = 32, QS = 6, QH = 2; static constexpr bool M = false, K = false; static constexpr int OFF = -16; };
template <> struct Fmt<SLHIP_FMT_Q5_1> { static constexpr int BB = 24, BS = 32, QS = 8, QH = 4; static constexpr bool M = true, K = false; static constexpr int OFF = 0; };
template <> struct Fmt<SLHIP_FMT_Q2_K> { static constexpr int BB = 84, BS = 256, QS = 0, QH = -1; static constexpr bool M = false, K = true; static constexpr int OFF = 0; };
template <> struct Fmt<SLHIP_FMT_Q3_K> { static constexpr int BB = 110, BS = 256, QS = 0, QH = -1; static constexpr bool M = false, K = true; static constexpr int OFF = 0; };
template <> struct Fmt<SLHIP_FMT_Q4_K> { static constexpr int BB = 144, BS = 256, QS = 0, QH = -1; static constexpr bool M = false, K = true; static constexpr int OFF = 0; };
template <> struct Fmt<SLHIP_FMT_Q5_K> { static constexpr int BB = 176, BS = 256, QS = 0, QH = -1; static constexpr bool M = false, K = true; static constexpr int OFF = 0; };
template <> struct Fmt<SLHIP_FMT_Q6_K> { static constexpr int BB = 210, BS = 256, QS = 0, QH = -1; static constexpr bool M = false, K = true; static constexpr int OFF = 0; };
template <> struct Fmt<SLHIP_FMT_IQ4_NL> { static constexpr int BB = 18, BS = 32, QS = 2, QH = -1; static constexpr bool M = false, K = true; static constexpr int OFF = 0; };
template <> struct Fmt<SLHIP_FMT_IQ4_XS> { static constexpr int BB = 136, BS = 256, QS = 0, QH = -1; static constexpr bool M = false, K = true; static constexpr int OFF = 0; };
template <> struct Fmt<SLHIP_FMT_TQ1_0> { static constexpr int BB = 54, BS = 256, QS = 0, QH = -1; static constexpr bool M = false, K = true; static constexpr int OFF = 0; };
template <> struct Fmt<SLHIP_FMT_TQ2_0> { static constexpr int BB = 66, BS = 256, QS = 0, QH = -1; static constexpr bool M = false, K = true; static constexpr int OFF = 0; };
template <> struct Fmt<SLHIP_FMT_MXFP4> { static constexpr int BB = 17, BS = 32, QS = 0, QH = -1; static constexpr bool M = false, K = true; static constexpr int OFF = 0; };
template <> struct Fmt<SLHIP_FMT_NVFP4> { static constexpr int BB = 36, BS = 64, QS = 0, QH = -1; static constexpr bool M = false, K = true; static constexpr int OFF = 0; };
template <> struct Fmt<SLHIP_FMT_IQ2_XXS> { static constexpr int BB = 66, BS = 256, QS = 0, QH = -1; static constexpr bool M = false, K = true; static constexpr int OFF = 0; };
template <> struct Fmt<SLHIP_FMT_IQ2_XS> { static constexpr int BB = 74, BS = 256, QS = 0, QH = -1; static constexpr bool M = false, K = true; static constexpr int OFF = 0; };
template <> struct Fmt<SLHIP_FMT_IQ2_S> { static constexpr int BB = 82, BS = 256, QS = 0, QH = -1; static constexpr bool M = false, K = true; static constexpr int OFF = 0; };
template <> struct Fmt<SLHIP_FMT_IQ3_XXS> { static constexpr int BB = 98, BS = 256, QS = 0, QH = -1; static constexpr bool M = false, K = true; static constexpr int OFF = 0; };
template <> struct Fmt<SLHIP_FMT_IQ3_S> { static constexpr int BB = 110, BS = 256, QS = 0, QH = -1; static constexpr bool M = false, K = true; static constexpr int OFF = 0; };
template <> struct Fmt<SLHIP_FMT_IQ1_S> { static constexpr int BB = 50, BS = 256, QS = 0, QH = -1; static constexpr bool M = false, K = true; static constexpr int OFF = 0; };
template <> struct Fmt<SLHIP_FMT_IQ1_M> { static constexpr int BB = 56, BS = 256, QS = 0, QH = -1; static constexpr bool M = false, K = true; static constexpr int OFF = 0; };
// The reference's own formats (src/Sharplight.Core/Tensors/DataType.cs:154-244), all decoded by decode_k.
#define SLHIP_KFMT(F, bb, bs) \
    template <> struct Fmt<F> { static constexpr int BB = bb, BS = bs, QS = 0, QH = -1; static constexpr bool M = false, K = true; static constexpr int OFF = 0; };
SLHIP_KFMT(SLHIP_FMT_Q1_0, 18, 128)
SLHIP_KFMT(SLHIP_FMT_Q2_0, 18, 64)
SLHIP_KFMT(SLHIP_FMT_Q2_0_G128, 34, 128)
SLHIP_KFMT(SLHIP_FMT_TERN1_G128, 28, 128)
SLHIP_KFMT(SLHIP_FMT_NVFP4_GS, 40, 64)
SLHIP_KFMT(SLHIP_FMT_Q4Z_G32, 20, 32)
SLHIP_KFMT(SLHIP_FMT_Q4Z_G128, 68, 128)
SLHIP_KFMT(SLHIP_FMT_Q8Z_G32, 36, 32)
SLHIP_KFMT(SLHIP_FMT_Q8Z_G128, 132, 128)
SLHIP_KFMT(SLHIP_FMT_NF4_B64, 36, 64)
SLHIP_KFMT(SLHIP_FMT_FP4_B64, 36, 64)
SLHIP_KFMT(SLHIP_FMT_Q8A_G32, 36, 32)
SLHIP_KFMT(SLHIP_FMT_Q2S_G128, 36, 128)
SLHIP_KFMT(SLHIP_FMT_F8E4M3, 1, 1)
SLHIP_KFMT(SLHIP_FMT_F8E5M2, 1, 1)
SLHIP_KFMT(SLHIP_FMT_F8E4M3_B32, 36, 32)
SLHIP_KFMT(SLHIP_FMT_F8E4M3_B128, 132, 128)
SLHIP_KFMT(SLHIP_FMT_TRELLIS_V4K8_G128, 34, 128)
SLHIP_KFMT(SLHIP_FMT_TRELLIS_V4K6_G128, 26, 128)
SLHIP_KFMT(SLHIP_FMT_TRELLIS_V4K7_G128, 30, 128)
SLHIP_KFMT(SLHIP_FMT_TRELLIS_V2K5_G128, 42, 128)
SLHIP_KFMT(SLHIP_FMT_TRELLIS_V2K6_G128, 50, 128)
SLHIP_KFMT(SLHIP_FMT_TRELLIS_V2K7_G128, 58, 128)
#undef SLHIP_KFMT

// The 16-entry code books of NF4_B64 and FP4_B64 (the f32 values bitsandbytes stores as quant_map, as the
// reference lists them: src/Sharplight.Core/Tensors/Grids/Nf4CodeBook.cs, Fp4CodeBook.cs). Format data;
// plain device globals, per-lane loads (see iq_grids.h).
SLHIP_GRID_QUAL const float kNf4Values[16] = {
    -1.0f, -0.6961928009986877f, -0.5250730514526367f, -0.39491748809814453f, -0.28444138169288635f, -0.18477343022823334f,
    -0.09105003625154495f, 0.0f, 0.07958029955625534f, 0.16093020141124725f, 0.24611230194568634f, 0.33791524171829224f,
    0.44070982933044434f, 0.5626170039176941f, 0.7229568362236023f, 1.0f};
SLHIP_GRID_QUAL const float kFp4Values[16] = {
    0.0f, 0.0052083334885537624f, 0.6666666865348816f, 1.0f, 0.3333333432674408f, 0.5f, 0.1666666716337204f, 0.25f,
    0.0f, -0.0052083334885537624f, -0.6666666865348816f, -1.0f, -0.3333333432674408f, -0.5f, -0.1666666716337204f, -0.25f};

constexpr bool is_reference_fmt(int f) { return f >= SLHIP_FMT_Q1_0 && f <= SLHIP_FMT_TRELLIS_V2K7_G128; }
constexpr bool is_trellis_fmt(int f) { return f >= SLHIP_FMT_TRELLIS_V4K8_G128 && f <= SLHIP_FMT_TRELLIS_V2K7_G128; }

// Trellis codebook point p: its two f16 values as one word (the table is 16-byte aligned).
__device__ __forceinline__ uint32_t trellis_point(uint32_t p)
{
    return reinterpret_cast<const uint32_t*>(kTrellisCodebook)[p];
}

// An OCP E4M3FN byte as f32 (exact): bias 7, exponent 0 subnormal (m * 2^-9), 0x7F and 0xFF NaN, no infinity
// (Quant.E4m3ToFloat, src/Sharplight.Cpu/Quant.Fp8.cs:37-49).
__device__ __forceinline__ float e4m3_value(uint32_t x)
{
    const uint32_t e = (x >> 3) & 0xFu, m = x & 7u, sign = (x & 0x80u) << 24;
    if (e == 0xFu && m == 7u) return __uint_as_float(0x7FC00000u | sign);
    const uint32_t mag = e == 0 ? __float_as_uint(static_cast<float>(m) * 0x1p-9f) : ((e + 120u) << 23) | (m << 20);
    return __uint_as_float(mag | sign);
}

// An E5M2 byte: the top byte of an IEEE half (Quant.BuildE5m2, Quant.Fp8.cs:62-72).
__device__ __forceinline__ float e5m2_value(uint32_t x)
{
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(x << 8)));
}

constexpr bool is_grid_iq(int f)
{
    return f == SLHIP_FMT_IQ2_XXS || f == SLHIP_FMT_IQ2_XS || f == SLHIP_FMT_IQ2_S || f == SLHIP_FMT_IQ3_XXS ||
           f == SLHIP_FMT_IQ3_S || f == SLHIP_FMT_IQ1_S || f == SLHIP_FMT_IQ1_M;
}

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

// Byte access to a block image: in LDS (words) or in global memory. Multi-byte reads are at even offsets.
struct LdsBytes {
    const uint32_t* s;
    __device__ __forceinline__ uint32_t u8(int off) const { return (s[off >> 2] >> (8 * (off & 3))) & 0xFFu; }
    __device__ __forceinline__ uint32_t u16(int off) const { return lds_u16(s, off); }
    __device__ __forceinline__ uint32_t u32(int off) const { return lds_u32(s, off); }
    __device__ __forceinline__ float h(int off) const { return half_at(s, off); }
};

struct GlobalBytes {
    const uint8_t* p;
    __device__ __forceinline__ uint32_t u8(int off) const { return p[off]; }
    __device__ __forceinline__ uint32_t u16(int off) const { return p[off] | (static_cast<uint32_t>(p[off + 1]) << 8); }
    __device__ __forceinline__ uint32_t u32(int off) const { return u16(off) | (u16(off + 2) << 16); }
    __device__ __forceinline__ float h(int off) const
    {
        return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(u16(off))));
    }
};

// The IQ4 codebook {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113}
// (src/Sharplight.Cpu/Quant.cs:409) looked up for four nibble bytes at once: v_perm_b32 picks entries
// 0..7 and 8..15 from the table held as four words, and bit 3 of each nibble selects between them.
__device__ __forceinline__ uint32_t iq4_lookup4(uint32_t nib4)
{
    const uint32_t sel = nib4 & 0x07070707u;
    const uint32_t lo = __builtin_amdgcn_perm(0xF6EADDCFu, 0xBFAD9881u, sel);
    const uint32_t hi = __builtin_amdgcn_perm(0x71594535u, 0x26190D01u, sel);
    const uint32_t m = ((nib4 >> 3) & 0x01010101u) * 0xFFu;
    return (hi & m) | (lo & ~m);
}

// The E2M1 values doubled {0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12} (src/Sharplight.Cpu/
// Quant.Fp4.cs:10) as int8, looked up for four nibble bytes as iq4_lookup4 does.
__device__ __forceinline__ uint32_t fp4_lookup4(uint32_t nib4)
{
    const uint32_t sel = nib4 & 0x07070707u;
    const uint32_t lo = __builtin_amdgcn_perm(0x0C080604u, 0x03020100u, sel);
    const uint32_t hi = __builtin_amdgcn_perm(0xF4F8FAFCu, 0xFDFEFF00u, sel);
    const uint32_t m = ((nib4 >> 3) & 0x01010101u) * 0xFFu;
    return (hi & m) | (lo & ~m);
}

// MXFP4's E8M0 scale halved (the stored E2M1 values are doubled): 2^(e - 128), the two smallest exponents
// as f32 denormals (Quant.E8M0Half, Quant.Fp4.cs:36-41).
__device__ __forceinline__ float e8m0_half(uint32_t e)
{
    return __uint_as_float(e < 2 ? 0x00200000u << e : (e - 1) << 23);
}

// NVFP4's UE4M3 scale byte halved: 4 exponent bits (bias 7) and 3 mantissa bits, the top bit ignored,
// 0 and 0x7F read as zero (Quant.BuildUe4m3, Quant.Fp4.cs:14-33). Every value is exact in f32.
__device__ __forceinline__ float ue4m3_half(uint32_t x)
{
    const int e = static_cast<int>((x >> 3) & 0xFu), m = static_cast<int>(x & 7u);
    const float v = e == 0 ? __builtin_ldexpf(static_cast<float>(m), -10) : __builtin_ldexpf(static_cast<float>(8 + m), e - 11);
    return (x == 0x7Fu) ? 0.0f : v;
}

// Base-3 digit n (0..4) of byte q, minus one: ((q * 3^n mod 256) * 3 >> 8) - 1 (Quant.BuildTrits,
// Quant.Ternary.cs:10-25).
__device__ __forceinline__ int trit(uint32_t q, int n)
{
    const uint32_t p3 = n == 0 ? 1u : n == 1 ? 3u : n == 2 ? 9u : n == 3 ? 27u : 81u;
    return static_cast<int>((((q * p3) & 0xFFu) * 3u) >> 8) - 1;
}

// ksigns_iq2xs: the 7-bit index i with its parity as the eighth sign bit (bit j set: value j negative).
__device__ __forceinline__ uint32_t ksign(uint32_t i) { return i | ((__popc(i) & 1u) << 7); }

// One 8-value group g (0..31) of a grid IQ block at byte offset o (Quant.Iq.cs:113-306): the eight grid
// bytes (two 4-byte entries for the IQ3 formats), the sign bits and the group's scale; the IQ1 formats
// give the delta (+-1/8) instead of signs. The scales keep the reference's order of f32 operations.
template <int FMT, class B>
__device__ __forceinline__ void iq_group(const B& b, int o, int g, uint2& gv, uint32_t& signs, float& scale, float& delta)
{
    const int ib = g / 4, l = g % 4;
    signs = 0;
    delta = 0.0f;
    if constexpr (FMT == SLHIP_FMT_IQ2_XXS) {
        const uint32_t idx = b.u32(o + 2 + 8 * ib), ss = b.u32(o + 6 + 8 * ib);
        scale = __fmul_rn(__fmul_rn(b.h(o), 0.5f + static_cast<float>(ss >> 28)), 0.25f);
        const uint64_t e = kIq2xxsGrid[(idx >> (8 * l)) & 0xFFu];
        gv = make_uint2(static_cast<uint32_t>(e), static_cast<uint32_t>(e >> 32));
        signs = ksign((ss >> (7 * l)) & 127u);
    } else if constexpr (FMT == SLHIP_FMT_IQ2_XS || FMT == SLHIP_FMT_IQ2_S) {
        const uint32_t sc = b.u8(o + (FMT == SLHIP_FMT_IQ2_XS ? 66 : 74) + ib);
        scale = __fmul_rn(__fmul_rn(b.h(o), 0.5f + static_cast<float>(l < 2 ? (sc & 0xFu) : (sc >> 4))), 0.25f);
        uint64_t e;
        if constexpr (FMT == SLHIP_FMT_IQ2_XS) {
            const uint32_t q = b.u16(o + 2 + 2 * (4 * ib + l));
            e = kIq2xsGrid[q & 511u];
            signs = ksign(q >> 9);
        } else {
            const uint32_t index = b.u8(o + 2 + 4 * ib + l) | ((b.u8(o + 66 + ib) << (8 - 2 * l)) & 0x300u);
            e = kIq2sGrid[index];
            signs = b.u8(o + 34 + 4 * ib + l);
        }
        gv = make_uint2(static_cast<uint32_t>(e), static_cast<uint32_t>(e >> 32));
    } else if constexpr (FMT == SLHIP_FMT_IQ3_XXS) {
        const uint32_t w = b.u32(o + 66 + 4 * ib);
        scale = __fmul_rn(__fmul_rn(b.h(o), 0.5f + static_cast<float>(w >> 28)), 0.5f);
        gv = make_uint2(kIq3xxsGrid[b.u8(o + 2 + 8 * ib + 2 * l)], kIq3xxsGrid[b.u8(o + 2 + 8 * ib + 2 * l + 1)]);
        signs = ksign((w >> (7 * l)) & 127u);
    } else if constexpr (FMT == SLHIP_FMT_IQ3_S) {
        const uint32_t s4 = b.u8(o + 106 + ib / 2);
        scale = __fmul_rn(b.h(o), static_cast<float>(1 + 2 * static_cast<int>(ib % 2 == 0 ? (s4 & 0xFu) : (s4 >> 4))));
        const uint32_t high = b.u8(o + 66 + ib);
        const uint32_t lo = b.u8(o + 2 + 8 * ib + 2 * l) | ((high << (8 - 2 * l)) & 256u);
        const uint32_t hi = b.u8(o + 2 + 8 * ib + 2 * l + 1) | ((high << (7 - 2 * l)) & 256u);
        gv = make_uint2(kIq3sGrid[lo], kIq3sGrid[hi]);
        signs = b.u8(o + 74 + 4 * ib + l);
    } else if constexpr (FMT == SLHIP_FMT_IQ1_S) {
        const uint32_t qh = b.u16(o + 34 + 2 * ib);
        scale = __fmul_rn(b.h(o), static_cast<float>(2 * static_cast<int>((qh >> 12) & 7u) + 1));
        delta = (qh & 0x8000u) ? -0.125f : 0.125f;
        const uint64_t e = kIq1sGrid[b.u8(o + 2 + 4 * ib + l) | (((qh >> (3 * l)) & 7u) << 8)];
        gv = make_uint2(static_cast<uint32_t>(e), static_cast<uint32_t>(e >> 32));
    } else {  // IQ1_M
        const uint32_t s0 = b.u16(o + 48), s1 = b.u16(o + 50), s2 = b.u16(o + 52), s3 = b.u16(o + 54);
        const uint32_t bits = (s0 >> 12) | ((s1 >> 8) & 0x00F0u) | ((s2 >> 4) & 0x0F00u) | (s3 & 0xF000u);
        const float d = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(bits)));
        const uint32_t sw = b.u16(o + 48 + 2 * (ib / 2));
        const int sh = 6 * (ib % 2) + (l < 2 ? 0 : 3);
        scale = __fmul_rn(d, static_cast<float>(2 * static_cast<int>((sw >> sh) & 7u) + 1));
        const uint32_t qh = b.u8(o + 32 + 2 * ib + l / 2);
        const uint32_t index = b.u8(o + 4 * ib + l) | ((l % 2 == 0 ? (qh << 8) : (qh << 4)) & 0x700u);
        delta = (qh & (l % 2 == 0 ? 0x08u : 0x80u)) ? -0.125f : 0.125f;
        const uint64_t e = kIq1sGrid[index];
        gv = make_uint2(static_cast<uint32_t>(e), static_cast<uint32_t>(e >> 32));
    }
}

// N (4 or 8) consecutive values k .. k+N-1 (k a multiple of N) of a block of the reference's own formats at
// byte offset o, in the reference's arithmetic (one f32 rounding per product, subtractions not fused).
template <int FMT, int N, class B>
__device__ __forceinline__ void decode_ref(const B& b, int o, int k, float* f)
{
    auto byte_at = [&](int off) { return b.u8(off); };
    if constexpr (FMT == SLHIP_FMT_Q1_0) {
        // bit i of byte j is value 8j + i: +d when set, -d when clear (Quant.Q1_0, Quant.cs:656-669)
        const float d = b.h(o);
        const uint32_t bits = byte_at(o + 2 + k / 8) >> (k % 8);
#pragma unroll
        for (int e = 0; e < N; e++) f[e] = __fmul_rn((bits >> e) & 1u ? 1.0f : -1.0f, d);
    } else if constexpr (FMT == SLHIP_FMT_Q2_0 || FMT == SLHIP_FMT_Q2_0_G128) {
        // byte j holds values 4j .. 4j+3, value 4j+i in bits 2i, 2i+1; (code - 1) * d (Quant.Q2_0, Quant.cs:673-686)
        const float d = b.h(o);
        const uint32_t w = N == 8 ? b.u16(o + 2 + k / 4) : byte_at(o + 2 + k / 4);
#pragma unroll
        for (int e = 0; e < N; e++) f[e] = __fmul_rn(static_cast<float>(static_cast<int>((w >> (2 * e)) & 3u) - 1), d);
    } else if constexpr (FMT == SLHIP_FMT_TERN1_G128) {
        // digit n of byte m: values n*16 + m (bytes 0..15), 80 + n*8 + m (bytes 16..23), 120 + 2n + h (bytes 24, 25);
        // digit times d (Quant.Tern1, Quant.cs:689-718)
        const float d = b.h(o + 26);
        if (k < 120) {
            const bool a = k < 80;
            const int n = a ? k / 16 : (k - 80) / 8;
            const int m = a ? k % 16 : 16 + (k - 80) % 8;
#pragma unroll
            for (int e = 0; e < N; e++) f[e] = __fmul_rn(static_cast<float>(trit(byte_at(o + m + e), n)), d);
        } else {
#pragma unroll
            for (int e = 0; e < N; e++) {
                const int r = k - 120 + e;
                f[e] = __fmul_rn(static_cast<float>(trit(byte_at(o + 24 + r % 2), r / 2)), d);
            }
        }
    } else if constexpr (FMT == SLHIP_FMT_NVFP4_GS) {
        // {f32 g; u8 d[4]; u8 qs[32]}: the sub-block multiplier UE4M3 * g rounded once, then times the doubled
        // E2M1 code, as NVFP4 (Quant.NVFP4_GS, Quant.Fp4.cs:86-107)
        const int sb = k / 16, i = k % 16;
        const float d = __fmul_rn(ue4m3_half(byte_at(o + 4 + sb)), __uint_as_float(b.u32(o)));
        uint32_t w[N / 4];
#pragma unroll
        for (int x = 0; x < N / 4; x++) w[x] = fp4_lookup4(((i >= 8 ? b.u32(o + 8 + 8 * sb + i % 8 + 4 * x) >> 4 : b.u32(o + 8 + 8 * sb + i % 8 + 4 * x))) & 0x0F0F0F0Fu);
#pragma unroll
        for (int e = 0; e < N; e++) f[e] = __fmul_rn(static_cast<float>(static_cast<int8_t>((w[e >> 2] >> (8 * (e & 3))) & 0xFFu)), d);
    } else if constexpr (FMT == SLHIP_FMT_Q4Z_G32 || FMT == SLHIP_FMT_Q4Z_G128 || FMT == SLHIP_FMT_NF4_B64 ||
                         FMT == SLHIP_FMT_FP4_B64) {
        // 32-value runs of 16 code bytes: value j the low nibble of byte j, j + 16 the high nibble.
        // Q4Z: {f16 d; f16 z; codes} -> (q - z) * d (Quant.Q4Z, Quant.Grouped.cs:66-83; Quant.StoreU8x16Zeroed,
        // Quant.Absmax.cs:13-23); NF4/FP4: {f32 d; codes} -> book[q] * d (Quant.LookupB64, Quant.Grouped.cs:107-127)
        constexpr bool Z = FMT == SLHIP_FMT_Q4Z_G32 || FMT == SLHIP_FMT_Q4Z_G128;
        const int run = k / 32, i = k % 32;
        const int qo = o + 4 + 16 * run + i % 16;
#pragma unroll
        for (int x = 0; x < N / 4; x++) {
            const uint32_t w = (i >= 16 ? b.u32(qo + 4 * x) >> 4 : b.u32(qo + 4 * x)) & 0x0F0F0F0Fu;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const uint32_t q = (w >> (8 * e)) & 0xFFu;
                if constexpr (Z) {
                    f[4 * x + e] = __fmul_rn(__fsub_rn(static_cast<float>(q), b.h(o + 2)), b.h(o));
                } else {
                    const float book = FMT == SLHIP_FMT_NF4_B64 ? kNf4Values[q] : kFp4Values[q];
                    f[4 * x + e] = __fmul_rn(book, __uint_as_float(b.u32(o)));
                }
            }
        }
    } else if constexpr (FMT == SLHIP_FMT_Q8Z_G32 || FMT == SLHIP_FMT_Q8Z_G128) {
        // {f16 d; f16 z; u8 q[group]} -> (q - z) * d (Quant.Q8Z, Quant.Grouped.cs:86-98)
        const float d = b.h(o), z = b.h(o + 2);
#pragma unroll
        for (int x = 0; x < N / 4; x++) {
            const uint32_t w = b.u32(o + 4 + k + 4 * x);
#pragma unroll
            for (int e = 0; e < 4; e++) f[4 * x + e] = __fmul_rn(__fsub_rn(static_cast<float>((w >> (8 * e)) & 0xFFu), z), d);
        }
    } else if constexpr (FMT == SLHIP_FMT_Q8A_G32) {
        // {f32 d; i8 q[32]} -> (q * d) * (1/127 as f32) (Quant.Q8A_G32, Quant.Absmax.cs:29-40)
        const float d = __uint_as_float(b.u32(o));
#pragma unroll
        for (int x = 0; x < N / 4; x++) {
            const uint32_t w = b.u32(o + 4 + k + 4 * x);
#pragma unroll
            for (int e = 0; e < 4; e++)
                f[4 * x + e] = __fmul_rn(__fmul_rn(static_cast<float>(static_cast<int8_t>((w >> (8 * e)) & 0xFFu)), d),
                                         7.874015718698502e-3f);
        }
    } else if constexpr (FMT == SLHIP_FMT_Q2S_G128) {
        // {f32 d; u8 qs[32]}: byte j holds values j, 32 + j, 64 + j, 96 + j in bits 6, 4, 2, 0 -> (code - 1) * d
        // (Quant.Q2S_G128, Quant.Absmax.cs:43-57)
        const float d = __uint_as_float(b.u32(o));
        const int sh = 6 - 2 * (k / 32);
#pragma unroll
        for (int x = 0; x < N / 4; x++) {
            const uint32_t w = b.u32(o + 4 + k % 32 + 4 * x);
#pragma unroll
            for (int e = 0; e < 4; e++)
                f[4 * x + e] = __fmul_rn(static_cast<float>(static_cast<int>((w >> (8 * e + sh)) & 3u) - 1), d);
        }
    } else if constexpr (is_trellis_fmt(FMT)) {
        // {f16 d; path bytes}: step t (V values) has a 16-bit state, for K = 8 the bytes t-1 (mod steps) and t,
        // otherwise the 16 bits at bit (steps-1-t)*K of the circular K*steps-bit stream, LSB first; the low 15
        // bits hash to x = s * 0x9e3779b1 (mod 2^32), codebook point x >> 21 gives values 0-1 of the step and
        // (V = 4) point (x >> 10) & 2047 values 2-3; value = d * point (TrellisBlocks.State / DecodeBlock,
        // src/Sharplight.Core/Tensors/TrellisBlocks.cs:61-102)
        constexpr int V = FMT <= SLHIP_FMT_TRELLIS_V4K7_G128 ? 4 : 2;
        constexpr int KB = FMT == SLHIP_FMT_TRELLIS_V4K8_G128 ? 8 : FMT == SLHIP_FMT_TRELLIS_V4K6_G128 ? 6
                         : FMT == SLHIP_FMT_TRELLIS_V4K7_G128 ? 7 : FMT == SLHIP_FMT_TRELLIS_V2K5_G128 ? 5
                         : FMT == SLHIP_FMT_TRELLIS_V2K6_G128 ? 6 : 7;
        constexpr int STEPS = 128 / V, BYTES = STEPS * KB / 8;
        const float d = b.h(o);
        const int qs = o + 2;
#pragma unroll
        for (int s = 0; s < N / V; s++) {
            const int t = k / V + s;
            uint32_t st;
            if constexpr (KB == 8) {
                st = (byte_at(qs + (t + STEPS - 1) % STEPS) << 8) | byte_at(qs + t);
            } else {
                const int off = (STEPS - 1 - t) * KB, i0 = off >> 3;
                const uint32_t w = byte_at(qs + i0) | (byte_at(qs + (i0 + 1) % BYTES) << 8) |
                                   (byte_at(qs + (i0 + 2) % BYTES) << 16);
                st = (w >> (off & 7)) & 0xFFFFu;
            }
            const uint32_t x = (st & 0x7FFFu) * 0x9E3779B1u;
            const uint32_t p0 = trellis_point(x >> 21);
            f[V * s + 0] = __fmul_rn(d, f16_lo(p0));
            f[V * s + 1] = __fmul_rn(d, f16_hi(p0));
            if constexpr (V == 4) {
                const uint32_t p1 = trellis_point((x >> 10) & 2047u);
                f[V * s + 2] = __fmul_rn(d, f16_lo(p1));
                f[V * s + 3] = __fmul_rn(d, f16_hi(p1));
            }
        }
    } else {
        // FP8: plain E4M3 / E5M2 bytes (times 1), or {f32 d; E4M3 q[block]} -> e4m3(q) * d
        // (Quant.DequantizeFp8 / ScaledE4m3Blocks / Lookup, Quant.Fp8.cs:78-137)
        constexpr bool SCALED = FMT == SLHIP_FMT_F8E4M3_B32 || FMT == SLHIP_FMT_F8E4M3_B128;
        const float d = SCALED ? __uint_as_float(b.u32(o)) : 1.0f;
        const int qo = SCALED ? o + 4 + k : o + k;
#pragma unroll
        for (int x = 0; x < N / 4; x++) {
            const uint32_t w = b.u32(qo + 4 * x);
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const uint32_t q = (w >> (8 * e)) & 0xFFu;
                f[4 * x + e] = __fmul_rn(FMT == SLHIP_FMT_F8E5M2 ? e5m2_value(q) : e4m3_value(q), d);
            }
        }
    }
}

// N (4 or 8) consecutive values k .. k+N-1 (k a multiple of N) of the K-quant or codebook block at byte
// offset o, decoded with the reference's arithmetic (src/Sharplight.Cpu/Quant.cs:407-446,500-624,
// Quant.KQuants.cs:36-107): the N values share one sub-block scale.
template <int FMT, int N, class B>
__device__ __forceinline__ void decode_k(const B& b, int o, int k, float* f)
{
    uint32_t w[N / 4];
    auto words = [&](int off) {
#pragma unroll
        for (int h = 0; h < N / 4; h++) w[h] = b.u32(off + 4 * h);
    };
    auto byte_of = [&](const uint32_t* ws, int e) { return (ws[e >> 2] >> (8 * (e & 3))) & 0xFFu; };
    if constexpr (FMT == SLHIP_FMT_Q4_K || FMT == SLHIP_FMT_Q5_K) {
        const int g = k / 64, half = (k % 64) / 32, i = k % 32, j = 2 * g + half;
        const int sb = o + 4;
        uint32_t sc, m;
        if (j < 4) {
            sc = b.u8(sb + j) & 63u;
            m = b.u8(sb + j + 4) & 63u;
        } else {
            sc = (b.u8(sb + j + 4) & 0xFu) | ((b.u8(sb + j - 4) >> 6) << 4);
            m = (b.u8(sb + j + 4) >> 4) | ((b.u8(sb + j) >> 6) << 4);
        }
        const float dl = b.h(o) * static_cast<float>(sc), mm = b.h(o + 2) * static_cast<float>(m);
        words(o + (FMT == SLHIP_FMT_Q5_K ? 48 : 16) + 32 * g + i);
        uint32_t hw[N / 4];
        if (FMT == SLHIP_FMT_Q5_K) {
#pragma unroll
            for (int h = 0; h < N / 4; h++) hw[h] = (b.u32(o + 16 + i + 4 * h) >> j) & 0x01010101u;
        }
#pragma unroll
        for (int h = 0; h < N / 4; h++) {
            w[h] = (w[h] >> (4 * half)) & 0x0F0F0F0Fu;
            if (FMT == SLHIP_FMT_Q5_K) w[h] |= hw[h] << 4;
        }
#pragma unroll
        for (int e = 0; e < N; e++) f[e] = __fmaf_rn(static_cast<float>(byte_of(w, e)), dl, -mm);
    } else if constexpr (FMT == SLHIP_FMT_Q6_K) {
        const int n = k / 128, r = k % 128, qt = r / 32, i = r % 32, h = i / 16;
        words(o + 64 * n + (qt & 1 ? 32 : 0) + i);
        uint32_t hw[N / 4];
#pragma unroll
        for (int x = 0; x < N / 4; x++) hw[x] = (b.u32(o + 128 + 32 * n + i + 4 * x) >> (2 * qt)) & 0x03030303u;
#pragma unroll
        for (int x = 0; x < N / 4; x++) w[x] = ((qt >= 2 ? w[x] >> 4 : w[x]) & 0x0F0F0F0Fu) | (hw[x] << 4);
        const float s = b.h(o + 208) * static_cast<float>(static_cast<int8_t>(b.u8(o + 192 + 8 * n + h + 2 * qt)));
#pragma unroll
        for (int e = 0; e < N; e++) f[e] = __fmaf_rn(static_cast<float>(byte_of(w, e)), s, -32.0f * s);
    } else if constexpr (FMT == SLHIP_FMT_Q2_K || FMT == SLHIP_FMT_Q3_K) {
        const int n = k / 128, r = k % 128, j = r / 32, h = (r % 32) / 16, i = r % 16;
        const int si = 8 * n + 2 * j + h;
        if constexpr (FMT == SLHIP_FMT_Q2_K) {
            words(o + 16 + 32 * n + 16 * h + i);
            const uint32_t sc = b.u8(o + si);
            const float dl = __fmul_rn(b.h(o + 80), static_cast<float>(sc & 0xFu));
            const float ml = __fmul_rn(b.h(o + 82), static_cast<float>(sc >> 4));
#pragma unroll
            for (int x = 0; x < N / 4; x++) w[x] = (w[x] >> (2 * j)) & 0x03030303u;
#pragma unroll
            for (int e = 0; e < N; e++) f[e] = __fsub_rn(__fmul_rn(static_cast<float>(byte_of(w, e)), dl), ml);
        } else {
            const int ww = si / 4, bb = si % 4;
            const uint32_t a = b.u8(o + 96 + 4 * (ww & 1) + bb);
            const uint32_t sc = (ww < 2 ? (a & 0xFu) : (a >> 4)) | (((b.u8(o + 104 + bb) >> (2 * ww)) & 3u) << 4);
            const float dl = __fmul_rn(b.h(o + 108), static_cast<float>(static_cast<int>(sc) - 32));
            words(o + 32 + 32 * n + 16 * h + i);
            uint32_t hw[N / 4];
#pragma unroll
            for (int x = 0; x < N / 4; x++) hw[x] = (b.u32(o + 16 * h + i + 4 * x) >> (4 * n + j)) & 0x01010101u;
#pragma unroll
            for (int e = 0; e < N; e++) {
                const int v = static_cast<int>((byte_of(w, e) >> (2 * j)) & 3u) + 4 * static_cast<int>(byte_of(hw, e)) - 4;
                f[e] = __fmul_rn(static_cast<float>(v), dl);
            }
        }
    } else if constexpr (is_grid_iq(FMT)) {
        // (grid byte * (+-1)) * scale for IQ2/IQ3 (Quant.StoreSigned8/4x2), (grid + delta) * scale for IQ1
        // (Quant.StoreIq1): one rounding per value
        uint2 gv;
        uint32_t signs;
        float scale, delta;
        iq_group<FMT>(b, o, k / 8, gv, signs, scale, delta);
        const int j0 = k % 8;  // 0, or 4 when N = 4
        // The word is chosen by a select: indexed as a two-entry array with the runtime j0, the compiler
        // folded the index into the table address and loaded it as if it were the same for every lane.
        const uint32_t w_lo = N == 8 ? gv.x : (j0 == 0 ? gv.x : gv.y);
#pragma unroll
        for (int e = 0; e < N; e++) {
            const int j = j0 + e;
            const uint32_t byte = ((e < 4 ? w_lo : gv.y) >> (8 * (e & 3))) & 0xFFu;
            if constexpr (FMT == SLHIP_FMT_IQ1_S || FMT == SLHIP_FMT_IQ1_M) {
                f[e] = __fmul_rn(static_cast<float>(static_cast<int8_t>(byte)) + delta, scale);
            } else {
                const float v = static_cast<float>(byte);
                f[e] = __fmul_rn((signs >> j) & 1u ? -v : v, scale);
            }
        }
    } else if constexpr (FMT == SLHIP_FMT_MXFP4) {
        // {u8 e; u8 qs[16]}: value j < 16 the low nibble of qs[j], j >= 16 the high nibble of qs[j - 16]
        // (Quant.MXFP4, Quant.Fp4.cs:43-58); value = fp4 * scale
        const float d = e8m0_half(b.u8(o));
        const int i = k % 32;
        words(o + 1 + (i % 16));
#pragma unroll
        for (int x = 0; x < N / 4; x++) w[x] = fp4_lookup4(((i >= 16) ? w[x] >> 4 : w[x]) & 0x0F0F0F0Fu);
#pragma unroll
        for (int e = 0; e < N; e++) f[e] = __fmul_rn(static_cast<float>(static_cast<int8_t>(byte_of(w, e))), d);
    } else if constexpr (FMT == SLHIP_FMT_NVFP4) {
        // {u8 d[4]; u8 qs[32]}: four 16-value sub-blocks, each with a UE4M3 scale and 8 code bytes, low
        // nibbles first (Quant.NVFP4, Quant.Fp4.cs:60-80)
        const int sb = k / 16, i = k % 16;
        const float d = ue4m3_half(b.u8(o + sb));
        words(o + 4 + 8 * sb + (i % 8));
#pragma unroll
        for (int x = 0; x < N / 4; x++) w[x] = fp4_lookup4(((i >= 8) ? w[x] >> 4 : w[x]) & 0x0F0F0F0Fu);
#pragma unroll
        for (int e = 0; e < N; e++) f[e] = __fmul_rn(static_cast<float>(static_cast<int8_t>(byte_of(w, e))), d);
    } else if constexpr (FMT == SLHIP_FMT_TQ2_0) {
        // {u8 qs[64]; f16 d}: value (4j + l) * 32 + m = ((qs[32j + m] >> 2l) & 3) - 1, times d
        // (Quant.TQ2_0, Quant.Ternary.cs:66-86)
        const int j = k / 128, l = (k % 128) / 32, m = k % 32;
        const float d = b.h(o + 64);
        words(o + 32 * j + m);
#pragma unroll
        for (int e = 0; e < N; e++)
            f[e] = __fmul_rn(static_cast<float>(static_cast<int>((byte_of(w, e) >> (2 * l)) & 3u) - 1), d);
    } else if constexpr (FMT == SLHIP_FMT_TQ1_0) {
        // {u8 qs[48]; u8 qh[4]; f16 d}: five base-3 digits per byte -- values n*32 + m from digit n of
        // qs[m], 160 + n*16 + m from qs[32 + m], 240 + n*4 + j from qh[j] (Quant.TQ1_0, Quant.Ternary.cs:27-64)
        const float d = b.h(o + 52);
        if (k < 240) {  // N values of one digit of consecutive bytes
            const bool a = k < 160;
            const int n = a ? k / 32 : (k - 160) / 16;
            words(o + (a ? k % 32 : 32 + (k - 160) % 16));
#pragma unroll
            for (int e = 0; e < N; e++) f[e] = __fmul_rn(static_cast<float>(trit(byte_of(w, e), n)), d);
        } else {  // the last 16: digit n of qh[j] for value 240 + 4n + j
            const uint32_t qh = b.u32(o + 48);
#pragma unroll
            for (int e = 0; e < N; e++) {
                const int r = k - 240 + e;
                f[e] = __fmul_rn(static_cast<float>(trit((qh >> (8 * (r % 4))) & 0xFFu, r / 4)), d);
            }
        }
    } else if constexpr (is_reference_fmt(FMT)) {
        decode_ref<FMT, N>(b, o, k, f);
    } else {  // IQ4_NL, IQ4_XS
        float dl;
        int qo, i;
        if constexpr (FMT == SLHIP_FMT_IQ4_NL) {
            dl = b.h(o);
            i = k % 32;
            qo = o + 2 + (i % 16);
        } else {
            const int ib = k / 32;
            i = k % 32;
            const uint32_t ls = ((b.u8(o + 4 + ib / 2) >> (4 * (ib % 2))) & 0xFu) | (((b.u16(o + 2) >> (2 * ib)) & 3u) << 4);
            dl = __fmul_rn(b.h(o), static_cast<float>(static_cast<int>(ls) - 32));
            qo = o + 8 + 16 * ib + (i % 16);
        }
        words(qo);
#pragma unroll
        for (int x = 0; x < N / 4; x++) w[x] = iq4_lookup4(((i >= 16) ? w[x] >> 4 : w[x]) & 0x0F0F0F0Fu);
#pragma unroll
        for (int e = 0; e < N; e++) f[e] = __fmul_rn(dl, static_cast<float>(static_cast<int8_t>(byte_of(w, e))));
    }
}

// Decodes N (4 or 8) consecutive values starting at value j0 (a multiple of N) of the row image in LDS.
template <int FMT, int N>
__device__ __forceinline__ void decode(const uint32_t* s, int j0, float* f)
{
    if constexpr (Fmt<FMT>::K) {
        decode_k<FMT, N>(LdsBytes{s}, (j0 / Fmt<FMT>::BS) * Fmt<FMT>::BB, j0 % Fmt<FMT>::BS, f);
    } else {
        float q[N], d, add;
        codes<FMT, N>(s, j0, q, d, add);
#pragma unroll
        for (int e = 0; e < N; e++) f[e] = __fmaf_rn(q[e], d, add);
    }
}

}  // namespace slhip
