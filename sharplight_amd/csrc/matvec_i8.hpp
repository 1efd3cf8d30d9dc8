#pragma once
// The integer-dot decode matvec's kernels and launch templates. matvec_i8.hip holds the activation
// quantization, the entry points and the description of the numerics; matvec_i8_0..3.hip instantiate the
// weight formats in separate units so that they compile in parallel.
#include "act.hpp"
#include "common.hpp"
#include "lds_dma.hpp"
#include "quant.hpp"

#include <limits.h>
#include <stdlib.h>

#include <type_traits>

namespace slhip {


struct I8Args {
    const uint8_t* xq;  // [T, 1.5 K] quantized activation rows
    const char* wg;     // N rows of wrow bytes
    const char* wu;     // the second matrix of a dual matvec, else null
    int64_t wrow;
    void* y;  // [T, N], row stride ys elements
    int64_t ys;
    int64_t T, K, N;
    int64_t t0;        // first activation row of this launch
    int yt;            // SLHIP_F32 / SLHIP_BF16
    int act;           // dual: SLHIP_ACT_*
    const float* bias;  // [N] f32 added to each output row (single matvec), or null
};

constexpr int kI8Threads = 256;

// ---- weight units ------------------------------------------------------------------------------------------

template <int FMT>
constexpr int kUnitsPerBlock = Fmt<FMT>::BS / 32;  // 32-value units per format block

// How a unit's terms combine: one (a, b) per 32 values; one a per 32 and no offset (signed codes); or an
// (a, b) pair per 16 values (Q6_K).
enum { kScale32Off = 0, kScale32 = 1, kScale16Off = 2 };
template <int FMT>
constexpr int kUnitForm = FMT == SLHIP_FMT_Q6_K ? kScale16Off
                          : (FMT == SLHIP_FMT_Q8_0 || FMT == SLHIP_FMT_IQ4_NL || FMT == SLHIP_FMT_IQ4_XS ||
                             FMT == SLHIP_FMT_MXFP4)
                              ? kScale32
                              : kScale32Off;

struct I8Unit {
    uint32_t c[8];  // value 4k + e in byte e of c[k]
    float a0, a1, b0, b1;
};

// Unit b (0 .. K/32 - 1) of a row image in LDS: the codes and scales of IntDot.Decode (IntDot.Decode.cs:89-293).
template <int FMT>
__device__ __forceinline__ I8Unit i8_unit(const uint32_t* s, int b)
{
    I8Unit r;
    const LdsBytes B{s};
    r.b0 = r.b1 = 0.0f;
    if constexpr (FMT == SLHIP_FMT_Q8_0) {  // {f16 d; i8 q[32]}: the signed codes, b = 0
        const int o = b * 34;
        r.a0 = r.a1 = half_at(s, o);
#pragma unroll
        for (int k = 0; k < 8; k++) r.c[k] = lds_u32(s, o + 2 + 4 * k);
    } else if constexpr (FMT == SLHIP_FMT_Q4_0 || FMT == SLHIP_FMT_Q4_1 || FMT == SLHIP_FMT_IQ4_NL ||
                         FMT == SLHIP_FMT_Q5_0 || FMT == SLHIP_FMT_Q5_1) {
        using F = Fmt<FMT>;
        const int o = b * F::BB;
        const float d = half_at(s, o);
        r.a0 = r.a1 = d;
        if constexpr (FMT != SLHIP_FMT_IQ4_NL)
            r.b0 = r.b1 = F::M ? half_at(s, o + 2) : static_cast<float>(F::OFF) * d;
        uint32_t qh = 0;
        if constexpr (F::QH >= 0) qh = lds_u32(s, o + F::QH);
#pragma unroll
        for (int k = 0; k < 4; k++) {  // value 4k + e: low nibble of byte 4k + e; value 16 + 4k + e: high nibble
            const uint32_t w = lds_u32(s, o + F::QS + 4 * k);
            uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
            if constexpr (F::QH >= 0) {  // bit k of qh to bit 4 of byte k: four bits spread to four bytes
                lo |= ((((qh >> (4 * k)) & 0xFu) * 0x00204081u) & 0x01010101u) << 4;
                hi |= ((((qh >> (16 + 4 * k)) & 0xFu) * 0x00204081u) & 0x01010101u) << 4;
            }
            if constexpr (FMT == SLHIP_FMT_IQ4_NL) {
                lo = iq4_lookup4(lo);
                hi = iq4_lookup4(hi);
            }
            r.c[k] = lo;
            r.c[4 + k] = hi;
        }
    } else if constexpr (FMT == SLHIP_FMT_MXFP4) {  // {u8 e; u8 qs[16]}: the doubled E2M1 values, halved scale
        const int o = b * 17;
        r.a0 = r.a1 = e8m0_half(B.u8(o));
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const uint32_t w = lds_u32(s, o + 1 + 4 * k);
            r.c[k] = fp4_lookup4(w & 0x0F0F0F0Fu);
            r.c[4 + k] = fp4_lookup4((w >> 4) & 0x0F0F0F0Fu);
        }
    } else if constexpr (FMT == SLHIP_FMT_Q4_K || FMT == SLHIP_FMT_Q5_K) {
        // {f16 d, f16 dmin, u8 scales[12], [u8 qh[32]], u8 qs[128]}: sub-block j = nibble j & 1 of qs[32 (j / 2) ..]
        constexpr bool K5 = FMT == SLHIP_FMT_Q5_K;
        const int sb = b >> 3, j = b & 7;
        const int o = sb * (K5 ? 176 : 144);  // 16-byte aligned
        uint32_t sc, mn;
        if (j < 4) {
            sc = B.u8(o + 4 + j) & 63u;
            mn = B.u8(o + 8 + j) & 63u;
        } else {
            sc = (B.u8(o + 8 + j) & 0xFu) | ((B.u8(o + j) >> 6) << 4);
            mn = (B.u8(o + 8 + j) >> 4) | ((B.u8(o + 4 + j) >> 6) << 4);
        }
        r.a0 = r.a1 = __fmul_rn(half_at(s, o), static_cast<float>(sc));
        r.b0 = r.b1 = -__fmul_rn(half_at(s, o + 2), static_cast<float>(mn));
        const uint32_t* q = s + (o + (K5 ? 48 : 16) + 32 * (j >> 1)) / 4;
        const uint32_t* qh = s + (o + 16) / 4;
#pragma unroll
        for (int k = 0; k < 8; k++) {
            uint32_t w = (q[k] >> (4 * (j & 1))) & 0x0F0F0F0Fu;
            if (K5) w |= ((qh[k] >> j) & 0x01010101u) << 4;
            r.c[k] = w;
        }
    } else if constexpr (FMT == SLHIP_FMT_Q6_K) {
        // {ql[128], qh[64], i8 scales[16], f16 d} (2-byte aligned): quarter qt of half n is the nibble qt / 2 of
        // ql[64 n + 32 (qt & 1) ..] with bits 2 qt of qh[32 n ..]; codes 0..63, a = d sc, b = -32 a per 16 values
        const int sb = b >> 3, j = b & 7, n = j >> 2, qt = j & 3;
        const int o = sb * 210;
        const float d = half_at(s, o + 208);
        r.a0 = __fmul_rn(d, static_cast<float>(static_cast<int8_t>(B.u8(o + 192 + 8 * n + 2 * qt))));
        r.a1 = __fmul_rn(d, static_cast<float>(static_cast<int8_t>(B.u8(o + 193 + 8 * n + 2 * qt))));
        r.b0 = -32.0f * r.a0;
        r.b1 = -32.0f * r.a1;
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const uint32_t l = lds_u32(s, o + 64 * n + 32 * (qt & 1) + 4 * k);
            const uint32_t h = lds_u32(s, o + 128 + 32 * n + 4 * k);
            r.c[k] = ((qt >= 2 ? l >> 4 : l) & 0x0F0F0F0Fu) | (((h >> (2 * qt)) & 0x03030303u) << 4);
        }
    } else {  // IQ4_XS {f16 d, u16 scales_h, u8 scales_l[4], u8 qs[128]}: sub-block ib, d (ls - 32), codebook
        const int sb = b >> 3, ib = b & 7;
        const int o = sb * 136;  // 8-byte aligned
        const uint32_t sh = lds_u16(s, o + 2);
        const int ls = static_cast<int>(((B.u8(o + 4 + ib / 2) >> (4 * (ib & 1))) & 0xFu) | (((sh >> (2 * ib)) & 3u) << 4));
        r.a0 = r.a1 = __fmul_rn(half_at(s, o), static_cast<float>(ls - 32));
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const uint32_t w = lds_u32(s, o + 8 + 16 * ib + 4 * k);
            r.c[k] = iq4_lookup4(w & 0x0F0F0F0Fu);
            r.c[4 + k] = iq4_lookup4((w >> 4) & 0x0F0F0F0Fu);
        }
    }
    return r;
}

// A unit's share for one token from its quantized activation values (two 16-byte vectors) and block scales.
template <int FMT>
__device__ __forceinline__ float unit_dot(const I8Unit& u, const uint4& x0, const uint4& x1, const float4& sc)
{
    int s0 = __builtin_amdgcn_sdot4(static_cast<int>(u.c[0]), static_cast<int>(x0.x), 0, false);
    s0 = __builtin_amdgcn_sdot4(static_cast<int>(u.c[1]), static_cast<int>(x0.y), s0, false);
    s0 = __builtin_amdgcn_sdot4(static_cast<int>(u.c[2]), static_cast<int>(x0.z), s0, false);
    s0 = __builtin_amdgcn_sdot4(static_cast<int>(u.c[3]), static_cast<int>(x0.w), s0, false);
    constexpr int form = kUnitForm<FMT>;
    if constexpr (form == kScale16Off) {
        int s1 = __builtin_amdgcn_sdot4(static_cast<int>(u.c[4]), static_cast<int>(x1.x), 0, false);
        s1 = __builtin_amdgcn_sdot4(static_cast<int>(u.c[5]), static_cast<int>(x1.y), s1, false);
        s1 = __builtin_amdgcn_sdot4(static_cast<int>(u.c[6]), static_cast<int>(x1.z), s1, false);
        s1 = __builtin_amdgcn_sdot4(static_cast<int>(u.c[7]), static_cast<int>(x1.w), s1, false);
        return fmaf(u.a0, __fmul_rn(sc.x, static_cast<float>(s0)),
                    fmaf(u.a1, __fmul_rn(sc.x, static_cast<float>(s1)), fmaf(u.b0, sc.y, __fmul_rn(u.b1, sc.z))));
    } else {
        int s = __builtin_amdgcn_sdot4(static_cast<int>(u.c[4]), static_cast<int>(x1.x), s0, false);
        s = __builtin_amdgcn_sdot4(static_cast<int>(u.c[5]), static_cast<int>(x1.y), s, false);
        s = __builtin_amdgcn_sdot4(static_cast<int>(u.c[6]), static_cast<int>(x1.z), s, false);
        s = __builtin_amdgcn_sdot4(static_cast<int>(u.c[7]), static_cast<int>(x1.w), s, false);
        const float p = __fmul_rn(u.a0, __fmul_rn(sc.x, static_cast<float>(s)));
        if constexpr (form == kScale32Off) return fmaf(u.b0, sc.y + sc.z, p);
        else return p;
    }
}

#include "matvec_i8_reg.hpp"

// ---- several tokens on the integer matrix cores ----------------------------------------------------------
//
// v_mfma_i32_16x16x32_i8 multiplies 16 tokens' q8 values of one 32-value unit (A: lane l holds token l % 16,
// values 8 (l / 16) .. + 7) with a 16-row tile's codes of the unit (B: lane l holds row l % 16, the same values)
// into exact int32 sums (lane l: tokens 4 (l / 16) + i, row l % 16, so each lane decodes its own row's
// multiplier and offset once per unit), so each unit's sums for 16 rows x 16 tokens take one
// instruction and the scaling a (d s) + b gs per output runs on the VALU. Q6_K's two 16-value scale groups take
// two instructions, each with the other half's codes masked to zero. A block of 8 waves takes TN tiles (gate/up
// pairs of tiles: TN = 1 or 2 by format); stages of SU units (512 or 1024 values) of the tiles' rows go through
// LDS, double- or triple-buffered: the next stage's (or the next two stages') rows and q8 scales move from HBM
// straight into LDS (global_load_lds, no registers) while the current one is computed; each wave takes SU / 8 units of a stage for every tile; the
// waves' partial sums meet in LDS at the end.

// Bytes of one row per 1024 values, the width of the staging loads, the 32-value units per stage and 16-row
// tiles per block (SU, TN), and whether the multipliers go through a per-wave table (below). Measured on
// [14336, 4096] pairs at 16 tokens (µs): one tile of 1024-value stages is where the kernel started; Q8_0's large
// rows take 512-value stages (51.8 -> 44); two tiles of 512-value stages per block (448 blocks: every tile in
// one round of two blocks per CU, and each x load and q8 scale shared by two tiles) for Q4_0 / Q4_1 / Q5_0 /
// Q5_1 / IQ4_NL / MXFP4 / Q4_K / IQ4_XS: 35.6 / 35.1 / 38.6 / 38.8 / 36.3 / 37.7 / 38.8 / 40.3 -> 29.4 / 28.2 /
// 35.1 / 32.6 / 29.6 / 31.8 / 31.7 / 33.5. Q5_K and Q6_K measured level or slower with two (their decode
// state: 135 registers), and two Q8_0 tiles would hold one block per CU. NB: stage buffers; three (loads two
// stages ahead) for Q8_0 only: 44.0 -> 39.9; the others measured level or slower with three (LDS then holds one
// block per CU for Q4_1 / Q5_1 / Q5_K / Q6_K, and Q4_0 / Q4_K need more registers than two blocks leave).
template <int FMT> struct I8Stage;
template <> struct I8Stage<SLHIP_FMT_Q8_0> { static constexpr int RB = 32 * 34, UB = 16, SU = 16, TN = 1, NB = 3; static constexpr bool TABLE = false; };
template <> struct I8Stage<SLHIP_FMT_Q4_0> { static constexpr int RB = 32 * 18, UB = 16, SU = 16, TN = 2, NB = 2; static constexpr bool TABLE = false; };
template <> struct I8Stage<SLHIP_FMT_Q4_1> { static constexpr int RB = 32 * 20, UB = 16, SU = 16, TN = 2, NB = 2; static constexpr bool TABLE = false; };
template <> struct I8Stage<SLHIP_FMT_Q5_0> { static constexpr int RB = 32 * 22, UB = 16, SU = 16, TN = 2, NB = 2; static constexpr bool TABLE = false; };
template <> struct I8Stage<SLHIP_FMT_Q5_1> { static constexpr int RB = 32 * 24, UB = 16, SU = 16, TN = 2, NB = 2; static constexpr bool TABLE = false; };
template <> struct I8Stage<SLHIP_FMT_IQ4_NL> { static constexpr int RB = 32 * 18, UB = 16, SU = 16, TN = 2, NB = 2; static constexpr bool TABLE = false; };
template <> struct I8Stage<SLHIP_FMT_MXFP4> { static constexpr int RB = 32 * 17, UB = 16, SU = 16, TN = 2, NB = 2; static constexpr bool TABLE = false; };
template <> struct I8Stage<SLHIP_FMT_Q4_K> { static constexpr int RB = 4 * 144, UB = 16, SU = 16, TN = 2, NB = 2; static constexpr bool TABLE = true; };
template <> struct I8Stage<SLHIP_FMT_Q5_K> { static constexpr int RB = 4 * 176, UB = 16, SU = 32, TN = 1, NB = 2; static constexpr bool TABLE = true; };
template <> struct I8Stage<SLHIP_FMT_Q6_K> { static constexpr int RB = 4 * 210, UB = 4, SU = 32, TN = 1, NB = 2; static constexpr bool TABLE = false; };
template <> struct I8Stage<SLHIP_FMT_IQ4_XS> { static constexpr int RB = 4 * 136, UB = 16, SU = 16, TN = 2, NB = 2; static constexpr bool TABLE = true; };

constexpr int kI8MfWaves = 8;

// The 8 codes of values 8 g .. 8 g + 7 of unit b of a row image (the bytes i8_unit's c[2 g], c[2 g + 1] hold).
template <int FMT>
__device__ __forceinline__ uint2 i8_codes8(const uint32_t* s, int b, int g)
{
    const LdsBytes B{s};
    if constexpr (FMT == SLHIP_FMT_Q8_0) {
        return lds_u64(s, b * 34 + 2 + 8 * g);
    } else if constexpr (FMT == SLHIP_FMT_Q4_0 || FMT == SLHIP_FMT_Q4_1 || FMT == SLHIP_FMT_IQ4_NL ||
                         FMT == SLHIP_FMT_Q5_0 || FMT == SLHIP_FMT_Q5_1 || FMT == SLHIP_FMT_MXFP4) {
        constexpr int BB = FMT == SLHIP_FMT_MXFP4 ? 17 : Fmt<FMT>::BB;
        constexpr int QS = FMT == SLHIP_FMT_MXFP4 ? 1 : Fmt<FMT>::QS;
        const int o = b * BB;
        const uint2 w = lds_u64(s, o + QS + 8 * (g & 1));
        const uint32_t sh = g >= 2 ? 4u : 0u;
        uint32_t lo = (w.x >> sh) & 0x0F0F0F0Fu, hi = (w.y >> sh) & 0x0F0F0F0Fu;
        if constexpr (FMT == SLHIP_FMT_Q5_0 || FMT == SLHIP_FMT_Q5_1) {  // bit v of qh for value v
            const uint32_t qh = lds_u32(s, o + Fmt<FMT>::QH) >> (8 * g);
            lo |= ((((qh & 0xFu) * 0x00204081u) & 0x01010101u) << 4);
            hi |= (((((qh >> 4) & 0xFu) * 0x00204081u) & 0x01010101u) << 4);
        }
        if constexpr (FMT == SLHIP_FMT_IQ4_NL) {
            lo = iq4_lookup4(lo);
            hi = iq4_lookup4(hi);
        }
        if constexpr (FMT == SLHIP_FMT_MXFP4) {
            lo = fp4_lookup4(lo);
            hi = fp4_lookup4(hi);
        }
        return make_uint2(lo, hi);
    } else if constexpr (FMT == SLHIP_FMT_Q4_K || FMT == SLHIP_FMT_Q5_K) {
        constexpr bool K5 = FMT == SLHIP_FMT_Q5_K;
        const int sb = b >> 3, j = b & 7;
        const int o = sb * (K5 ? 176 : 144);
        const uint32_t* q = s + (o + (K5 ? 48 : 16) + 32 * (j >> 1) + 8 * g) / 4;
        uint32_t lo = (q[0] >> (4 * (j & 1))) & 0x0F0F0F0Fu, hi = (q[1] >> (4 * (j & 1))) & 0x0F0F0F0Fu;
        if constexpr (K5) {
            const uint32_t* qh = s + (o + 16 + 8 * g) / 4;
            lo |= ((qh[0] >> j) & 0x01010101u) << 4;
            hi |= ((qh[1] >> j) & 0x01010101u) << 4;
        }
        return make_uint2(lo, hi);
    } else if constexpr (FMT == SLHIP_FMT_Q6_K) {
        const int sb = b >> 3, j = b & 7, n = j >> 2, qt = j & 3;
        const int o = sb * 210;
        const uint2 l = lds_u64(s, o + 64 * n + 32 * (qt & 1) + 8 * g);
        const uint2 h = lds_u64(s, o + 128 + 32 * n + 8 * g);
        const uint32_t ls = qt >= 2 ? 4u : 0u, hs = 2u * static_cast<uint32_t>(qt);
        return make_uint2(((l.x >> ls) & 0x0F0F0F0Fu) | (((h.x >> hs) & 0x03030303u) << 4),
                          ((l.y >> ls) & 0x0F0F0F0Fu) | (((h.y >> hs) & 0x03030303u) << 4));
    } else {  // IQ4_XS
        const int sb = b >> 3, ib = b & 7;
        const uint2 w = lds_u64(s, sb * 136 + 8 + 16 * ib + 8 * (g & 1));
        const uint32_t sh = g >= 2 ? 4u : 0u;
        return make_uint2(iq4_lookup4((w.x >> sh) & 0x0F0F0F0Fu), iq4_lookup4((w.y >> sh) & 0x0F0F0F0Fu));
    }
    (void)B;
}

// The multipliers and offsets of unit b of a row image (i8_unit's scales without the codes).
template <int FMT>
__device__ __forceinline__ float4 i8_scales(const uint32_t* s, int b)
{
    const LdsBytes B{s};
    if constexpr (FMT == SLHIP_FMT_Q8_0) {
        const float d = half_at(s, b * 34);
        return make_float4(d, d, 0.0f, 0.0f);
    } else if constexpr (FMT == SLHIP_FMT_Q4_0 || FMT == SLHIP_FMT_Q4_1 || FMT == SLHIP_FMT_IQ4_NL ||
                         FMT == SLHIP_FMT_Q5_0 || FMT == SLHIP_FMT_Q5_1) {
        using F = Fmt<FMT>;
        const int o = b * F::BB;
        const float d = half_at(s, o);
        const float off = FMT == SLHIP_FMT_IQ4_NL ? 0.0f : F::M ? half_at(s, o + 2) : static_cast<float>(F::OFF) * d;
        return make_float4(d, d, off, off);
    } else if constexpr (FMT == SLHIP_FMT_MXFP4) {
        const float d = e8m0_half(B.u8(b * 17));
        return make_float4(d, d, 0.0f, 0.0f);
    } else if constexpr (FMT == SLHIP_FMT_Q4_K || FMT == SLHIP_FMT_Q5_K) {
        const int sb = b >> 3, j = b & 7;
        const int o = sb * (FMT == SLHIP_FMT_Q5_K ? 176 : 144);
        uint32_t sc, mn;
        if (j < 4) {
            sc = B.u8(o + 4 + j) & 63u;
            mn = B.u8(o + 8 + j) & 63u;
        } else {
            sc = (B.u8(o + 8 + j) & 0xFu) | ((B.u8(o + j) >> 6) << 4);
            mn = (B.u8(o + 8 + j) >> 4) | ((B.u8(o + 4 + j) >> 6) << 4);
        }
        const float a = __fmul_rn(half_at(s, o), static_cast<float>(sc));
        const float m = -__fmul_rn(half_at(s, o + 2), static_cast<float>(mn));
        return make_float4(a, a, m, m);
    } else if constexpr (FMT == SLHIP_FMT_Q6_K) {
        const int sb = b >> 3, j = b & 7, n = j >> 2, qt = j & 3;
        const int o = sb * 210;
        const float d = half_at(s, o + 208);
        const float a0 = __fmul_rn(d, static_cast<float>(static_cast<int8_t>(B.u8(o + 192 + 8 * n + 2 * qt))));
        const float a1 = __fmul_rn(d, static_cast<float>(static_cast<int8_t>(B.u8(o + 193 + 8 * n + 2 * qt))));
        return make_float4(a0, a1, -32.0f * a0, -32.0f * a1);
    } else {
        const int sb = b >> 3, ib = b & 7;
        const int o = sb * 136;
        const uint32_t sh = lds_u16(s, o + 2);
        const int ls = static_cast<int>(((B.u8(o + 4 + ib / 2) >> (4 * (ib & 1))) & 0xFu) | (((sh >> (2 * ib)) & 3u) << 4));
        const float a = __fmul_rn(half_at(s, o), static_cast<float>(ls - 32));
        return make_float4(a, a, 0.0f, 0.0f);
    }
}

// The multiplier and offset (a, b) of unit 4 h + j (j < 4) of a super-block from its first 16 bytes held in
// registers (Q4_K / Q5_K: d, dmin, the 12 packed 6-bit scale and min bytes; IQ4_XS: d, scales_h, scales_l),
// the same arithmetic as i8_scales on the LDS image.
template <int FMT>
__device__ __forceinline__ float2 hdr_scales(const uint4& q, int h, int j)
{
    auto byte = [](uint32_t w, int k) { return (w >> (8 * k)) & 0xFFu; };
    const float d = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(q.x & 0xFFFFu)));
    if constexpr (FMT == SLHIP_FMT_Q4_K || FMT == SLHIP_FMT_Q5_K) {
        const float dmin = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(q.x >> 16)));
        uint32_t sc, mn;
        if (h == 0) {  // units 0..3: bytes 4 + j and 8 + j, low 6 bits
            sc = byte(q.y, j) & 63u;
            mn = byte(q.z, j) & 63u;
        } else {  // units 4..7: low nibbles of bytes 12 + j with the top bits of bytes j + 4, j + 8 (units 0..3's)
            sc = (byte(q.w, j) & 0xFu) | ((byte(q.y, j) >> 6) << 4);
            mn = (byte(q.w, j) >> 4) | ((byte(q.z, j) >> 6) << 4);
        }
        return make_float2(__fmul_rn(d, static_cast<float>(sc)), -__fmul_rn(dmin, static_cast<float>(mn)));
    } else {  // IQ4_XS: ib = 4 h + j; ls = 4 bits of scales_l[ib / 2] | 2 bits of scales_h << 4
        const int ib = 4 * h + j;
        const uint32_t sh = q.x >> 16;
        const uint32_t lo = (byte(q.y, ib >> 1) >> (4 * (ib & 1))) & 0xFu;
        const int ls = static_cast<int>(lo | (((sh >> (2 * ib)) & 3u) << 4));
        return make_float2(__fmul_rn(d, static_cast<float>(ls - 32)), 0.0f);
    }
}


typedef int i32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));


// s_waitcnt vmcnt(n) (n < 16; expcnt and lgkmcnt left at their maxima); n from a wave-uniform value
__device__ __forceinline__ void wait_vm_le(int n)
{
    switch (n < 15 ? n : 15) {
#define SLHIP_VM_CASE(k) \
    case k: __builtin_amdgcn_s_waitcnt(0x0F70 | k); break;
        SLHIP_VM_CASE(0) SLHIP_VM_CASE(1) SLHIP_VM_CASE(2) SLHIP_VM_CASE(3) SLHIP_VM_CASE(4) SLHIP_VM_CASE(5)
        SLHIP_VM_CASE(6) SLHIP_VM_CASE(7) SLHIP_VM_CASE(8) SLHIP_VM_CASE(9) SLHIP_VM_CASE(10) SLHIP_VM_CASE(11)
        SLHIP_VM_CASE(12) SLHIP_VM_CASE(13) SLHIP_VM_CASE(14) SLHIP_VM_CASE(15)
#undef SLHIP_VM_CASE
    }
}

// Global loads into registers written as inline assembly: the compiler neither counts them nor waits for them,
// so the caller's explicit vmcnt waits must cover every read of the result (the three-buffer pipeline below,
// whose counted waits would otherwise be forced down to vmcnt(0) by the compiler's own wait for these).
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint2 ld_async_u2(const void* p)
{
    u32x2_t r;
    asm volatile("global_load_dwordx2 %0, %1, off" : "=v"(r) : "v"(p) : "memory");
    return make_uint2(r.x, r.y);
}
__device__ __forceinline__ uint4 ld_async_u4(const void* p)
{
    u32x4_t r;
    asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(r) : "v"(p) : "memory");
    return make_uint4(r.x, r.y, r.z, r.w);
}

// NB stage buffers: 2 (the next stage loads while the current one is computed) or 3 (the stage after next
// loads too: twice the bytes in flight per block, at 1.5x the LDS)
template <int FMT, bool DUAL, int SU, int TN, int NB>
__global__ __launch_bounds__(64 * kI8MfWaves) __attribute__((amdgpu_waves_per_eu(SU == 16 && TN == 1 ? 6 : NB == 3 || TN == 2 ? 4 : 1))) void matvec_i8_mfma(I8Args a)
{
    constexpr int NM = DUAL ? 2 : 1;
    constexpr int G = NM * TN;  // row groups of 16 rows: group q = tile q / NM of matrix q % NM
    constexpr int RB = I8Stage<FMT>::RB * SU / 32, UB = I8Stage<FMT>::UB;  // SU 32-value units per stage
    constexpr int PITCH = stage_pitch(RB, UB, NB == 3);
    constexpr int SPR = PITCH / UB;  // load slots per staged row; those past RB / UB are padding
    constexpr int MS = (16 * SPR + 63) / 64 * 64;  // slots per matrix: whole waves, so a wave's run is in one
    constexpr int SLOTS = G * MS;
    constexpr int SW = SLOTS * UB / 4;  // words per stage buffer
    constexpr int NT = 64 * kI8MfWaves;
    constexpr int LPT = (SLOTS + NT - 1) / NT;  // loads per thread and stage
    constexpr int BPW = SU / kI8MfWaves;  // units per wave and stage
    constexpr bool H16 = kUnitForm<FMT> == kScale16Off;
    static_assert(RB % UB == 0 && (UB == 16 || UB == 4), "stage shape");
    static_assert(NT >= 16 * SU && (SU == 16 || SU == 32), "one thread per token and unit of a stage stages the q8 scales");
    static_assert(NB * SLOTS * UB >= static_cast<int>(sizeof(float)) * kI8MfWaves * G * 4 * 64,
                  "the cross-wave reduction reuses the weight stage");
    static_assert(NB == 2 || NB == 3, "stage buffers");
    // [buffer][matrix: 16 rows of PITCH bytes, padding], then the q8 scales {d, d s_lo, d s_hi, 0} of
    // [buffer][unit][token] (the 4 tokens a lane group reads at once are 64 bytes apart: different banks; the
    // reads past the last staged row land there)
    __shared__ __align__(16) uint32_t stage_mem[NB * SW + NB * SU * 16 * 4];
    float4* const xsc = reinterpret_cast<float4*>(&stage_mem[NB * SW]);
    auto rowp = [&](int b, int m, int rr) -> const uint32_t* { return &stage_mem[b * SW + (m * MS * UB + rr * PITCH) / 4]; };
    const int lane = threadIdx.x & 63;
    const int wave = wave_id();
    const int r = lane & 15, g = lane >> 4;
    const int64_t n0 = static_cast<int64_t>(blockIdx.x) * 16 * TN;
    const int K = static_cast<int>(a.K);
    const int ns = K / (32 * SU);
    const int64_t xstride = K + K / 2;
    int64_t tok = a.t0 + r;
    tok = tok < a.T ? tok : a.T - 1;
    const uint8_t* xrow = a.xq + tok * xstride;
    // the scale this thread stages: token threadIdx % 16 of the pass, unit threadIdx / 16 of each stage
    int64_t stok = a.t0 + (threadIdx.x & 15);
    stok = stok < a.T ? stok : a.T - 1;
    // (offset from the pass's first q8 row: 16 rows, below 2^31 bytes)
    const uint8_t* xs_base = a.xq + a.t0 * xstride + K;
    const uint32_t xs_off = static_cast<uint32_t>((stok - a.t0) * xstride + 16 * (threadIdx.x >> 4));

    // Load slot q = threadIdx + NT i is byte UB q of the stage: matrix q / MS, row rr, slot c of SPR; a padding
    // slot (the row's last 16 bytes, or the matrix's tail) loads a real piece again (the LDS image is
    // contiguous, so the lanes of a wave fill one run, and a wave's run lies in one matrix). src: the byte
    // offset from the matrix start (below 2^31), so that the address is a scalar base plus one register.
    uint32_t src[LPT];
#pragma unroll
    for (int i = 0; i < LPT; i++) {
        int q = static_cast<int>(threadIdx.x) + NT * i;
        q = q < SLOTS ? q : SLOTS - 1;
        const int m = q / MS, rem = q - m * MS;
        int rr = rem / SPR, c = rem - rr * SPR;
        if (rr > 15) {
            rr = 15;
            c = 0;
        }
        c = c < RB / UB ? c : RB / UB - 1;
        int64_t row = n0 + 16 * (m / NM) + rr;
        row = row < a.N ? row : a.N - 1;
        src[i] = static_cast<uint32_t>(row * a.wrow + UB * c);
    }
    auto fetch = [&](int b, int s) {
#pragma unroll
        for (int i = 0; i < LPT; i++) {
            if (NT * i + 64 * wave >= SLOTS) break;  // wave-uniform: the LDS run of a wave starts in the stage
            if (NT * (i + 1) > SLOTS && static_cast<int>(threadIdx.x) + NT * i >= SLOTS) continue;
            char* base = reinterpret_cast<char*>(&stage_mem[b * SW]) + UB * (NT * i + 64 * wave);
            const char* mat = (((NT * i + 64 * wave) / MS) % NM ? a.wu : a.wg) + static_cast<int64_t>(s) * RB;
            load_to_lds<UB>(mat, src[i], base);
        }
        if (64 * wave < 16 * SU) {  // wave-uniform; the base made visibly uniform for the scalar operand
            const uint64_t xb = reinterpret_cast<uint64_t>(xs_base + static_cast<int64_t>(s) * (16 * SU));
            // (readfirstlane returns int: each half goes through uint32_t, or the low half would sign-extend)
            const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(xb)));
            const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(xb >> 32)));
            const uint64_t xbu = (static_cast<uint64_t>(hi) << 32) | lo;
            load_to_lds<16>(reinterpret_cast<const void*>(xbu), xs_off, xsc + b * SU * 16 + 64 * wave);
        }
    };
    constexpr bool TABLE = I8Stage<FMT>::TABLE;
    constexpr int SBB = FMT == SLHIP_FMT_Q4_K ? 144 : FMT == SLHIP_FMT_Q5_K ? 176 : 136;  // super-block bytes
    // (TABLE formats) the super-block header of the wave's units for row lane % (16 NM): its first 16 bytes,
    // loaded from HBM with the stage (the same lines the stage moves into LDS)
    const char* hdr_src = nullptr;
    if constexpr (TABLE) {
        const int rr = lane % (G * 16), grp = rr / 16;
        int64_t row = n0 + 16 * (grp / NM) + rr % 16;
        row = row < a.N ? row : a.N - 1;
        hdr_src = (grp % NM ? a.wu : a.wg) + row * a.wrow + (wave * BPW / 8) * SBB;
    }
    struct Xs {
        uint2 q[BPW];
        uint4 hdr;
    };
    auto fetch_x = [&](Xs& x, int s) {
        if constexpr (NB == 3) {
#pragma unroll
            for (int j = 0; j < BPW; j++) x.q[j] = ld_async_u2(xrow + (s * SU + wave * BPW + j) * 32 + 8 * g);
            // (IQ4_XS: only the 8 header bytes it decodes; a register the load writes but the code never reads
            // would be free for the compiler to reuse while the load is still in flight)
            if constexpr (TABLE && FMT == SLHIP_FMT_IQ4_XS) {
                const uint2 h = ld_async_u2(hdr_src + static_cast<int64_t>(s) * (SU / 8) * SBB);
                x.hdr = make_uint4(h.x, h.y, 0u, 0u);
            } else if constexpr (TABLE) {
                x.hdr = ld_async_u4(hdr_src + static_cast<int64_t>(s) * (SU / 8) * SBB);
            }
        } else {
#pragma unroll
            for (int j = 0; j < BPW; j++) x.q[j] = *reinterpret_cast<const uint2*>(xrow + (s * SU + wave * BPW + j) * 32 + 8 * g);
            if constexpr (TABLE) x.hdr = *reinterpret_cast<const uint4*>(hdr_src + static_cast<int64_t>(s) * (SU / 8) * SBB);
        }
    };
    // acc[m][i]: weight row n0 + r of matrix m, token t0 + 4 g + i (the MFMA's A operand is the q8 tokens, B the
    // weight codes, so each lane decodes the multipliers of its own row once per unit)
    float acc[G][4];
#pragma unroll
    for (int m = 0; m < G; m++)
        for (int i = 0; i < 4; i++) acc[m][i] = 0.0f;
    constexpr bool OFF = kUnitForm<FMT> == kScale32Off;  // formats with one offset per unit
    f32x4_t acc_off[G];
#pragma unroll
    for (int m = 0; m < G; m++) acc_off[m] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    // The K-quants' and IQ4_XS's multipliers and offsets (6-bit fields spread over the super-block header) for
    // the wave's units and the tile's rows are decoded once each, by the lane holding the row's header, into
    // the wave's own LDS table, and read there by the 4 lanes of a row; the other formats' (one f16 or e8m0
    // field) are read from the stage directly.
    constexpr int NENT = G * 16 * BPW;
    static_assert(8 % BPW == 0, "a wave's units lie in one super-block");
    __shared__ __align__(16) float2 wsc[TABLE ? kI8MfWaves : 1][TABLE ? NENT : 1];
    float2* my = wsc[TABLE ? wave : 0];
    auto compute = [&](int b, const Xs& x) {
        if constexpr (TABLE) {
            static_assert(!H16, "the table holds one multiplier and offset per unit");
            if (lane < G * 16) {
#pragma unroll
                for (int j = 0; j < BPW; j++) {
                    const int u8 = (wave * BPW + j) & 7;  // the unit's place in its super-block
                    my[j * G * 16 + lane] = hdr_scales<FMT>(x.hdr, u8 >> 2, u8 & 3);
                }
            }
            wave_lds_sync();
        }
        // The offset terms b gs of the wave's units are a 16 x 16 x 4 product (tokens x units . units x rows):
        // one f32 matrix-core instruction per matrix, accumulated over the stages in acc_off; lane (r, g)
        // supplies token r's q8 sum of unit g and row r's offset of unit g. (Q6_K's offsets, one per 16-value
        // half, are added with its products.)
        if constexpr (OFF) {
            // (with two units per wave, lane groups 2 and 3 supply zeros for the instruction's other two)
            const int gu = g < BPW ? g : 0;
            const float4 xo = xsc[(b * SU + wave * BPW + gu) * 16 + r];
            const float xg = g < BPW ? xo.y + xo.z : 0.0f;
#pragma unroll
            for (int m = 0; m < G; m++) {
                float4 so;
                if constexpr (TABLE) {
                    const float2 s2 = my[gu * G * 16 + m * 16 + r];
                    so = make_float4(s2.x, s2.x, s2.y, s2.y);
                } else {
                    so = i8_scales<FMT>(rowp(b, m, r), wave * BPW + gu);
                }
                acc_off[m] = __builtin_amdgcn_mfma_f32_16x16x4f32(xg, so.z, acc_off[m], 0, 0, 0);
            }
        }
#pragma unroll
        for (int j = 0; j < BPW; j++) {
            const int u = wave * BPW + j;
            const long xb = static_cast<long>(__builtin_bit_cast(uint64_t, x.q[j]));
            float d[4];
#pragma unroll
            for (int i = 0; i < 4; i++) d[i] = xsc[(b * SU + u) * 16 + 4 * g + i].x;
#pragma unroll
            for (int m = 0; m < G; m++) {
                const uint2 c = i8_codes8<FMT>(rowp(b, m, r), u, g);
                float4 sc;
                if constexpr (TABLE) {
                    sc.x = my[j * G * 16 + m * 16 + r].x;
                } else {
                    sc = i8_scales<FMT>(rowp(b, m, r), u);
                }
                const i32x4_t z = {0, 0, 0, 0};
                if constexpr (H16) {
                    const bool first = g < 2;
                    const long c0 = first ? static_cast<long>(__builtin_bit_cast(uint64_t, c)) : 0;
                    const long c1 = first ? 0 : static_cast<long>(__builtin_bit_cast(uint64_t, c));
                    const i32x4_t S0 = __builtin_amdgcn_mfma_i32_16x16x32_i8(xb, c0, z, 0, 0, 0);
                    const i32x4_t S1 = __builtin_amdgcn_mfma_i32_16x16x32_i8(xb, c1, z, 0, 0, 0);
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const float4 xs = xsc[(b * SU + u) * 16 + 4 * g + i];
                        acc[m][i] += fmaf(sc.x, __fmul_rn(xs.x, static_cast<float>(S0[i])),
                                          fmaf(sc.y, __fmul_rn(xs.x, static_cast<float>(S1[i])),
                                               fmaf(sc.z, xs.y, __fmul_rn(sc.w, xs.z))));
                    }
                } else {
                    const i32x4_t S = __builtin_amdgcn_mfma_i32_16x16x32_i8(xb, static_cast<long>(__builtin_bit_cast(uint64_t, c)), z, 0, 0, 0);
#pragma unroll
                    for (int i = 0; i < 4; i++) acc[m][i] = fmaf(__fmul_rn(sc.x, d[i]), static_cast<float>(S[i]), acc[m][i]);
                }
            }
        }
    };
    // vmcnt(0): the stage's LDS writes by global_load_lds (and the q8 codes in registers) have landed
    constexpr int kWaitLoads = 0x0F70;
    if constexpr (NB == 2) {
        Xs xa, xb2;
        fetch(0, 0);
        fetch_x(xa, 0);
        __builtin_amdgcn_s_waitcnt(kWaitLoads);
        __syncthreads();
        for (int s = 0; s < ns; s += 2) {  // two stages per iteration: the code register sets alternate statically
            if (s + 1 < ns) {
                fetch(1, s + 1);
                fetch_x(xb2, s + 1);
            }
            compute(0, xa);
            __builtin_amdgcn_s_waitcnt(kWaitLoads);
            __syncthreads();
            if (s + 1 >= ns) break;
            if (s + 2 < ns) {
                fetch(0, s + 2);
                fetch_x(xa, s + 2);
            }
            compute(1, xb2);
            __builtin_amdgcn_s_waitcnt(kWaitLoads);
            __syncthreads();
        }
    } else {
        // The loads this wave issues per stage (every one a vector-memory instruction counted by vmcnt, and
        // the only ones in the loop): waiting for vmcnt <= that number after issuing stage s + 2 leaves
        // exactly stage s + 2 in flight, since loads complete in order.
        int per_stage = BPW + (TABLE ? 1 : 0) + (64 * wave < 16 * SU ? 1 : 0);
#pragma unroll
        for (int i = 0; i < LPT; i++) per_stage += NT * i + 64 * wave < SLOTS ? 1 : 0;
        per_stage = __builtin_amdgcn_readfirstlane(per_stage);
        Xs x0, x1, x2;
        // stage s in buffer and register set b = s % 3; its loads were issued two stages earlier
        auto step = [&](int s, int b, const Xs& xc, Xs& xn) {
            const bool more = s + 2 < ns;
            if (more) {
                fetch((b + 2) % 3, s + 2);
                fetch_x(xn, s + 2);
            }
            // (the buffer index taken from s at run time, so that the compiler keeps one set of LDS addresses,
            // not one per buffer)
            compute(__builtin_amdgcn_readfirstlane(s - s / 3 * 3), xc);
            wait_vm_le(more ? per_stage : 0);  // stage s + 1 has landed
            __syncthreads();
        };
        fetch(0, 0);
        fetch_x(x0, 0);
        if (ns > 1) {
            fetch(1, 1);
            fetch_x(x1, 1);
        }
        wait_vm_le(ns > 1 ? per_stage : 0);
        __syncthreads();
        for (int s = 0; s < ns; s += 3) {  // three stages per iteration: the register sets rotate statically
            step(s, 0, x0, x2);
            if (s + 1 >= ns) break;
            step(s + 1, 1, x1, x0);
            if (s + 2 >= ns) break;
            step(s + 2, 2, x2, x1);
        }
    }
    if constexpr (OFF) {
#pragma unroll
        for (int m = 0; m < G; m++)
            for (int i = 0; i < 4; i++) acc[m][i] += acc_off[m][i];
    }
    // every wave is past its last read of the stage (the loop ends on a barrier): reuse it for the reduction
    float* red = reinterpret_cast<float*>(&stage_mem[0]);  // [wave][group][i][lane]
#pragma unroll
    for (int m = 0; m < G; m++)
        for (int i = 0; i < 4; i++) red[((wave * G + m) * 4 + i) * 64 + lane] = acc[m][i];
    __syncthreads();
    if (wave < TN) {  // wave tl finishes tile tl
        const int tl = wave;
        float v[NM][4];
#pragma unroll
        for (int m = 0; m < NM; m++)
            for (int i = 0; i < 4; i++) {
                float t = 0.0f;
                for (int w = 0; w < kI8MfWaves; w++) t += red[((w * G + tl * NM + m) * 4 + i) * 64 + lane];
                v[m][i] = t;
            }
        const int64_t n = n0 + 16 * tl + r;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int64_t tt = a.t0 + 4 * g + i;
            float out = v[0][i];
            if constexpr (DUAL) {
                const float act = a.act == SLHIP_ACT_SILU        ? activate<SLHIP_ACT_SILU>(out)
                                  : a.act == SLHIP_ACT_GELU_TANH ? activate<SLHIP_ACT_GELU_TANH>(out)
                                                                 : activate<SLHIP_ACT_GELU_ERF>(out);
                out = act * v[NM - 1][i];
            }
            if (tt < a.T && n < a.N) {
                if (!DUAL && a.bias) out = out + a.bias[n];
                if (a.yt == SLHIP_F32)
                    static_cast<float*>(a.y)[tt * a.ys + n] = out;
                else
                    static_cast<uint16_t*>(a.y)[tt * a.ys + n] = static_cast<uint16_t>(f32_to_bf16_bits(out));
            }
        }
    }
}

// A row's 16-byte chunk at byte offset off, read as 16 / U loads of U bytes (rows that are not 16-byte
// multiples are only U-byte aligned); pieces past the row's end repeat its last U bytes.
template <int U>
__device__ __forceinline__ uint4 load_chunk(const char* row, int64_t off, int64_t wrow)
{
    if constexpr (U == 16) {
        return load_nt(row + off);
    } else {
        uint32_t w[4];
#pragma unroll
        for (int k = 0; k < 16 / U; k++) {
            int64_t o = off + k * U;
            o = o < wrow ? o : wrow - U;
            if constexpr (U == 8) {
                const uint2 t = *reinterpret_cast<const uint2*>(row + o);
                w[2 * k] = t.x;
                w[2 * k + 1] = t.y;
            } else if constexpr (U == 4) {
                w[k] = *reinterpret_cast<const uint32_t*>(row + o);
            } else {
                const uint32_t h = *reinterpret_cast<const uint16_t*>(row + o);
                if (k & 1) w[k / 2] |= h << 16;
                else w[k / 2] = h;
            }
        }
        return make_uint4(w[0], w[1], w[2], w[3]);
    }
}

template <int FMT, int TT, int CH, bool DUAL, int U>
__global__ __launch_bounds__(kI8Threads) void matvec_i8(I8Args a)
{
    extern __shared__ uint32_t smem[];
    constexpr int R = DUAL ? 2 : 1;
    const int lane = threadIdx.x & 63;
    const int wave = wave_id();
    const int nch = static_cast<int>((a.wrow + 15) / 16);  // 16-byte chunks per row (the last may be partial)
    const int rbw = nch * 4 + 4;                           // words per row image (+ a pad word group)
    uint32_t* rows = smem + wave * R * rbw;
    const int K = static_cast<int>(a.K);
    const int xrow = K + K / 2;
    uint8_t* xs = reinterpret_cast<uint8_t*>(smem + (kI8Threads / 64) * R * rbw);
    const int nb = K / 32;  // units per row

    // 16-byte rows: each matrix's chunks are padded to whole groups of 64, so a group of 64 chunks (one load
    // per lane) lies in one matrix and reads from a wave-uniform row base (no per-lane address arithmetic);
    // lanes past the row's end load nothing and store nothing. Other rows: one run over both rows' chunks,
    // clamped to the last one.
    const int ncp = U == 16 ? (nch + 63) / 64 * 64 : nch;
    const int tot = R * ncp;
    auto load_batch = [&](int64_t n, int base, uint4* v) {
#pragma unroll
        for (int c = 0; c < CH; c++) {
            const int g0 = base + c * 64;
            if (g0 >= tot) break;  // wave-uniform
            if constexpr (U == 16) {
                const int r = g0 >= ncp ? 1 : 0;  // wave-uniform
                const int w = g0 - r * ncp + lane;
                const char* row = (r ? a.wu : a.wg) + n * a.wrow;
                if (w < nch) v[c] = load_nt(row + static_cast<uint32_t>(w) * 16u);
            } else {
                int idx = g0 + lane;
                idx = idx < tot ? idx : tot - 1;
                const int r = idx >= nch ? 1 : 0;
                v[c] = load_chunk<U>((r ? a.wu : a.wg) + n * a.wrow, static_cast<int64_t>(idx - r * nch) * 16, a.wrow);
            }
        }
    };
    auto store_batch = [&](int base, const uint4* v) {
#pragma unroll
        for (int c = 0; c < CH; c++) {
            const int g0 = base + c * 64;
            if (g0 >= tot) break;  // wave-uniform
            if constexpr (U == 16) {
                const int r = g0 >= ncp ? 1 : 0;
                const int w = g0 - r * ncp + lane;
                if (w < nch) reinterpret_cast<uint4*>(rows + r * rbw)[w] = v[c];
            } else {
                int idx = g0 + lane;
                idx = idx < tot ? idx : tot - 1;
                const int r = idx >= nch ? 1 : 0;
                reinterpret_cast<uint4*>(rows + r * rbw)[idx - r * nch] = v[c];
            }
        }
    };
    auto rest = [&](int64_t n, uint4* v) {  // batches after the first, loaded and stored in turn
        for (int base = CH * 64; base < tot; base += CH * 64) {
            load_batch(n, base, v);
            store_batch(base, v);
        }
    };
    const int64_t stride = static_cast<int64_t>(gridDim.x) * (kI8Threads / 64);
    int64_t n = static_cast<int64_t>(blockIdx.x) * (kI8Threads / 64) + wave;
    const int64_t n_first = n < a.N ? n : a.N - 1;
    uint4 v[CH];
    load_batch(n_first, 0, v);
    __builtin_amdgcn_sched_barrier(0);  // the weight loads go out before the staging loads
    {  // the block's TT quantized rows (16-byte chunks; rows past T repeat row T - 1)
        const int per = xrow / 16;
        for (int u = threadIdx.x; u < TT * per; u += kI8Threads) {
            const int t = u / per;
            int64_t tok = a.t0 + t;
            tok = tok < a.T ? tok : a.T - 1;
            reinterpret_cast<uint4*>(xs)[u] = reinterpret_cast<const uint4*>(a.xq + tok * xrow)[u - t * per];
        }
    }
    store_batch(0, v);
    rest(n_first, v);
    __syncthreads();

    for (; n < a.N; n += stride) {  // wave-uniform
        const int64_t next = n + stride;
        const bool more = next < a.N;
        if (more) load_batch(next, 0, v);
        float ag[TT], au[TT];
#pragma unroll
        for (int t = 0; t < TT; t++) ag[t] = au[t] = 0.0f;
        auto unit = [&](int b, bool own) {
            const I8Unit ug = i8_unit<FMT>(rows, b);
            I8Unit uu{};
            if constexpr (DUAL) uu = i8_unit<FMT>(rows + rbw, b);
#pragma unroll
            for (int t = 0; t < TT; t++) {
                const uint4* xp = reinterpret_cast<const uint4*>(xs + t * xrow + 32 * b);
                const uint4 x0 = xp[0], x1 = xp[1];
                const float4 sc = reinterpret_cast<const float4*>(xs + t * xrow + K)[b];
                const float pg = unit_dot<FMT>(ug, x0, x1, sc);
                ag[t] += own ? pg : 0.0f;
                if (DUAL) {
                    const float pu = unit_dot<FMT>(uu, x0, x1, sc);
                    au[t] += own ? pu : 0.0f;
                }
            }
        };
        if (kSliceLds<FMT, TT> && K % 64 == 0) {  // wave-uniform; K-quants always, block formats with an even block count
            // a 64-value slice per lane, its bytes read from the row images as words
            const int nsl = K / 64;
            auto slice = [&](int sl, bool own) {
                I8Unit g0, g1, u0, u1;
                int j0, j1;
                slice_units<FMT>(rows, sl, g0, g1, j0, j1);
                if constexpr (DUAL) slice_units<FMT>(rows + rbw, sl, u0, u1, j0, j1);
#pragma unroll
                for (int t = 0; t < TT; t++) {
                    const uint8_t* xt = xs + t * xrow;
                    const uint4 x00 = *reinterpret_cast<const uint4*>(xt + 32 * j0);
                    const uint4 x01 = *reinterpret_cast<const uint4*>(xt + 32 * j0 + 16);
                    const uint4 x10 = *reinterpret_cast<const uint4*>(xt + 32 * j1);
                    const uint4 x11 = *reinterpret_cast<const uint4*>(xt + 32 * j1 + 16);
                    const float4 sc0 = *reinterpret_cast<const float4*>(xt + K + 16 * j0);
                    const float4 sc1 = *reinterpret_cast<const float4*>(xt + K + 16 * j1);
                    const float pg = unit_dot<FMT>(g0, x00, x01, sc0) + unit_dot<FMT>(g1, x10, x11, sc1);
                    ag[t] += own ? pg : 0.0f;
                    if constexpr (DUAL) {
                        const float pu = unit_dot<FMT>(u0, x00, x01, sc0) + unit_dot<FMT>(u1, x10, x11, sc1);
                        au[t] += own ? pu : 0.0f;
                    }
                }
            };
            const int full = nsl / 64;
            for (int i = 0; i < full; i++) slice(lane + 64 * i, true);
            if (full * 64 < nsl) {  // wave-uniform
                const int sl = lane + 64 * full;
                slice(sl < nsl ? sl : nsl - 1, sl < nsl);
            }
        } else {
            const int full = nb / 64;  // iterations in which every lane has a unit
            for (int i = 0; i < full; i++) unit(lane + 64 * i, true);
            if (full * 64 < nb) {  // wave-uniform
                const int b = lane + 64 * full;
                unit(b < nb ? b : nb - 1, b < nb);
            }
        }
#pragma unroll
        for (int t = 0; t < TT; t++) {
            float out = wave_sum(ag[t]);
            if (DUAL) {
                const float u = wave_sum(au[t]);
                const float g = out;
                const float act = a.act == SLHIP_ACT_SILU        ? activate<SLHIP_ACT_SILU>(g)
                                  : a.act == SLHIP_ACT_GELU_TANH ? activate<SLHIP_ACT_GELU_TANH>(g)
                                                                 : activate<SLHIP_ACT_GELU_ERF>(g);
                out = act * u;
            } else if (a.bias) {
                out = out + a.bias[n];
            }
            int64_t tok = a.t0 + t;
            tok = tok < a.T ? tok : a.T - 1;
            if (a.yt == SLHIP_F32)
                static_cast<float*>(a.y)[tok * a.ys + n] = out;
            else
                static_cast<uint16_t*>(a.y)[tok * a.ys + n] = static_cast<uint16_t>(f32_to_bf16_bits(out));
        }
        if (more) {
            store_batch(0, v);
            rest(next, v);
        }
    }
}

// ---- host side ---------------------------------------------------------------------------------------------

inline int device_cus_i8()
{
    static int cus = 0;
    if (!cus) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            cus <= 0)
            cus = 256;
    }
    return cus;
}

constexpr size_t kI8MaxLds = 160 * 1024;

inline size_t i8_lds(int tt, int64_t K, int64_t wrow, bool dual)
{
    const int64_t rbw = (wrow + 15) / 16 * 4 + 4;
    return static_cast<size_t>(kI8Threads / 64) * (dual ? 2 : 1) * rbw * 4 + static_cast<size_t>(tt) * (K + K / 2);
}

struct I8Geom {
    int bs, bb;
};
inline I8Geom i8_geom(int fmt)
{
    switch (fmt) {
    case SLHIP_FMT_Q8_0: return {32, 34};
    case SLHIP_FMT_Q4_0: return {32, 18};
    case SLHIP_FMT_Q4_1: return {32, 20};
    case SLHIP_FMT_Q5_0: return {32, 22};
    case SLHIP_FMT_Q5_1: return {32, 24};
    case SLHIP_FMT_IQ4_NL: return {32, 18};
    case SLHIP_FMT_MXFP4: return {32, 17};
    case SLHIP_FMT_Q4_K: return {256, 144};
    case SLHIP_FMT_Q5_K: return {256, 176};
    case SLHIP_FMT_Q6_K: return {256, 210};
    case SLHIP_FMT_IQ4_XS: return {256, 136};
    default: return {0, 0};
    }
}

template <int FMT, int TT, int CH, bool DUAL, int U>
static int launch_i8(const I8Args& a, hipStream_t st)
{
    const size_t lds = i8_lds(TT, a.K, a.wrow, DUAL);
    auto kernel = matvec_i8<FMT, TT, CH, DUAL, U>;
    if (lds > 65536) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
        if (e != hipSuccess) return fail(SLHIP_ERR_HIP, "matvec_q8: %zu bytes of LDS refused: %s", lds, hipGetErrorString(e));
    }
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, kI8Threads, lds) != hipSuccess || per_cu < 1)
        per_cu = 1;
    const int64_t blocks = (a.N + kI8Threads / 64 - 1) / (kI8Threads / 64);
    const int64_t resident = static_cast<int64_t>(device_cus_i8()) * per_cu;
    kernel<<<dim3(static_cast<unsigned>(blocks < resident ? blocks : resident)), kI8Threads, lds, st>>>(a);
    return check_launch("matvec_i8");
}

template <int FMT, int TT, bool DUAL>
static int i8_ch(const I8Args& a, hipStream_t st)
{
    // rows that are not 16-byte multiples (K not a multiple of 256 for the 32-value formats; Q6_K, IQ4_XS and
    // MXFP4 rows of 210 / 136 / 17 bytes per block): 8-byte loads where they align, else 2-byte loads
    if (a.wrow % 16 != 0)
        return a.wrow % 8 == 0 ? launch_i8<FMT, TT, 8, DUAL, 8>(a, st) : launch_i8<FMT, TT, 8, DUAL, 2>(a, st);
    return launch_i8<FMT, TT, 8, DUAL, 16>(a, st);
}

// The register-piece kernel: a persistent grid of as many waves as fit, trimmed so that every wave gets the
// same number of rows.
template <int FMT, int TT, bool DUAL, int D>
static int launch_i8_reg(const I8Args& a, hipStream_t st)
{
    const size_t lds = static_cast<size_t>(TT) * static_cast<size_t>(a.K + a.K / 2);
    auto kernel = matvec_i8_reg<FMT, TT, DUAL, D>;
    if (lds > 65536) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
        if (e != hipSuccess) return fail(SLHIP_ERR_HIP, "matvec_q8: %zu bytes of LDS refused: %s", lds, hipGetErrorString(e));
    }
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, kI8RegThreads, lds) != hipSuccess || per_cu < 1)
        per_cu = 1;
    constexpr int wpb = kI8RegThreads / 64;
    const int64_t resident = static_cast<int64_t>(device_cus_i8()) * per_cu * wpb;
    const int64_t per_wave = (a.N + resident - 1) / resident;
    const int64_t waves = (a.N + per_wave - 1) / per_wave;
    kernel<<<dim3(static_cast<unsigned>((waves + wpb - 1) / wpb)), kI8RegThreads, lds, st>>>(a);
    return check_launch("matvec_i8_reg");
}

// Whether the register-piece kernel takes T tokens: for its formats at kRegPieceMinT to four tokens with K a
// multiple of 64 (SLHIP_MATVEC_I8_REG=0 turns it off).
template <int FMT>
inline bool i8_reg_takes(const I8Args& a)
{
    static int v = -1;
    if (v == -1) {
        const char* e = getenv("SLHIP_MATVEC_I8_REG");
        v = e ? atoi(e) : 1;
    }
    return v != 0 && kRegPieceKernel<FMT> && a.T >= kRegPieceMinT<FMT> && a.T <= 4 && a.K % 64 == 0 && 4 * (a.K + a.K / 2) <= static_cast<int64_t>(kI8MaxLds);
}

template <int FMT, bool DUAL>
static int run_i8_reg(I8Args a, hipStream_t st)
{
    const int tt = a.T <= 3 ? static_cast<int>(a.T) : 4;
    for (int64_t t0 = 0; t0 < a.T; t0 += tt) {
        a.t0 = t0;
        // two register sets (one item in flight while one is computed): three measured slower
        const int r = tt == 1   ? launch_i8_reg<FMT, 1, DUAL, 2>(a, st)
                      : tt == 2 ? launch_i8_reg<FMT, 2, DUAL, 2>(a, st)
                      : tt == 3 ? launch_i8_reg<FMT, 3, DUAL, 2>(a, st)
                                : launch_i8_reg<FMT, 4, DUAL, 2>(a, st);
        if (r != SLHIP_OK) return r;
    }
    return SLHIP_OK;
}

template <int FMT, bool DUAL>
static int i8_tt(const I8Args& a, int tt, hipStream_t st)
{
    switch (tt) {
    case 1: return i8_ch<FMT, 1, DUAL>(a, st);
    case 2: return i8_ch<FMT, 2, DUAL>(a, st);
    case 3: return i8_ch<FMT, 3, DUAL>(a, st);
    case 4: return i8_ch<FMT, 4, DUAL>(a, st);
    default: return i8_ch<FMT, 8, DUAL>(a, st);
    }
}

// Tokens from which the integer-dot matvec takes the matrix cores, when K is a multiple of the stage (whole
// stages), per format: measured on MI355X, [14336, 4096] gate/up pairs, µs at T = 2 / 3 / 4 (VALU kernel ->
// matrix cores): Q8_0 29.3 / 36.9 / 39.6 -> 32.8 / 32.9 / 33.4; Q4_K 24.4 / 28.6 / 32.6 -> 25.0 / 26.2 / 26.9;
// IQ4_NL 25.7 / 29.3 / 32.3 -> 27.1 / 28.4 / 28.0; Q5_K T4 37.4 -> 34.6; MXFP4 / Q4_0 / Q4_1 T4 32.1 / 28.7 /
// 27.3 -> 31.0 / 28.1 / 26.4; Q5_0 / Q5_1 / IQ4_XS level or behind at T4 and Q6_K 37.4 -> 53.2, so those from
// 5 (where the VALU kernel takes an 8-token pass and falls 1.6-1.9x behind). SLHIP_MATVEC_I8_MFMA_MIN_T
// overrides it for every format (0 disables).
template <int FMT>
inline int i8_mfma_min_tokens()
{
    static int v = -2;
    if (v == -2) {
        const char* e = getenv("SLHIP_MATVEC_I8_MFMA_MIN_T");
        v = e ? atoi(e) : -1;
    }
    if (v != -1) return v;
    switch (FMT) {
    case SLHIP_FMT_Q8_0:
    case SLHIP_FMT_Q4_K:
    case SLHIP_FMT_IQ4_NL: return 3;
    case SLHIP_FMT_Q5_K:
    case SLHIP_FMT_MXFP4:
    case SLHIP_FMT_Q4_0:
    case SLHIP_FMT_Q4_1: return 4;
    default: return 5;
    }
}

template <int FMT>
int run_i8_mfma(I8Args a, bool dual, hipStream_t st)
{
    constexpr int SU = I8Stage<FMT>::SU, TN = I8Stage<FMT>::TN, NB = I8Stage<FMT>::NB;
    const dim3 gridt(static_cast<unsigned>((a.N + 16 * TN - 1) / (16 * TN)));
    for (int64_t t0 = 0; t0 < a.T; t0 += 16) {
        a.t0 = t0;
        if (dual) matvec_i8_mfma<FMT, true, SU, TN, NB><<<gridt, 64 * kI8MfWaves, 0, st>>>(a);
        else matvec_i8_mfma<FMT, false, SU, TN, NB><<<gridt, 64 * kI8MfWaves, 0, st>>>(a);
        const int r = check_launch("matvec_i8_mfma");
        if (r != SLHIP_OK) return r;
    }
    return SLHIP_OK;
}

template <int FMT>
int run_i8(I8Args a, bool dual, hipStream_t st)
{
    const int mt = i8_mfma_min_tokens<FMT>();
    if (mt > 0 && a.T >= mt && a.K % (32 * I8Stage<FMT>::SU) == 0 && a.wrow % I8Stage<FMT>::UB == 0 && a.N * a.wrow < (int64_t{1} << 31))
        return run_i8_mfma<FMT>(a, dual, st);
    if constexpr (kRegPieceKernel<FMT>)
        if (i8_reg_takes<FMT>(a)) return dual ? run_i8_reg<FMT, true>(a, st) : run_i8_reg<FMT, false>(a, st);
    int tt = 8;
    while (tt > 1 && (tt / 2 >= a.T || i8_lds(tt, a.K, a.wrow, dual) > kI8MaxLds)) tt /= 2;
    if (a.T == 3 && tt == 4) tt = 3;  // three tokens: no idle fourth row in the pass
    if (i8_lds(tt, a.K, a.wrow, dual) > kI8MaxLds)
        return fail(SLHIP_ERR_UNSUPPORTED, "matvec_q8: K = %lld does not fit in LDS for this format", static_cast<long long>(a.K));
    for (int64_t t0 = 0; t0 < a.T; t0 += tt) {
        a.t0 = t0;
        const int r = dual ? i8_tt<FMT, true>(a, tt, st) : i8_tt<FMT, false>(a, tt, st);
        if (r != SLHIP_OK) return r;
    }
    return SLHIP_OK;
}

// instantiated in matvec_i8_*.hip, one group of formats per unit
int run_i8_part0(int fmt, const I8Args& a, bool dual, hipStream_t st);
int run_i8_part1(int fmt, const I8Args& a, bool dual, hipStream_t st);
int run_i8_part2(int fmt, const I8Args& a, bool dual, hipStream_t st);
int run_i8_part3(int fmt, const I8Args& a, bool dual, hipStream_t st);

}  // namespace slhip
