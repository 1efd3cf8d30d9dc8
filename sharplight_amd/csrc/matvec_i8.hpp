#pragma once
// The integer-dot decode matvec's kernels and launch templates. matvec_i8.hip holds the activation
// quantization, the entry points and the description of the numerics; matvec_i8_0..3.hip instantiate the
// weight formats in separate units so that they compile in parallel.
#include "act.hpp"
#include "common.hpp"
#include "quant.hpp"

#include <limits.h>

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

    const int tot = R * nch;
    auto load_batch = [&](int64_t n, int base, uint4* v) {
#pragma unroll
        for (int c = 0; c < CH; c++) {
            if (base + c * 64 >= tot) break;  // wave-uniform
            int idx = base + c * 64 + lane;
            idx = idx < tot ? idx : tot - 1;
            const int r = idx >= nch ? 1 : 0;
            v[c] = load_chunk<U>((r ? a.wu : a.wg) + n * a.wrow, static_cast<int64_t>(idx - r * nch) * 16, a.wrow);
        }
    };
    auto store_batch = [&](int base, const uint4* v) {
#pragma unroll
        for (int c = 0; c < CH; c++) {
            if (base + c * 64 >= tot) break;  // wave-uniform
            int idx = base + c * 64 + lane;
            idx = idx < tot ? idx : tot - 1;
            const int r = idx >= nch ? 1 : 0;
            reinterpret_cast<uint4*>(rows + r * rbw)[idx - r * nch] = v[c];
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
        const int full = nb / 64;  // iterations in which every lane has a unit
        for (int i = 0; i < full; i++) unit(lane + 64 * i, true);
        if (full * 64 < nb) {  // wave-uniform
            const int b = lane + 64 * full;
            unit(b < nb ? b : nb - 1, b < nb);
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

template <int FMT, bool DUAL>
static int i8_tt(const I8Args& a, int tt, hipStream_t st)
{
    switch (tt) {
    case 1: return i8_ch<FMT, 1, DUAL>(a, st);
    case 2: return i8_ch<FMT, 2, DUAL>(a, st);
    case 4: return i8_ch<FMT, 4, DUAL>(a, st);
    default: return i8_ch<FMT, 8, DUAL>(a, st);
    }
}

template <int FMT>
int run_i8(I8Args a, bool dual, hipStream_t st)
{
    int tt = 8;
    while (tt > 1 && (tt / 2 >= a.T || i8_lds(tt, a.K, a.wrow, dual) > kI8MaxLds)) tt /= 2;
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
