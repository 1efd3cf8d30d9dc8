// Decode matvec y = x . W^T and the dual gate/up matvec y = act(x . Wg^T) * (x . Wu^T), for few activation
// rows (T up to a few dozen): the step before the gated activation in a decode FFN.
//
// Semantics: the reference computes MatMul per activation row with f32 products of the dequantized weights
// and f32 accumulation (src/Sharplight.Cpu/MatMulOp.cs:376-465; the fused Q8_0/Q4_0 one-row dots,
// Quant.cs:738-803, scale each block's sum by its d), then the activation and Mul as f32 ops
// (ScalarMath.cs:552-641, BinaryOp.cs:8-103); the Vulkan lowerer fuses the pair and the elementwise group
// into one dual matvec launch (FoldDualMatMuls, src/Sharplight.Shaders/Lowering/GraphLowerer.Fusion.cs:
// 286-353). The sums here run in another order, so they agree with the reference within f32 rounding of
// a K-term dot product, not bit for bit.
//
// Layout and schedule (weight-bandwidth-bound: every weight byte is read once, x is tiny):
//   * a block of 8 waves owns 8 / WPR row pairs (gate row n and up row n; one row for the plain matvec);
//     WPR waves split a row's K, each lane holding NV 16-byte weight vectors per row -- lane-contiguous,
//     so each load instruction covers 1 KiB of a row;
//   * the weight loads are issued first; then the block's TT activation rows are staged in LDS as f32
//     (their loads complete after the weights', which the in-order completion of vector loads enforces
//     anyway); each lane then reads the x values of its own vectors from LDS;
//   * per row and token, one f32 partial per lane -> wave butterfly -> (WPR > 1) one LDS exchange;
//   * the epilogue (activation, product, output rounding) runs on the reduced sums, one store per token.
// Rows past N and lanes past the row end work on clamped indices and store the same values as their
// owners, so every lane issues the same memory operations (a divergent branch around loads makes the
// compiler wait for all outstanding ones).
#include "act.hpp"
#include "common.hpp"
#include "mq.hpp"
#include "quant.hpp"

#include <stdlib.h>

#include <type_traits>

namespace slhip {

constexpr int kMvThreads = 512;

// Stages activation rows t0 .. t0+TT-1 (rows past T repeat row T-1) into LDS as f32 [TT][K], up to four
// 8-value groups per thread per pass; with XSUM also the sum of each 8-value group, [TT][K/8]. Slices wholly
// past the end are skipped (a block-uniform test); in the last partial slice the spare lanes repeat the last
// group (identical values; a duplicate LDS write of one address by many lanes would serialize).
template <int TT, bool XSUM>
__device__ __forceinline__ void stage_x(const MatvecArgs& a, float* xsh, float* xsum, int threads)
{
    const int per_row = static_cast<int>(a.K / 8);  // 8-value groups per row
    const int units = TT * per_row;
    for (int base = 0; base < units; base += 4 * threads) {
        float v[4][8];
#pragma unroll
        for (int q = 0; q < 4; q++) {
            if (base + q * threads >= units) break;
            int u = base + q * threads + static_cast<int>(threadIdx.x);
            u = u < units ? u : units - 1;
            const int t = u / per_row;
            const int c = u - t * per_row;
            int64_t tok = a.t0 + t;
            tok = tok < a.T ? tok : a.T - 1;
            if (a.xt == SLHIP_F32) {
                const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(a.x) + tok * a.xs + c * 8);
                const float4 f0 = p[0], f1 = p[1];
                v[q][0] = f0.x; v[q][1] = f0.y; v[q][2] = f0.z; v[q][3] = f0.w;
                v[q][4] = f1.x; v[q][5] = f1.y; v[q][6] = f1.z; v[q][7] = f1.w;
            } else {
                const uint4 b = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(a.x) + tok * a.xs + c * 8);
                Vec<SLHIP_BF16>::unpack(b, v[q]);
            }
        }
#pragma unroll
        for (int q = 0; q < 4; q++) {
            if (base + q * threads >= units) break;
            int u = base + q * threads + static_cast<int>(threadIdx.x);
            u = u < units ? u : units - 1;
            float4* d = reinterpret_cast<float4*>(xsh) + 2 * u;
            d[0] = make_float4(v[q][0], v[q][1], v[q][2], v[q][3]);
            d[1] = make_float4(v[q][4], v[q][5], v[q][6], v[q][7]);
            if (XSUM) xsum[u] = ((v[q][0] + v[q][1]) + (v[q][2] + v[q][3])) + ((v[q][4] + v[q][5]) + (v[q][6] + v[q][7]));
        }
    }
}

// Stages activation rows t0 .. t0+TT-1 for the block-format kernel: each 32-value block of x at a stride of
// 36 floats ([TT][K/32][36] f32; the pad makes lanes that read consecutive blocks hit distinct LDS banks; its
// first two floats hold the sums of the block's 16-value halves), and the sum of each block, [TT][K/32]. Two
// blocks per thread per pass.
template <int TT>
__device__ __forceinline__ void stage_x_blocks(const MatvecArgs& a, float* xsh, float* xsum, int threads)
{
    const int per_row = static_cast<int>(a.K / 32);
    const int units = TT * per_row;
    for (int base = 0; base < units; base += 2 * threads) {
        float v[2][32];
#pragma unroll
        for (int q = 0; q < 2; q++) {
            if (base + q * threads >= units) break;
            int u = base + q * threads + static_cast<int>(threadIdx.x);
            u = u < units ? u : units - 1;
            const int t = u / per_row;
            const int c = u - t * per_row;
            int64_t tok = a.t0 + t;
            tok = tok < a.T ? tok : a.T - 1;
            if (a.xt == SLHIP_F32) {
                const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(a.x) + tok * a.xs + c * 32);
#pragma unroll
                for (int k = 0; k < 8; k++) {
                    const float4 f = p[k];
                    v[q][4 * k] = f.x; v[q][4 * k + 1] = f.y; v[q][4 * k + 2] = f.z; v[q][4 * k + 3] = f.w;
                }
            } else {
                const uint4* p = reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(a.x) + tok * a.xs + c * 32);
#pragma unroll
                for (int k = 0; k < 4; k++) Vec<SLHIP_BF16>::unpack(p[k], v[q] + 8 * k);
            }
        }
#pragma unroll
        for (int q = 0; q < 2; q++) {
            if (base + q * threads >= units) break;
            int u = base + q * threads + static_cast<int>(threadIdx.x);
            u = u < units ? u : units - 1;
            float4* d = reinterpret_cast<float4*>(xsh + u * 36);
            float sum = 0.0f, half[2] = {0.0f, 0.0f};
#pragma unroll
            for (int k = 0; k < 8; k++) {
                d[k] = make_float4(v[q][4 * k], v[q][4 * k + 1], v[q][4 * k + 2], v[q][4 * k + 3]);
                const float p = (v[q][4 * k] + v[q][4 * k + 1]) + (v[q][4 * k + 2] + v[q][4 * k + 3]);
                sum += p;
                half[k >> 2] += p;
            }
            xsum[u] = sum;
            xsh[u * 36 + 32] = half[0];  // the pad holds the sums of the two 16-value halves (Q6_K)
            xsh[u * 36 + 33] = half[1];
        }
    }
}

// The epilogue of a wave holding the reduced sums of row n for tokens t0 .. t0+TT-1 (every lane holds all of
// them): act(g) * u for a dual matvec, else g, stored for each token by every lane (identical values to one
// address; a per-lane choice of token would be a dynamically indexed register array, i.e. scratch memory).
template <int TT, bool DUAL>
__device__ __forceinline__ void store_row(const MatvecArgs& a, int64_t n, const float (&ag)[TT], const float (&au)[TT])
{
#pragma unroll
    for (int t = 0; t < TT; t++) {
        float out = ag[t];
        if (DUAL) {
            const float g = ag[t];
            const float act = a.act == SLHIP_ACT_SILU        ? activate<SLHIP_ACT_SILU>(g)
                              : a.act == SLHIP_ACT_GELU_TANH ? activate<SLHIP_ACT_GELU_TANH>(g)
                                                             : activate<SLHIP_ACT_GELU_ERF>(g);
            out = act * au[t];
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
}

template <int WT, int TT, int NV, bool DUAL>
__global__ __launch_bounds__(kMvThreads) void matvec_dense(MatvecArgs a, int wpr)
{
    using VW = Vec<WT>;
    constexpr int E = VW::N;  // weights per 16-byte vector
    extern __shared__ float xsh[];  // [TT][K] f32

    const int lane = threadIdx.x & 63;
    const int wave = wave_id();
    const int rpb = (kMvThreads / 64) / wpr;
    const int rp = wave / wpr;
    const int wk = wave - rp * wpr;
    const int64_t n0 = static_cast<int64_t>(blockIdx.x) * rpb + rp;
    const int64_t n = n0 < a.N ? n0 : a.N - 1;
    const int nvr = static_cast<int>(a.K / E);
    const int stride = 64 * wpr;

    int jv[NV];
    bool own[NV];
#pragma unroll
    for (int k = 0; k < NV; k++) {
        const int j = wk * 64 + lane + k * stride;
        own[k] = j < nvr;
        jv[k] = own[k] ? j : nvr - 1;
    }
    uint4 rg[NV], ru[NV];
    const char* pg = a.wg + n * a.wrow;
#pragma unroll
    for (int k = 0; k < NV; k++) rg[k] = load_nt(pg + static_cast<int64_t>(jv[k]) * 16);
    if (DUAL) {
        const char* pu = a.wu + n * a.wrow;
#pragma unroll
        for (int k = 0; k < NV; k++) ru[k] = load_nt(pu + static_cast<int64_t>(jv[k]) * 16);
    }
    __builtin_amdgcn_sched_barrier(0);  // the weight loads go out before the staging loads

    stage_x<TT, false>(a, xsh, nullptr, kMvThreads);
    __syncthreads();

    float ag[TT], au[TT];
#pragma unroll
    for (int t = 0; t < TT; t++) ag[t] = au[t] = 0.0f;
#pragma unroll
    for (int k = 0; k < NV; k++) {
        float w[E], u[E];
        VW::unpack(rg[k], w);
        if (DUAL) VW::unpack(ru[k], u);
        const float* xr = xsh + static_cast<int64_t>(jv[k]) * E;
#pragma unroll
        for (int t = 0; t < TT; t++) {
            float xv[E];
#pragma unroll
            for (int q = 0; q < E / 4; q++) {
                const float4 f = reinterpret_cast<const float4*>(xr + t * a.K)[q];
                xv[4 * q + 0] = f.x;
                xv[4 * q + 1] = f.y;
                xv[4 * q + 2] = f.z;
                xv[4 * q + 3] = f.w;
            }
            float pg_ = 0.0f, pu_ = 0.0f;
#pragma unroll
            for (int e = 0; e < E; e++) {
                pg_ = fmaf(w[e], xv[e], pg_);
                if (DUAL) pu_ = fmaf(u[e], xv[e], pu_);
            }
            ag[t] += own[k] ? pg_ : 0.0f;
            if (DUAL) au[t] += own[k] ? pu_ : 0.0f;
        }
    }
#pragma unroll
    for (int t = 0; t < TT; t++) {
        ag[t] = wave_sum(ag[t]);
        if (DUAL) au[t] = wave_sum(au[t]);
    }
    if (wpr > 1) {  // block-uniform: every wave takes the same path through the barriers
        __shared__ float red[kMvThreads / 64][2 * 8];
        if (lane == 0) {
#pragma unroll
            for (int t = 0; t < TT; t++) {
                red[wave][t] = ag[t];
                red[wave][8 + t] = au[t];
            }
        }
        __syncthreads();
#pragma unroll
        for (int t = 0; t < TT; t++) {
            float sg = 0.0f, su = 0.0f;
            for (int i = 0; i < wpr; i++) {
                sg += red[rp * wpr + i][t];
                su += red[rp * wpr + i][8 + t];
            }
            ag[t] = sg;
            au[t] = su;
        }
    }
    if (wk != 0) return;  // wave-uniform

    store_row<TT, DUAL>(a, n, ag, au);
}

// Quantized weights (Q8_0, Q4_0, Q4_1, Q5_0, Q5_1; Q2_K, Q3_K, Q4_K, Q5_K, Q6_K by 32-value sub-blocks): persistent
// blocks of 4 waves; each wave walks row
// (pairs) n, n + 4 * gridDim.x, ... . A row's block images go to the wave's own LDS region with 16-byte loads
// (the blocks are only 2-byte aligned); the loads of the next row (pair) are issued before the current one
// is computed, so their latency hides behind that work. The block stages x (32-value blocks padded to 36
// floats) and the sum of every x block once. Each lane takes whole blocks: with the block's scale d and
// additive term (OFF * d or m), sum_k x_k (q_k d + add) = d * sum x q + add * sum x, the form of the
// reference's fused Q4_0 dot (Quant.cs:770-803).
// A K-quant row image in LDS, 32-value sub-block b (of super-block b / 8): its scale terms and 32 codes, one
// per byte of w (Quant.cs:518-624). Q4_K / Q5_K: value = fma(q, d0, -m), d0 = d * sc, m = dmin * mn; Q6_K:
// value = (q - 32) * s per 16 values, s = d * scale (d0 for values 0-15, d1 for 16-31); codes 0..63 here,
// the -32 applied to the halves' sums of x. Q3_K: value = (q - 4) * s per 16 values (q = 2 low bits + 4 * the
// hmask bit; s = d (sc - 32) with the 6-bit packed scales), the -4 applied like Q6_K's -32; Q2_K: value =
// q * d0 - m per 16 values (d0 = d * (sc & 15), m = dmin * (sc >> 4); second half d1, m1).
struct KSub {
    float d0, d1, m, m1;
    uint32_t w[8];
};

// Formats whose 32-value sub-block holds two 16-value scale groups.
template <int FMT>
constexpr bool kHalves = FMT == SLHIP_FMT_Q6_K || FMT == SLHIP_FMT_Q3_K || FMT == SLHIP_FMT_Q2_K;

template <int FMT>
__device__ __forceinline__ KSub ksub(const uint32_t* s, int b)
{
    KSub r;
    const int sb = b >> 3, j = b & 7;
    const LdsBytes B{s};
    if constexpr (FMT == SLHIP_FMT_Q4_K || FMT == SLHIP_FMT_Q5_K) {
        constexpr bool K5 = FMT == SLHIP_FMT_Q5_K;
        const int o = sb * (K5 ? 176 : 144);  // super-blocks of 144 / 176 bytes: 16-byte aligned
        uint32_t sc, mn;
        if (j < 4) {
            sc = B.u8(o + 4 + j) & 63u;
            mn = B.u8(o + 8 + j) & 63u;
        } else {
            sc = (B.u8(o + 8 + j) & 0xFu) | ((B.u8(o + j) >> 6) << 4);
            mn = (B.u8(o + 8 + j) >> 4) | ((B.u8(o + 4 + j) >> 6) << 4);
        }
        r.d0 = __fmul_rn(half_at(s, o), static_cast<float>(sc));
        r.d1 = r.d0;
        r.m = __fmul_rn(half_at(s, o + 2), static_cast<float>(mn));
        r.m1 = r.m;
        const uint32_t* q = s + (o + (K5 ? 48 : 16) + 32 * (j >> 1)) / 4;
        const uint32_t* qh = s + (o + 16) / 4;
#pragma unroll
        for (int k = 0; k < 8; k++) {
            uint32_t w = (q[k] >> (4 * (j & 1))) & 0x0F0F0F0Fu;
            if (K5) w |= ((qh[k] >> j) & 0x01010101u) << 4;
            asm("" : "+v"(w));  // hides the zero high bits: each byte then converts with one v_cvt_f32_ubyte
            r.w[k] = w;
        }
    } else if constexpr (FMT == SLHIP_FMT_Q2_K) {  // {scales[16], qs[64], f16 d, f16 dmin}, 84 bytes
        const int o = sb * 84, n = j >> 2, jj = j & 3;
        const float d = half_at(s, o + 80), dm = half_at(s, o + 82);
        const uint32_t c0 = B.u8(o + 8 * n + 2 * jj), c1 = B.u8(o + 8 * n + 2 * jj + 1);
        r.d0 = __fmul_rn(d, static_cast<float>(c0 & 15u));
        r.d1 = __fmul_rn(d, static_cast<float>(c1 & 15u));
        r.m = __fmul_rn(dm, static_cast<float>(c0 >> 4));
        r.m1 = __fmul_rn(dm, static_cast<float>(c1 >> 4));
#pragma unroll
        for (int k = 0; k < 8; k++) {  // values 4k .. 4k + 3 of the sub-block: 2-bit field 2jj of qs[32n + v]
            uint32_t w = (lds_u32(s, o + 16 + 32 * n + 4 * k) >> (2 * jj)) & 0x03030303u;
            asm("" : "+v"(w));
            r.w[k] = w;
        }
    } else if constexpr (FMT == SLHIP_FMT_Q3_K) {  // {hmask[32], qs[64], scales[12], f16 d}, 110 bytes
        const int o = sb * 110, n = j >> 2, jj = j & 3;
        const float d = half_at(s, o + 108);
        // 6-bit scales s = 8n + 2jj + 0..1: low 4 bits from byte 96 + 4 (w & 1) + b (low nibble for w < 2),
        // high 2 bits from bits 2w of byte 104 + b, w = s / 4, b = s % 4
        auto scale = [&](int sidx) {
            const int w = sidx >> 2, b = sidx & 3;
            const uint32_t a = B.u8(o + 96 + 4 * (w & 1) + b);
            const uint32_t lo = w < 2 ? (a & 15u) : (a >> 4);
            const uint32_t hi = (B.u8(o + 104 + b) >> (2 * w)) & 3u;
            return static_cast<float>(static_cast<int>(lo | (hi << 4)) - 32);
        };
        r.d0 = __fmul_rn(d, scale(8 * n + 2 * jj));
        r.d1 = __fmul_rn(d, scale(8 * n + 2 * jj + 1));
        r.m = r.m1 = 0.0f;
#pragma unroll
        for (int k = 0; k < 8; k++) {  // 2-bit field 2jj of qs[32n + v], plus 4 with bit 4n + jj of hmask[v]
            const uint32_t l = lds_u32(s, o + 32 + 32 * n + 4 * k), h = lds_u32(s, o + 4 * k);
            uint32_t w = ((l >> (2 * jj)) & 0x03030303u) | (((h >> (4 * n + jj)) & 0x01010101u) << 2);
            asm("" : "+v"(w));
            r.w[k] = w;
        }
    } else {  // Q6_K: {ql[128], qh[64], int8 scales[16], f16 d}, 210 bytes (2-byte aligned)
        const int o = sb * 210, n = j >> 2, qt = j & 3;
        const float d = half_at(s, o + 208);
        r.d0 = __fmul_rn(d, static_cast<float>(static_cast<int8_t>(B.u8(o + 192 + 8 * n + 2 * qt))));
        r.d1 = __fmul_rn(d, static_cast<float>(static_cast<int8_t>(B.u8(o + 193 + 8 * n + 2 * qt))));
        r.m = r.m1 = 0.0f;
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const uint32_t l = lds_u32(s, o + 64 * n + 32 * (qt & 1) + 4 * k);
            const uint32_t h = lds_u32(s, o + 128 + 32 * n + 4 * k);
            uint32_t w = ((qt >= 2 ? l >> 4 : l) & 0x0F0F0F0Fu) | (((h >> (2 * qt)) & 0x03030303u) << 4);
            asm("" : "+v"(w));
            r.w[k] = w;
        }
    }
    return r;
}

// A two-half sub-block's share from the halves' sums of x q and of x (hx[0], hx[1]): Q6_K and Q3_K
// s0 (sum x q + OFF sum x) + s1 (...), their offset (-32, -4) applied once per half; Q2_K
// d0 sum x q - m sum x + d1 (...) - m1 (...).
template <int FMT>
__device__ __forceinline__ float half_terms(const KSub& k, float sq0, float sq1, const float* hx)
{
    if constexpr (FMT == SLHIP_FMT_Q2_K) {
        return fmaf(k.d1, sq1, fmaf(-k.m1, hx[1], fmaf(k.d0, sq0, -k.m * hx[0])));
    } else {
        constexpr float OFF = FMT == SLHIP_FMT_Q3_K ? -4.0f : -32.0f;
        return fmaf(k.d1, fmaf(OFF, hx[1], sq1), k.d0 * fmaf(OFF, hx[0], sq0));
    }
}

constexpr int kMqThreads = 256;
constexpr bool PAIR = true;  // both rows of a dual pair per x read (every block format but Q8_0)

// U: the width of the staging loads, 16 bytes unless the rows are not 16-byte multiples (Q6_K rows of K not
// a multiple of 2048: 210 (K / 256) bytes, aligned to the largest power of two dividing them); a row's
// 16-byte chunk is then read as 16 / U loads, the pieces past the row's end repeating its last unit (their
// bytes land in the row image's padding).
template <int U>
__device__ __forceinline__ uint4 load16_as(const char* row, int64_t off, int64_t wrow)
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

template <int FMT, int TT, int CH, bool DUAL, int U = 16>
__global__ __launch_bounds__(kMqThreads) void matvec_quant(MatvecArgs a)
{
    extern __shared__ uint32_t smem[];
    constexpr int R = DUAL ? 2 : 1;
    const int lane = threadIdx.x & 63;
    const int wave = wave_id();
    const int nch = static_cast<int>((a.wrow + 15) / 16);  // 16-byte chunks per row (the last may be partial)
    const int rbw = nch * 4;                         // words per row
    uint32_t* rows = smem + wave * R * rbw;
    float* xsh = reinterpret_cast<float*>(smem + (kMqThreads / 64) * R * rbw);
    const int nb = static_cast<int>(a.K / 32);  // blocks per row
    float* xsum = xsh + TT * nb * 36;

    const int tot = R * nch;
    auto load_batch = [&](int64_t n, int base, uint4* v) {
#pragma unroll
        for (int c = 0; c < CH; c++) {
            if (base + c * 64 >= tot) break;  // wave-uniform
            int idx = base + c * 64 + lane;
            idx = idx < tot ? idx : tot - 1;
            const int r = idx >= nch ? 1 : 0;
            v[c] = load16_as<U>((r ? a.wu : a.wg) + n * a.wrow, static_cast<int64_t>(idx - r * nch) * 16, a.wrow);
        }
    };
    auto store_batch = [&](int base, const uint4* v) {
#pragma unroll
        for (int c = 0; c < CH; c++) {
            if (base + c * 64 >= tot) break;  // wave-uniform
            int idx = base + c * 64 + lane;
            idx = idx < tot ? idx : tot - 1;
            reinterpret_cast<uint4*>(rows)[idx] = v[c];
        }
    };
    auto rest = [&](int64_t n, uint4* v) {  // batches after the first, loaded and stored in turn
        for (int base = CH * 64; base < tot; base += CH * 64) {
            load_batch(n, base, v);
            store_batch(base, v);
        }
    };
    const int64_t stride = static_cast<int64_t>(gridDim.x) * (kMqThreads / 64);
    int64_t n = static_cast<int64_t>(blockIdx.x) * (kMqThreads / 64) + wave;
    const int64_t n_first = n < a.N ? n : a.N - 1;
    uint4 v[CH];
    load_batch(n_first, 0, v);
    __builtin_amdgcn_sched_barrier(0);  // the weight loads go out before the staging loads
    stage_x_blocks<TT>(a, xsh, xsum, kMqThreads);
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
        // One block of both rows for every token; OWN false: a lane past the row's end adds nothing.
        // One row's block for every token (Q8_0's 32 code bytes take 8 registers per row, so the rows of a
        // pair go one after the other rather than side by side).
        auto row_block = [&](const uint32_t* img, int b, bool own, float* acc) {
            if constexpr (Fmt<FMT>::K) {
                // K-quants: sum x q over the sub-block (Q6_K: per 16-value half), then
                // d0 * sum - m * sum x (Q4_K, Q5_K) or the halves' (sum x q - 32 sum x) scaled (Q6_K)
                const KSub ks = ksub<FMT>(img, b);
                float s0[TT], s1[TT];
#pragma unroll
                for (int t = 0; t < TT; t++) s0[t] = s1[t] = 0.0f;
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    float q[8];
#pragma unroll
                    for (int e = 0; e < 8; e++) {
                        q[e] = static_cast<float>((ks.w[2 * j + (e >> 2)] >> (8 * (e & 3))) & 0xFFu);
                    }
#pragma unroll
                    for (int t = 0; t < TT; t++) {
                        const float4* xp = reinterpret_cast<const float4*>(xsh + (t * nb + b) * 36 + 8 * j);
                        const float4 x0 = xp[0], x1 = xp[1];
                        const float xv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
                        float& acc_h = (kHalves<FMT> && j >= 2) ? s1[t] : s0[t];
#pragma unroll
                        for (int e = 0; e < 8; e++) acc_h = fmaf(q[e], xv[e], acc_h);
                    }
                }
#pragma unroll
                for (int t = 0; t < TT; t++) {
                    const float* hx = xsh + (t * nb + b) * 36 + 32;
                    const float p = kHalves<FMT> ? half_terms<FMT>(ks, s0[t], s1[t], hx)
                                                          : fmaf(-ks.m, xsum[t * nb + b], ks.d0 * s0[t]);
                    acc[t] += own ? p : 0.0f;
                }
                return;
            }
            const BlockWords<FMT> bw = block_words<FMT>(img, b);
            float sx[TT];
#pragma unroll
            for (int t = 0; t < TT; t++) sx[t] = 0.0f;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                float q[8];
                block_codes8<FMT>(bw, j, q);
#pragma unroll
                for (int t = 0; t < TT; t++) {
                    const float4* xp = reinterpret_cast<const float4*>(xsh + (t * nb + b) * 36 + 8 * j);
                    const float4 x0 = xp[0], x1 = xp[1];
                    const float xv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
                    for (int e = 0; e < 8; e++) sx[t] = fmaf(q[e], xv[e], sx[t]);
                }
            }
#pragma unroll
            for (int t = 0; t < TT; t++) {
                float p = bw.d * sx[t];
                if (FMT != SLHIP_FMT_Q8_0) p = fmaf(bw.add, xsum[t * nb + b], p);
                acc[t] += own ? p : 0.0f;
            }
        };
        // Both rows of a pair at once (not Q8_0, whose codes take 8 registers per row): each x vector is read
        // from LDS once for the gate and the up row.
        auto pair_block = [&](int b, bool own) {
            float g0[TT], g1[TT], u0[TT], u1[TT];
#pragma unroll
            for (int t = 0; t < TT; t++) g0[t] = g1[t] = u0[t] = u1[t] = 0.0f;
            auto dot8 = [&](const float* qg, const float* qu, int j, bool second) {
#pragma unroll
                for (int t = 0; t < TT; t++) {
                    const float4* xp = reinterpret_cast<const float4*>(xsh + (t * nb + b) * 36 + 8 * j);
                    const float4 x0 = xp[0], x1 = xp[1];
                    const float xv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
                    float& ag_h = second ? g1[t] : g0[t];
                    float& au_h = second ? u1[t] : u0[t];
#pragma unroll
                    for (int e = 0; e < 8; e++) {
                        ag_h = fmaf(qg[e], xv[e], ag_h);
                        au_h = fmaf(qu[e], xv[e], au_h);
                    }
                }
            };
            if constexpr (Fmt<FMT>::K) {
                const KSub kg = ksub<FMT>(rows, b), ku = ksub<FMT>(rows + rbw, b);
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    float qg[8], qu[8];
#pragma unroll
                    for (int e = 0; e < 8; e++) {
                        qg[e] = static_cast<float>((kg.w[2 * j + (e >> 2)] >> (8 * (e & 3))) & 0xFFu);
                        qu[e] = static_cast<float>((ku.w[2 * j + (e >> 2)] >> (8 * (e & 3))) & 0xFFu);
                    }
                    dot8(qg, qu, j, kHalves<FMT> && j >= 2);
                }
#pragma unroll
                for (int t = 0; t < TT; t++) {
                    const float* hx = xsh + (t * nb + b) * 36 + 32;
                    const float pg = kHalves<FMT> ? half_terms<FMT>(kg, g0[t], g1[t], hx)
                                                           : fmaf(-kg.m, xsum[t * nb + b], kg.d0 * g0[t]);
                    const float pu = kHalves<FMT> ? half_terms<FMT>(ku, u0[t], u1[t], hx)
                                                           : fmaf(-ku.m, xsum[t * nb + b], ku.d0 * u0[t]);
                    ag[t] += own ? pg : 0.0f;
                    au[t] += own ? pu : 0.0f;
                }
            } else {
                const BlockWords<FMT> bg = block_words<FMT>(rows, b), bu = block_words<FMT>(rows + rbw, b);
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    float qg[8], qu[8];
                    block_codes8<FMT>(bg, j, qg);
                    block_codes8<FMT>(bu, j, qu);
                    dot8(qg, qu, j, false);
                }
#pragma unroll
                for (int t = 0; t < TT; t++) {
                    const float pg = fmaf(bg.add, xsum[t * nb + b], bg.d * g0[t]);
                    const float pu = fmaf(bu.add, xsum[t * nb + b], bu.d * u0[t]);
                    ag[t] += own ? pg : 0.0f;
                    au[t] += own ? pu : 0.0f;
                }
            }
        };
        auto block = [&](int b, bool own) {
            if constexpr (DUAL && FMT != SLHIP_FMT_Q8_0 && PAIR) {
                pair_block(b, own);
            } else {
                row_block(rows, b, own, ag);
                if (DUAL) row_block(rows + rbw, b, own, au);
            }
        };
        const int full = nb / 64;  // iterations in which every lane has a block
        for (int i = 0; i < full; i++) block(lane + 64 * i, true);
        if (full * 64 < nb) {  // wave-uniform
            const int b = lane + 64 * full;
            block(b < nb ? b : nb - 1, b < nb);
        }
#pragma unroll
        for (int t = 0; t < TT; t++) {
            ag[t] = wave_sum(ag[t]);
            if (DUAL) au[t] = wave_sum(au[t]);
        }
        store_row<TT, DUAL>(a, n, ag, au);
        if (more) {
            store_batch(0, v);
            rest(next, v);
        }
    }
}

// bf16 weights at several tokens on the matrix cores: v_mfma_f32_16x16x32_bf16 multiplies a 16-row weight
// tile (A: lane l holds row l % 16, eight K values of group l / 16) by 16 tokens of x (B: lane l holds token
// l % 16, the same K values) into a 16 x 16 f32 tile (lane l: rows 4 (l / 16) + i, token l % 16). f32 x is
// split into three bf16 parts h + m + l = x exactly (each part the round-to-nearest-even of the remainder;
// f32 has 24 significant bits, bf16 8), so every product w * part is exact and the sums stay f32: the
// result has the error of f32 accumulation, like the VALU kernel. bf16 x is one part. A block of 8 waves
// takes a 16-row tile (pair); the waves split K, each lane loading 2 x 16 bytes per row per 64 values (two
// instructions covering 64 contiguous bytes of 16 rows each); partial tiles meet in LDS.
constexpr int kMmWaves = 8;

template <bool DUAL, bool XF32>
__global__ __launch_bounds__(64 * kMmWaves) void matvec_mfma(MatvecArgs a)
{
    __shared__ f32x4_t red[kMmWaves][2][64];
    const int lane = threadIdx.x & 63;
    const int wave = wave_id();
    const int r = lane & 15, g = lane >> 4;
    const int64_t n0 = static_cast<int64_t>(blockIdx.x) * 16;
    const int64_t row = n0 + r < a.N ? n0 + r : a.N - 1;
    int64_t tok = a.t0 + r;
    tok = tok < a.T ? tok : a.T - 1;
    const int nc = static_cast<int>(a.K / 64);
    const int c0 = wave * nc / kMmWaves, c1 = (wave + 1) * nc / kMmWaves;
    const char* wg = a.wg + row * a.wrow;
    const char* wu = DUAL ? a.wu + row * a.wrow : nullptr;
    f32x4_t ag = {0.0f, 0.0f, 0.0f, 0.0f}, au = {0.0f, 0.0f, 0.0f, 0.0f};
    // One chunk's operands as loaded: weights (gate, up: two 16-byte vectors each) and x (f32: four float4;
    // bf16: two uint4 in xb). The next chunk's loads are issued before the current chunk is computed.
    struct Ops {
        uint4 A0, A1, U0, U1;
        float4 xf[4];
        uint4 xb[2];
    };
    auto load = [&](int c, Ops& o) {
        const int64_t k0 = static_cast<int64_t>(c) * 64 + 8 * g;  // step 0: 64c + 8g + j; step 1: + 32
        o.A0 = load_nt(wg + k0 * 2);
        o.A1 = load_nt(wg + (k0 + 32) * 2);
        if (DUAL) {
            o.U0 = load_nt(wu + k0 * 2);
            o.U1 = load_nt(wu + (k0 + 32) * 2);
        }
        if (XF32) {
            const float* xr = static_cast<const float*>(a.x) + tok * a.xs + k0;
            o.xf[0] = *reinterpret_cast<const float4*>(xr);
            o.xf[1] = *reinterpret_cast<const float4*>(xr + 4);
            o.xf[2] = *reinterpret_cast<const float4*>(xr + 32);
            o.xf[3] = *reinterpret_cast<const float4*>(xr + 36);
        } else {
            const uint16_t* xr = static_cast<const uint16_t*>(a.x) + tok * a.xs + k0;
            o.xb[0] = *reinterpret_cast<const uint4*>(xr);
            o.xb[1] = *reinterpret_cast<const uint4*>(xr + 32);
        }
    };
    auto compute = [&](const Ops& o) {
        uint4 B[2][3];
        int np = 1;
        if (XF32) {
#pragma unroll
            for (int s2 = 0; s2 < 2; s2++) {
                const float4 f0 = o.xf[2 * s2], f1 = o.xf[2 * s2 + 1];
                const float xv[8] = {f0.x, f0.y, f0.z, f0.w, f1.x, f1.y, f1.z, f1.w};
                split3(xv, B[s2][0], B[s2][1], B[s2][2]);
            }
            np = 3;
        } else {
            B[0][0] = o.xb[0];
            B[1][0] = o.xb[1];
        }
#pragma unroll
        for (int p = 0; p < 3; p++) {
            if (p >= np) break;
            ag = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(o.A0), as_bf16x8(B[0][p]), ag, 0, 0, 0);
            ag = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(o.A1), as_bf16x8(B[1][p]), ag, 0, 0, 0);
            if (DUAL) {
                au = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(o.U0), as_bf16x8(B[0][p]), au, 0, 0, 0);
                au = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(o.U1), as_bf16x8(B[1][p]), au, 0, 0, 0);
            }
        }
    };
    // Two operand sets in alternation (a copy between them would wait for the loads): each chunk's loads are
    // issued before the previous chunk is computed. The scheduling barriers keep them there -- left free, the
    // scheduler sinks the loads below the MFMAs and every chunk waits for its own loads.
    const int n = c1 - c0;
    if (n > 0) {  // wave-uniform
        Ops oa, ob;
        load(c0, oa);
        int i = 0;
        for (; i + 2 < n; i += 2) {  // branch-free body: a merge would make the load counter waits exact-zero
            load(c0 + i + 1, ob);
            __builtin_amdgcn_sched_barrier(0);
            compute(oa);
            __builtin_amdgcn_sched_barrier(0);
            load(c0 + i + 2, oa);
            __builtin_amdgcn_sched_barrier(0);
            compute(ob);
            __builtin_amdgcn_sched_barrier(0);
        }
        if (i + 1 < n) {  // two chunks left
            load(c0 + i + 1, ob);
            __builtin_amdgcn_sched_barrier(0);
            compute(oa);
            __builtin_amdgcn_sched_barrier(0);
            compute(ob);
        } else {
            compute(oa);
        }
    }
    red[wave][0][lane] = ag;
    if (DUAL) red[wave][1][lane] = au;
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int w = 1; w < kMmWaves; w++) {
        ag += red[w][0][lane];
        if (DUAL) au += red[w][1][lane];
    }
    // lane: token column r, rows 4g + i
    const int64_t t = a.t0 + r;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int64_t n = n0 + 4 * g + i;
        float out = ag[i];
        if (DUAL) {
            const float act = a.act == SLHIP_ACT_SILU        ? activate<SLHIP_ACT_SILU>(ag[i])
                              : a.act == SLHIP_ACT_GELU_TANH ? activate<SLHIP_ACT_GELU_TANH>(ag[i])
                                                             : activate<SLHIP_ACT_GELU_ERF>(ag[i]);
            out = act * au[i];
        }
        if (t < a.T && n < a.N) {
            if (!DUAL && a.bias) out = out + a.bias[n];
            if (a.yt == SLHIP_F32)
                static_cast<float*>(a.y)[t * a.ys + n] = out;
            else
                static_cast<uint16_t*>(a.y)[t * a.ys + n] = static_cast<uint16_t>(f32_to_bf16_bits(out));
        }
    }
}

// The same product with the weights staged row by row: reading a 16-row tile straight into MFMA operands
// puts 16 rows x 64 bytes in every load instruction, a pattern HBM serves at ~5.0 TB/s, while 1 KiB of one
// or two rows per instruction streams at ~6.4 TB/s. So per stage of SK values, the block loads the tile's
// rows contiguously into LDS (row pitch SK*2 + 16 bytes: the 16 rows of an A fragment fall 4 banks apart),
// and each wave reads its A fragments from there. Stages are double-buffered: the next stage's rows (and
// this wave's x) are in flight while the current one is multiplied, one barrier per stage.
template <bool DUAL, bool XF32, int SK, int NT>
__global__ __launch_bounds__(64 * kMmWaves) void matvec_mfma_lds(MatvecArgs a)
{
    constexpr int NM = DUAL ? 2 : 1;
    constexpr int ROWS = 16 * NT;               // rows per block: NT tiles share each x fragment
    constexpr int RB = SK * 2;                  // bytes of one row per stage
    constexpr int PITCH = RB + 16;
    constexpr int RPI = 1024 / RB;              // rows per 1 KiB load instruction
    constexpr int LPR = 64 / RPI;               // lanes per row in one instruction
    constexpr int UNITS = NM * ROWS / RPI;      // load instructions per stage
    constexpr int UPW = UNITS / kMmWaves;       // ... per wave
    constexpr int KPW = SK / 32 / kMmWaves;     // MFMA k-steps per wave per stage
    static_assert(UNITS % kMmWaves == 0 && UPW >= 1 && KPW >= 1, "stage shape");
    __shared__ __align__(16) uint8_t stage[2][NM][ROWS][PITCH];
    const int lane = threadIdx.x & 63;
    const int wave = wave_id();
    const int r = lane & 15, g = lane >> 4;
    const int64_t n0 = static_cast<int64_t>(blockIdx.x) * ROWS;
    int64_t tok = a.t0 + r;
    tok = tok < a.T ? tok : a.T - 1;
    const int ns = static_cast<int>(a.K / SK);

    // this lane's 16 bytes of each of the wave's load instructions
    const char* src[UPW];
    int dst[UPW];
#pragma unroll
    for (int i = 0; i < UPW; i++) {
        const int u = wave + kMmWaves * i;
        const int m = u / (ROWS / RPI), rr = (u % (ROWS / RPI)) * RPI + lane / LPR;
        const int byte = (lane % LPR) * 16;
        int64_t row = n0 + rr;
        row = row < a.N ? row : a.N - 1;
        src[i] = (m == 0 ? a.wg : a.wu) + row * a.wrow + byte;
        dst[i] = (m * ROWS + rr) * PITCH + byte;
    }
    // Weight rows two stages ahead, in two register sets (the LDS holds the current and the next stage):
    // stage s + 2 is loaded while s is multiplied, and s + 1 is written to LDS at the end of stage s.
    uint4 pa[UPW], pb[UPW];
    auto fetch_w = [&](uint4* pw, int s) {
#pragma unroll
        for (int i = 0; i < UPW; i++) pw[i] = load_nt(src[i] + static_cast<int64_t>(s) * RB);
    };
    auto put_w = [&](const uint4* pw, int b) {
#pragma unroll
        for (int i = 0; i < UPW; i++) *reinterpret_cast<uint4*>(&stage[b][0][0][0] + dst[i]) = pw[i];
    };
    // x of this wave's k-steps: f32 two float4, bf16 one uint4 per k-step (one stage ahead)
    float4 xf[KPW][2];
    uint4 xb[KPW];
    auto fetch_x = [&](int s) {
#pragma unroll
        for (int q = 0; q < KPW; q++) {
            const int64_t k0 = static_cast<int64_t>(s) * SK + (wave * KPW + q) * 32 + 8 * g;
            if (XF32) {
                const float* xr = static_cast<const float*>(a.x) + tok * a.xs + k0;
                xf[q][0] = *reinterpret_cast<const float4*>(xr);
                xf[q][1] = *reinterpret_cast<const float4*>(xr + 4);
            } else {
                xb[q] = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(a.x) + tok * a.xs + k0);
            }
        }
    };
    f32x4_t ag[NT], au[NT];
#pragma unroll
    for (int tt = 0; tt < NT; tt++) ag[tt] = au[tt] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    // Stage s from LDS buffer s & 1. Issue order matters for the in-order load counter: x(s + 1) before
    // w(s + 2), so that waiting for x at the next stage leaves w(s + 2) in flight.
    auto run_stage = [&](int s, uint4* wnext, uint4* wfree) {
        const int b = s & 1;
        uint4 B[KPW][3];
        uint4 Ag[KPW][NT], Au[KPW][NT];
#pragma unroll
        for (int q = 0; q < KPW; q++) {
            if (XF32) {
                const float v[8] = {xf[q][0].x, xf[q][0].y, xf[q][0].z, xf[q][0].w,
                                    xf[q][1].x, xf[q][1].y, xf[q][1].z, xf[q][1].w};
                split3(v, B[q][0], B[q][1], B[q][2]);
            } else {
                B[q][0] = xb[q];
            }
            const int kb = ((wave * KPW + q) * 32 + 8 * g) * 2;
#pragma unroll
            for (int tt = 0; tt < NT; tt++) {
                Ag[q][tt] = *reinterpret_cast<const uint4*>(&stage[b][0][16 * tt + r][kb]);
                if (DUAL) Au[q][tt] = *reinterpret_cast<const uint4*>(&stage[b][NM - 1][16 * tt + r][kb]);
            }
        }
        if (s + 1 < ns) fetch_x(s + 1);        // block-uniform conditions
        if (s + 2 < ns) fetch_w(wfree, s + 2);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int q = 0; q < KPW; q++) {
#pragma unroll
            for (int p = 0; p < (XF32 ? 3 : 1); p++) {
#pragma unroll
                for (int tt = 0; tt < NT; tt++) {
                    ag[tt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(Ag[q][tt]), as_bf16x8(B[q][p]), ag[tt], 0, 0, 0);
                    if (DUAL)
                        au[tt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(Au[q][tt]), as_bf16x8(B[q][p]), au[tt], 0, 0, 0);
                }
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        if (s + 1 < ns) put_w(wnext, b ^ 1);
        __syncthreads();
    };
    fetch_x(0);
    fetch_w(pa, 0);
    if (ns > 1) fetch_w(pb, 1);
    put_w(pa, 0);
    __syncthreads();
    // stage s: the next stage's rows are in pb (s even) or pa (s odd); the other set is free
    int s = 0;
    for (; s + 1 < ns; s += 2) {
        run_stage(s, pb, pa);
        run_stage(s + 1, pa, pb);
    }
    if (s < ns) run_stage(s, pb, pa);
    // partial tiles meet in the (now idle) stage memory: [wave][tile][matrix][lane]
    f32x4_t* red = reinterpret_cast<f32x4_t*>(&stage[0][0][0][0]);
    static_assert(sizeof(stage) >= sizeof(f32x4_t) * kMmWaves * NM * NT * 64, "reduction space");
#pragma unroll
    for (int tt = 0; tt < NT; tt++) {
        red[((wave * NT + tt) * NM) * 64 + lane] = ag[tt];
        if (DUAL) red[((wave * NT + tt) * NM + 1) * 64 + lane] = au[tt];
    }
    __syncthreads();
    // wave tt < NT finishes tile tt
    if (wave >= NT) return;
    const int tt = wave;
    f32x4_t sg = red[(tt * NM) * 64 + lane], su = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    if (DUAL) su = red[(tt * NM + 1) * 64 + lane];
#pragma unroll
    for (int w = 1; w < kMmWaves; w++) {
        sg += red[((w * NT + tt) * NM) * 64 + lane];
        if (DUAL) su += red[((w * NT + tt) * NM + 1) * 64 + lane];
    }
    const int64_t t = a.t0 + r;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int64_t n = n0 + 16 * tt + 4 * g + i;
        float out = sg[i];
        if (DUAL) {
            const float act = a.act == SLHIP_ACT_SILU        ? activate<SLHIP_ACT_SILU>(sg[i])
                              : a.act == SLHIP_ACT_GELU_TANH ? activate<SLHIP_ACT_GELU_TANH>(sg[i])
                                                             : activate<SLHIP_ACT_GELU_ERF>(sg[i]);
            out = act * su[i];
        }
        if (t < a.T && n < a.N) {
            if (!DUAL && a.bias) out = out + a.bias[n];
            if (a.yt == SLHIP_F32)
                static_cast<float*>(a.y)[t * a.ys + n] = out;
            else
                static_cast<uint16_t*>(a.y)[t * a.ys + n] = static_cast<uint16_t>(f32_to_bf16_bits(out));
        }
    }
}

// ---- block formats at several tokens on the matrix cores -------------------------------------------------
//
// The VALU kernel decodes every weight once per group of tokens, so its time grows with T (Q4_0 dual at
// [14336, 4096]: 18 us at T = 1, 57 at 4, 218 at 16). Here a 16-row tile's blocks are staged raw in LDS and
// each code is decoded once into a bf16 A fragment that serves all 16 token columns of
// v_mfma_f32_16x16x32_bf16: a 32-value block is one MFMA k-step, so each block's sums (16 rows x 16 tokens)
// come out of one short MFMA chain and take the block scale d on the VALU (acc += d * sum). The codes enter
// exactly (Q4_0: q - 8, Q8_0: q; small integers are exact in bf16); f32 x enters as two bf16 parts h + m
// (h = bf16(x), m = bf16(x - h): |x - h - m| <= 2^-18 |x|, inside the matvec bound), bf16 x as it is. Q4_K
// takes the same path with its 32-value sub-blocks as the blocks (a stage is 4 super-blocks, 576 bytes of a
// row, and a wave half a super-block): codes q enter as they are, and the sub-block's d0 = d sc and minimum
// m = dmin mn are applied on the VALU as acc += d0 sum(q x) - m sum(x), sum(x) of the lane's token summed
// across its four lane groups (Quant.cs:518-545's value d0 q - m). Q6_K too (a stage is 2 super-blocks, 420
// bytes staged with 4-byte loads, and a wave a quarter super-block): codes enter as q - 32, and since a
// 32-value block holds two 16-value scale groups, each block takes two MFMA chains, lane groups 0-1 (the
// first group's values) in one and 2-3 in the other, the other half's codes masked to zero. The other block
// formats follow the same pattern: Q4_1 and Q5_1 add m sum(x) per block, Q5_0 and Q5_1 take the 17th code
// bit from their qh word, Q5_K is Q4_K with qh bit j of byte l, and Q2_K / Q3_K (16-value scale groups, as
// Q6_K; Q3_K's codes q + 4h - 4, Q2_K's per-half minimum dmin m sum(x) over each half). A block of 8 waves
// takes one tile; the waves split each stage's blocks; the stage's row bytes are loaded two stages
// ahead into registers and written to LDS one stage ahead (as the bf16 kernel above); partial sums meet in
// LDS at the end.
__device__ __forceinline__ void q4k_scales(const uint4& hdr, int j, float& d0, float& m);  // defined below

template <int FMT, bool DUAL, bool XF32>
__global__ __launch_bounds__(64 * kMqWaves) void matvec_mfma_q(MatvecArgs a)
{
    constexpr int BB = Fmt<FMT>::BB;
    constexpr int NM = DUAL ? 2 : 1;
    constexpr int SKB = MqGeom<FMT>::SKB;
    constexpr bool KQ = FMT == SLHIP_FMT_Q4_K || FMT == SLHIP_FMT_Q5_K;  // 8 sub-blocks, d0 q - m
    constexpr bool Q2K = FMT == SLHIP_FMT_Q2_K, Q3K = FMT == SLHIP_FMT_Q3_K;
    constexpr bool K6 = FMT == SLHIP_FMT_Q6_K || Q2K || Q3K;  // two 16-value scale groups per 32-value block
    constexpr bool MB = Fmt<FMT>::M && !Fmt<FMT>::K;  // Q4_1, Q5_1: d q + m per 32-value block
    constexpr int SBB = Fmt<FMT>::BB;                  // K-quant super-block bytes
    constexpr int RB = MqGeom<FMT>::RB;  // bytes of one row per stage
    constexpr int UB = MqGeom<FMT>::UB;  // bytes per staging load
    using WU = std::conditional_t<UB == 16, uint4, std::conditional_t<UB == 8, uint2, uint32_t>>;
    constexpr int PITCH = RB + 16;
    constexpr int UPR = RB / UB;  // staging units of a row per stage
    constexpr int UNITS = NM * 16 * UPR;
    constexpr int UPL = (UNITS + 64 * kMqWaves - 1) / (64 * kMqWaves);
    constexpr int BPW = SKB / kMqWaves;  // blocks per wave and stage
    static_assert(RB % UB == 0 && PITCH % UB == 0 && SKB % kMqWaves == 0, "stage shape");
    static_assert(!(KQ || K6) || 8 % BPW == 0, "a K-quant wave takes whole blocks of one super-block");
    static_assert(!KQ || BPW == 4, "a Q4_K wave takes the four sub-blocks of one packed scale word");
    __shared__ __align__(16) uint8_t stage[2][NM][16][PITCH];
    const int lane = threadIdx.x & 63;
    const int wave = wave_id();
    const int r = lane & 15, g = lane >> 4;
    const int64_t n0 = static_cast<int64_t>(blockIdx.x) * 16;
    int64_t tok = a.t0 + r;
    tok = tok < a.T ? tok : a.T - 1;
    const int ns = static_cast<int>(a.K / (SKB * 32));  // stages (each SKB * 32 values of the row)

    // this thread's 16-byte units of the stage (threads past the last unit repeat it)
    const char* src[UPL];
    int dst[UPL];
#pragma unroll
    for (int i = 0; i < UPL; i++) {
        int u = static_cast<int>(threadIdx.x) + 64 * kMqWaves * i;
        u = u < UNITS ? u : UNITS - 1;
        const int m = u / (16 * UPR), rem = u - m * (16 * UPR), rr = rem / UPR, c = rem - rr * UPR;
        int64_t row = n0 + rr;
        row = row < a.N ? row : a.N - 1;
        src[i] = (m == 0 ? a.wg : a.wu) + row * a.wrow + UB * c;
        dst[i] = (m * 16 + rr) * PITCH + UB * c;
    }
    WU pa[UPL], pb[UPL];
    auto fetch_w = [&](WU* pw, int s) {
#pragma unroll
        for (int i = 0; i < UPL; i++) {
            const char* p = src[i] + static_cast<int64_t>(s) * RB;
            if constexpr (UB == 16) {
                pw[i] = load_nt(p);
            } else if constexpr (UB == 8) {
                const u32x2 v = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(p));
                pw[i] = make_uint2(v.x, v.y);
            } else {
                pw[i] = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(p));
            }
        }
    };
    auto put_w = [&](const WU* pw, int b) {
#pragma unroll
        for (int i = 0; i < UPL; i++) *reinterpret_cast<WU*>(&stage[b][0][0][0] + dst[i]) = pw[i];
    };
    // x of the wave's blocks, one stage ahead in two register sets: lane (g, token r) holds values 8g .. 8g + 7
    struct Xs {
        float4 f[BPW][2];
        uint4 b[BPW];
    };
    auto fetch_x = [&](Xs& x, int s) {
#pragma unroll
        for (int j = 0; j < BPW; j++) {
            const int64_t k0 = (static_cast<int64_t>(s) * SKB + wave * BPW + j) * 32 + 8 * g;
            if (XF32) {
                const float* xr = static_cast<const float*>(a.x) + tok * a.xs + k0;
                x.f[j][0] = *reinterpret_cast<const float4*>(xr);
                x.f[j][1] = *reinterpret_cast<const float4*>(xr + 4);
            } else {
                x.b[j] = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(a.x) + tok * a.xs + k0);
            }
        }
    };
    f32x4_t ag = {0.0f, 0.0f, 0.0f, 0.0f}, au = {0.0f, 0.0f, 0.0f, 0.0f};
    // Stage s from LDS buffer s & 1 with x in xc; the next stage's x (into xn) and the weights two ahead go
    // out first, then each block in turn: its codes and scales from LDS, x split, the MFMAs, the scaling.
    auto run_stage = [&](int s, const Xs& xc, Xs& xn, WU* wnext, WU* wfree) {
        const int b = s & 1;
        if (s + 1 < ns) fetch_x(xn, s + 1);  // block-uniform conditions
        if (s + 2 < ns) fetch_w(wfree, s + 2);
        __builtin_amdgcn_sched_barrier(0);
        // Q4_K: the wave's half super-block (sub-blocks 4 (wave & 1) ..); the headers of the rows its sums
        // belong to (4g .. 4g + 3) are read once per stage. (Decoding the (d0, m) pairs once per wave into an
        // LDS table instead cost a block of residency per CU: 82 -> 116 us at 16 tokens.)
        // K-quants: the wave's blocks u0 .. u0 + BPW - 1 of the stage's super-block (wave BPW) / 8
        const int u0 = (wave * BPW) & 7;
        const int sbo = (KQ || K6) ? ((wave * BPW) >> 3) * SBB : 0;
        // Q4_K: per row 4g + i its d, dmin and the packed 6-bit scales and minima of the wave's four sub-blocks
        // (byte j of scw / mnw: sub-block u0 + j; Quant.cs:518-545's packing), so that a sub-block's d0 and m
        // are one byte conversion and one multiply each
        float kdg[4], kmg[4], kdu[4], kmu[4];
        uint32_t scg[4], mng[4], scu[4], mnu[4];
        // Q6_K / Q3_K / Q2_K: the super-block scale d (Q2_K: and dmin) of the rows 4g + i
        float d6g[4], d6u[4], n6g[4], n6u[4];
        if constexpr (K6) {
            constexpr int DO = Q2K ? 80 : Q3K ? 108 : 208;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                d6g[i] = static_cast<float>(*reinterpret_cast<const _Float16*>(&stage[b][0][4 * g + i][sbo + DO]));
                d6u[i] = DUAL ? static_cast<float>(*reinterpret_cast<const _Float16*>(&stage[b][NM - 1][4 * g + i][sbo + DO]))
                              : 0.0f;
                if constexpr (Q2K) {
                    n6g[i] = static_cast<float>(*reinterpret_cast<const _Float16*>(&stage[b][0][4 * g + i][sbo + 82]));
                    n6u[i] = DUAL ? static_cast<float>(*reinterpret_cast<const _Float16*>(&stage[b][NM - 1][4 * g + i][sbo + 82]))
                                  : 0.0f;
                }
            }
        }
        if constexpr (KQ) {
            auto words = [&](const uint4& h, float& d, float& dm, uint32_t& sc, uint32_t& mn) {
                d = f16_lo(h.x);
                dm = f16_hi(h.x);
                if (u0 < 4) {  // sub-blocks 0-3: the low 6 bits of bytes 4..7 (scales) and 8..11 (minima)
                    sc = h.y & 0x3F3F3F3Fu;
                    mn = h.z & 0x3F3F3F3Fu;
                } else {  // 4-7: low / high nibbles of bytes 12..15, top two bits of bytes 4..11
                    sc = (h.w & 0x0F0F0F0Fu) | ((h.y >> 2) & 0x30303030u);
                    mn = ((h.w >> 4) & 0x0F0F0F0Fu) | ((h.z >> 2) & 0x30303030u);
                }
            };
#pragma unroll
            for (int i = 0; i < 4; i++) {
                words(*reinterpret_cast<const uint4*>(&stage[b][0][4 * g + i][sbo]), kdg[i], kmg[i], scg[i], mng[i]);
                if (DUAL)
                    words(*reinterpret_cast<const uint4*>(&stage[b][NM - 1][4 * g + i][sbo]), kdu[i], kmu[i], scu[i], mnu[i]);
            }
        }
#pragma unroll
        for (int j = 0; j < BPW; j++) {
            const int off = (wave * BPW + j) * BB;
            const int sj = u0 + j;  // K-quant 32-value block (0..7) in its super-block
            uint4 Ag, Au;
            if constexpr (KQ) {
                constexpr bool FIVE = FMT == SLHIP_FMT_Q5_K;
                Ag = q4k_codes<FIVE>(&stage[b][0][r][0], sbo, sj, g);
                Au = DUAL ? q4k_codes<FIVE>(&stage[b][NM - 1][r][0], sbo, sj, g) : Ag;
            } else if constexpr (Q2K || Q3K) {
                Ag = q23k_codes<Q3K>(&stage[b][0][r][0], sbo, sj, g);
                Au = DUAL ? q23k_codes<Q3K>(&stage[b][NM - 1][r][0], sbo, sj, g) : Ag;
            } else if constexpr (K6) {
                Ag = q6k_codes(&stage[b][0][r][0], sbo, sj, g);
                Au = DUAL ? q6k_codes(&stage[b][NM - 1][r][0], sbo, sj, g) : Ag;
            } else {
                Ag = mq_codes<FMT>(&stage[b][0][r][0], off, g);
                Au = DUAL ? mq_codes<FMT>(&stage[b][NM - 1][r][0], off, g) : Ag;
            }
            float dg[4], du[4], mg[4], mu[4];
            float ng0[4], ng1[4], nu0[4], nu1[4];  // Q2_K: the two halves' minima dmin * m
#pragma unroll
            for (int i = 0; i < 4; i++) {  // the scales of the rows this lane's sums belong to (4g .. 4g + 3)
                if constexpr (Q2K) {
                    // scale bytes 8n + 2j + 0..1 (the block's two halves): d (low nibble), dmin (high nibble)
                    auto sc2 = [&](const uint8_t* row, float d, float dm, float& s0, float& s1, float& m0, float& m1) {
                        const uint32_t v = *reinterpret_cast<const uint16_t*>(row + sbo + 2 * sj);
                        s0 = __fmul_rn(d, static_cast<float>(v & 0xFu));
                        s1 = __fmul_rn(d, static_cast<float>((v >> 8) & 0xFu));
                        m0 = __fmul_rn(dm, static_cast<float>((v >> 4) & 0xFu));
                        m1 = __fmul_rn(dm, static_cast<float>(v >> 12));
                    };
                    sc2(&stage[b][0][4 * g + i][0], d6g[i], n6g[i], dg[i], mg[i], ng0[i], ng1[i]);
                    if (DUAL) sc2(&stage[b][NM - 1][4 * g + i][0], d6u[i], n6u[i], du[i], mu[i], nu0[i], nu1[i]);
                } else if constexpr (Q3K) {
                    // 6-bit scales s = 8n + 2j + 0..1: low 4 bits from bytes 96 + 4 (w & 1) + b (the low nibble
                    // for w < 2), high 2 from bits 2w of bytes 104 + b, w = s / 4, b = s % 4; d (s - 32)
                    const int s0 = 2 * sj, w = s0 >> 2, b0 = s0 & 3;
                    auto sc3 = [&](const uint8_t* row, float d, float& o0, float& o1) {
                        const uint32_t a = *reinterpret_cast<const uint16_t*>(row + sbo + 96 + 4 * (w & 1) + b0);
                        const uint32_t h = *reinterpret_cast<const uint16_t*>(row + sbo + 104 + b0);
                        const uint32_t lo = w < 2 ? (a & 0x0F0Fu) : ((a >> 4) & 0x0F0Fu);
                        const uint32_t sc = lo | (((h >> (2 * w)) & 0x0303u) << 4);
                        o0 = __fmul_rn(d, static_cast<float>(static_cast<int>(sc & 0xFFu) - 32));
                        o1 = __fmul_rn(d, static_cast<float>(static_cast<int>(sc >> 8) - 32));
                    };
                    sc3(&stage[b][0][4 * g + i][0], d6g[i], dg[i], mg[i]);
                    if (DUAL) sc3(&stage[b][NM - 1][4 * g + i][0], d6u[i], du[i], mu[i]);
                } else if constexpr (KQ) {
                    const uint32_t sh = 8 * static_cast<uint32_t>(j);  // byte j: sub-block u0 + j
                    dg[i] = __fmul_rn(kdg[i], static_cast<float>((scg[i] >> sh) & 0xFFu));
                    mg[i] = __fmul_rn(kmg[i], static_cast<float>((mng[i] >> sh) & 0xFFu));
                    if (DUAL) {
                        du[i] = __fmul_rn(kdu[i], static_cast<float>((scu[i] >> sh) & 0xFFu));
                        mu[i] = __fmul_rn(kmu[i], static_cast<float>((mnu[i] >> sh) & 0xFFu));
                    }
                } else if constexpr (K6) {
                    // the block's two 16-value scales sc[8 hf + 2k + 0..1] (2-byte aligned): d sc as (dg, mg)
                    const int so = sbo + 192 + 2 * sj;
                    const uint32_t sg = *reinterpret_cast<const uint16_t*>(&stage[b][0][4 * g + i][so]);
                    dg[i] = __fmul_rn(d6g[i], static_cast<float>(static_cast<int8_t>(sg & 0xFFu)));
                    mg[i] = __fmul_rn(d6g[i], static_cast<float>(static_cast<int8_t>(sg >> 8)));
                    if (DUAL) {
                        const uint32_t su = *reinterpret_cast<const uint16_t*>(&stage[b][NM - 1][4 * g + i][so]);
                        du[i] = __fmul_rn(d6u[i], static_cast<float>(static_cast<int8_t>(su & 0xFFu)));
                        mu[i] = __fmul_rn(d6u[i], static_cast<float>(static_cast<int8_t>(su >> 8)));
                    }
                } else {
                    dg[i] = static_cast<float>(*reinterpret_cast<const _Float16*>(&stage[b][0][4 * g + i][off]));
                    du[i] = DUAL ? static_cast<float>(*reinterpret_cast<const _Float16*>(&stage[b][NM - 1][4 * g + i][off]))
                                 : 0.0f;
                    if constexpr (MB) {  // the block minimum m (f16 after d)
                        mg[i] = static_cast<float>(*reinterpret_cast<const _Float16*>(&stage[b][0][4 * g + i][off + 2]));
                        mu[i] = DUAL ? static_cast<float>(*reinterpret_cast<const _Float16*>(&stage[b][NM - 1][4 * g + i][off + 2]))
                                     : 0.0f;
                    }
                }
            }
            uint4 Bh, Bm;
            float xsum = 0.0f;  // Q4_K: the sub-block's x sum of this lane's token (the min term)
            if (XF32) {
                const float v[8] = {xc.f[j][0].x, xc.f[j][0].y, xc.f[j][0].z, xc.f[j][0].w,
                                    xc.f[j][1].x, xc.f[j][1].y, xc.f[j][1].z, xc.f[j][1].w};
                split2(v, Bh, Bm);
                if constexpr (KQ || MB || Q2K) xsum = ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
            } else {
                Bh = xc.b[j];
                if constexpr (KQ || MB || Q2K) {
                    const uint4& w = xc.b[j];
                    xsum = ((bf16_lo(w.x) + bf16_hi(w.x)) + (bf16_lo(w.y) + bf16_hi(w.y))) +
                           ((bf16_lo(w.z) + bf16_hi(w.z)) + (bf16_lo(w.w) + bf16_hi(w.w)));
                }
            }
            if constexpr (KQ || MB) {  // the four lane groups of the token hold the block's four 8-value parts
                xsum += __shfl_xor(xsum, 16);
                xsum += __shfl_xor(xsum, 32);
            }
            float xh0 = 0.0f, xh1 = 0.0f;  // Q2_K: the token's x sums over the block's two 16-value halves
            if constexpr (Q2K) {
                const float p01 = xsum + __shfl_xor(xsum, 16);  // lane groups {0, 1} or {2, 3}
                const float other = __shfl_xor(p01, 32);
                xh0 = g < 2 ? p01 : other;
                xh1 = g < 2 ? other : p01;
            }
            if constexpr (K6) {
                // Q6_K, Q3_K, Q2_K: lane groups 0-1 hold the block's first 16 values (scale dg), 2-3 the second (scale mg):
                // one MFMA chain per half, the other half's codes masked to zero (a mask, not a select of
                // vectors, which the compiler would lower to a stack array)
                const uint32_t keep = g < 2 ? ~0u : 0u;
                auto half = [&](const uint4& A, uint32_t k) { return make_uint4(A.x & k, A.y & k, A.z & k, A.w & k); };
                const f32x4_t zero = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int m = 0; m < NM; m++) {
                    const uint4& A = m == 0 ? Ag : Au;
                    const uint4 A0 = half(A, keep), A1 = half(A, ~keep);
                    f32x4_t c0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(A0), as_bf16x8(Bh), zero, 0, 0, 0);
                    f32x4_t c1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(A1), as_bf16x8(Bh), zero, 0, 0, 0);
                    if (XF32) {
                        c0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(A0), as_bf16x8(Bm), c0, 0, 0, 0);
                        c1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(A1), as_bf16x8(Bm), c1, 0, 0, 0);
                    }
                    f32x4_t& acc = m == 0 ? ag : au;
                    const float* s0 = m == 0 ? dg : du;
                    const float* s1 = m == 0 ? mg : mu;
#pragma unroll
                    for (int i = 0; i < 4; i++) acc[i] = fmaf(s1[i], c1[i], fmaf(s0[i], c0[i], acc[i]));
                    if constexpr (Q2K) {  // - dmin m per half times the half's x sum
                        const float* n0 = m == 0 ? ng0 : nu0;
                        const float* n1 = m == 0 ? ng1 : nu1;
#pragma unroll
                        for (int i = 0; i < 4; i++) acc[i] = fmaf(-n1[i], xh1, fmaf(-n0[i], xh0, acc[i]));
                    }
                }
                continue;
            }
            f32x4_t cg = {0.0f, 0.0f, 0.0f, 0.0f}, cu = {0.0f, 0.0f, 0.0f, 0.0f};
            cg = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(Ag), as_bf16x8(Bh), cg, 0, 0, 0);
            if (XF32) cg = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(Ag), as_bf16x8(Bm), cg, 0, 0, 0);
            if (DUAL) {
                cu = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(Au), as_bf16x8(Bh), cu, 0, 0, 0);
                if (XF32) cu = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(Au), as_bf16x8(Bm), cu, 0, 0, 0);
            }
#pragma unroll
            for (int i = 0; i < 4; i++) {
                ag[i] = fmaf(dg[i], cg[i], ag[i]);
                if (DUAL) au[i] = fmaf(du[i], cu[i], au[i]);
                if constexpr (KQ) {  // Q4_K, Q5_K: d0 sum(q x) - m sum(x)
                    ag[i] = fmaf(-mg[i], xsum, ag[i]);
                    if (DUAL) au[i] = fmaf(-mu[i], xsum, au[i]);
                }
                if constexpr (MB) {  // Q4_1, Q5_1: d sum(q x) + m sum(x)
                    ag[i] = fmaf(mg[i], xsum, ag[i]);
                    if (DUAL) au[i] = fmaf(mu[i], xsum, au[i]);
                }
            }
        }
        if (s + 1 < ns) put_w(wnext, b ^ 1);
        __syncthreads();
    };
    Xs xa, xb;
    fetch_x(xa, 0);
    fetch_w(pa, 0);
    if (ns > 1) fetch_w(pb, 1);
    put_w(pa, 0);
    __syncthreads();
    int s = 0;
    for (; s + 1 < ns; s += 2) {
        run_stage(s, xa, xb, pb, pa);
        run_stage(s + 1, xb, xa, pa, pb);
    }
    if (s < ns) run_stage(s, xa, xb, pb, pa);
    // the waves' partial sums meet in the (now idle) stage memory: [wave][matrix][lane]
    f32x4_t* red = reinterpret_cast<f32x4_t*>(&stage[0][0][0][0]);
    static_assert(sizeof(stage) >= sizeof(f32x4_t) * kMqWaves * NM * 64, "reduction space");
    red[(wave * NM) * 64 + lane] = ag;
    if (DUAL) red[(wave * NM + 1) * 64 + lane] = au;
    __syncthreads();
    if (wave != 0) return;
    f32x4_t sg = red[lane], su = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    if (DUAL) su = red[64 + lane];
#pragma unroll
    for (int w = 1; w < kMqWaves; w++) {
        sg += red[(w * NM) * 64 + lane];
        if (DUAL) su += red[(w * NM + 1) * 64 + lane];
    }
    const int64_t t = a.t0 + r;  // lane: token column r, rows 4g + i
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int64_t n = n0 + 4 * g + i;
        float out = sg[i];
        if (DUAL) {
            const float act = a.act == SLHIP_ACT_SILU        ? activate<SLHIP_ACT_SILU>(sg[i])
                              : a.act == SLHIP_ACT_GELU_TANH ? activate<SLHIP_ACT_GELU_TANH>(sg[i])
                                                             : activate<SLHIP_ACT_GELU_ERF>(sg[i]);
            out = act * su[i];
        }
        if (t < a.T && n < a.N) {
            if (!DUAL && a.bias) out = out + a.bias[n];
            if (a.yt == SLHIP_F32)
                static_cast<float*>(a.y)[t * a.ys + n] = out;
            else
                static_cast<uint16_t*>(a.y)[t * a.ys + n] = static_cast<uint16_t>(f32_to_bf16_bits(out));
        }
    }
}

// ---- K-quant weights at one token on the matrix cores (integer MFMA) -------------------------------------
//
// The VALU kernel above spends ~4 lane instructions per Q4_K weight (code extraction, conversion, FMA), which
// holds a decode dual matvec at ~38% of the HBM peak. Here the products run on v_mfma_i32_16x16x64_i8, exact
// in integers, and the VALU keeps the code masking and the per-sub-block scaling:
//   * x is written as four 7-bit digits per value against its 32-value block's exponent e:
//     x = 2^(e-6) (d1 + d2 2^-7 + d3 2^-14 + d4 2^-21) to within 2^(e-28), far below f32 accumulation error
//     (kq_digits).
//   * B (64 K x 16 N) is 16 weight rows: lane l holds row l % 16 and 16 codes (bytes, as masked) of its
//     K-group l / 16. A (16 M x 64 K) holds "slots": K-group g's values appear in slots 4g .. 4g+3 as the four
//     digit planes, every other slot zero. Output slot 4g + p (lane l holds slots 4 (l / 16) + 0..3 of row
//     l % 16) is then the exact integer sum S_p of the lane's own codes times digit p.
//   * After a group's MFMA a lane forms sum q x = 2^(e-6) (S1 + 2^-7 (S2 + 2^-7 (S3 + 2^-7 S4))) and scales
//     it by its group's scale: Q4_K d0 (that) - m X (X the f32 sum of the block's x), Q6_K d sc (that), its
//     codes entering B as the signed bytes q - 32. Rows of zero weights contribute exactly 0 (Q6_K: codes 32)
//     or exactly -m X (Q4_K: codes 0).
typedef int i32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ i32x4_t as_i32x4(const uint4& v) { return __builtin_bit_cast(i32x4_t, v); }

// Q4_K sub-block j (0..7, runtime) of a super-block header {f16 d, f16 dmin, u8 scales[12]}: d0 = d * sc,
// m = dmin * mn with the 6-bit sc, mn of Quant.cs:518-545.
__device__ __forceinline__ void q4k_scales(const uint4& hdr, int j, float& d0, float& m)
{
    const int sh = 8 * (j & 3);
    const uint32_t by = (hdr.y >> sh) & 0xFFu, bz = (hdr.z >> sh) & 0xFFu, bw = (hdr.w >> sh) & 0xFFu;
    // both forms, then a select by mask (a lane-dependent ternary would become a branch)
    const uint32_t hi = j < 4 ? 0u : ~0u;
    const uint32_t sc = ((by & 63u) & ~hi) | (((bw & 15u) | ((by >> 6) << 4)) & hi);
    const uint32_t mn = ((bz & 63u) & ~hi) | (((bw >> 4) | ((bz >> 6) << 4)) & hi);
    d0 = __fmul_rn(f16_lo(hdr.x), static_cast<float>(sc));
    m = __fmul_rn(f16_hi(hdr.x), static_cast<float>(mn));
}

// sum q x of a lane's sub-block from the digit-plane sums S (slots 0..3) and the block's 2^(e-6)
__device__ __forceinline__ float digits_dot(const i32x4_t& S, float xs)
{
    float f = static_cast<float>(S[3]);
    f = fmaf(f, 0.0078125f, static_cast<float>(S[2]));
    f = fmaf(f, 0.0078125f, static_cast<float>(S[1]));
    f = fmaf(f, 0.0078125f, static_cast<float>(S[0]));
    return f * xs;
}

// Digits of x for the integer MFMA: per 32-value block (eight lanes) its exponent e (max |x| = f 2^e, f in [0.5, 1)), its f32
// sum, and the digit planes of X = rint(x 2^(27-e)) (|X| < 2^27): X = d1 2^21 + d2 2^14 + d3 2^7 + d4 with
// d2..d4 in 0..127 and d1 = X >> 21 in -64..63, so x = 2^(e-6) (d1 + d2 2^-7 + d3 2^-14 + d4 2^-21) to
// within 2^(e-28). Four values per lane (eight lanes per block): the four plane words (byte k = value k),
// 2^(e-6) and the block's sum.
__device__ __forceinline__ void kq_digits(const float (&xv)[4], uint32_t (&pl)[4], float& down, float& sm)
{
    float mx = fmaxf(fmaxf(fabsf(xv[0]), fabsf(xv[1])), fmaxf(fabsf(xv[2]), fabsf(xv[3])));
    sm = (xv[0] + xv[1]) + (xv[2] + xv[3]);
#pragma unroll
    for (int o = 1; o < 8; o <<= 1) {  // the 8 lanes of the block (consecutive lanes)
        mx = fmaxf(mx, __shfl_xor(mx, o));
        sm += __shfl_xor(sm, o);
    }
    int e;
    frexpf(mx, &e);  // 0 for mx = 0
    const bool finite = mx <= 3.4028234663852886e38f;
    // 2^(27-e) as two factors, each finite even for a block of subnormals (e down to -148)
    const int sh = 27 - e, sh1 = sh < 100 ? sh : 100;
    const float up1 = ldexpf(1.0f, sh1), up2 = ldexpf(1.0f, sh - sh1);
    down = finite ? ldexpf(1.0f, e - 6) : __builtin_nanf("");
    uint32_t y[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const int X = finite ? static_cast<int>(rintf((xv[k] * up1) * up2)) : 0;
        const uint32_t u = static_cast<uint32_t>(X);
        // bytes d4, d3, d2, d1 (the 7-bit fields moved to byte boundaries, d1 with its sign bits)
        y[k] = (u & 0x7Fu) | ((u << 1) & 0x7F00u) | ((u << 2) & 0x7F0000u) | ((u << 3) & 0xFF000000u);
    }
    // transpose: plane p (d1 .. d4) holds byte 3 - p of y[0..3]
    const uint32_t lo01 = __builtin_amdgcn_perm(y[1], y[0], 0x05010400u);  // y0.b0 y1.b0 y0.b1 y1.b1
    const uint32_t hi01 = __builtin_amdgcn_perm(y[1], y[0], 0x07030602u);  // y0.b2 y1.b2 y0.b3 y1.b3
    const uint32_t lo23 = __builtin_amdgcn_perm(y[3], y[2], 0x05010400u);
    const uint32_t hi23 = __builtin_amdgcn_perm(y[3], y[2], 0x07030602u);
    pl[0] = __builtin_amdgcn_perm(hi23, hi01, 0x07060302u);  // d1: byte 3 of y0..y3
    pl[1] = __builtin_amdgcn_perm(hi23, hi01, 0x05040100u);  // d2: byte 2
    pl[2] = __builtin_amdgcn_perm(lo23, lo01, 0x07060302u);  // d3: byte 1
    pl[3] = __builtin_amdgcn_perm(lo23, lo01, 0x05040100u);  // d4: byte 0
}

// The wave's four x values of super-block sb (values sb * 256 + 4 lane ..)
__device__ __forceinline__ void kq_load_x(const MatvecArgs& a, int sb, float (&xv)[4])
{
    const int v4 = sb * 64 + (threadIdx.x & 63);
    if (a.xt == SLHIP_F32) {
        const float4 t = reinterpret_cast<const float4*>(a.x)[v4];
        xv[0] = t.x; xv[1] = t.y; xv[2] = t.z; xv[3] = t.w;
    } else {
        const uint2 t = reinterpret_cast<const uint2*>(a.x)[v4];
        xv[0] = bf16_lo(t.x); xv[1] = bf16_hi(t.x); xv[2] = bf16_lo(t.y); xv[3] = bf16_hi(t.y);
    }
}

// A tile of 16 weight rows streamed through LDS by a persistent block of 16 waves. An item is one matrix's
// K segment of the tile (dual: the gate segment, then the up segment): wave w copies row w's segment -- one
// contiguous run -- with direct global -> LDS loads (no registers held), two items in flight while a third is
// computed (three LDS buffers). Long runs per wave read HBM at the rate of a linear stream; 16 rows read side
// by side in short pieces measured ~30% slower. Once an item has landed, every wave computes its share for
// all 16 rows on the matrix cores: Q4_K one super-block per wave (16 per segment), Q6_K one half super-block
// (8 per segment). x is digitized once per block for the whole K. A block takes tiles b, b + grid, ...; a
// tile's items in order, its sums kept in registers.
constexpr int kKqTileWaves = 16;
constexpr int kKqBufs = 3;  // item buffers in LDS (two landing while one is computed)

template <int FMT> struct KqGeom;
template <> struct KqGeom<SLHIP_FMT_Q4_K> {
    static constexpr int BB = 144, SEG_SB = 16;
    static constexpr int ROW = SEG_SB * BB + 16;  // LDS stride of a row's segment (padded: 580 words, banks 4n)
};
template <> struct KqGeom<SLHIP_FMT_Q6_K> {
    static constexpr int BB = 210, SEG_SB = 8;
    static constexpr int ROW = SEG_SB * BB;  // 420 words: rows start on banks 36n mod 64, distinct for n < 16
};

// LDS: x digit planes [4][K], 16 zero bytes, per 32-value block 2^(e-6) and sum, the waves' sums
// [2][waves][16], the item buffers.
template <int FMT>
static size_t kq_tile_lds(int64_t K)
{
    return static_cast<size_t>(K) * 4 + 16 + static_cast<size_t>(K / 32) * 8 + 2 * kKqTileWaves * 16 * 4 +
           static_cast<size_t>(kKqBufs) * kKqTileWaves * KqGeom<FMT>::ROW;
}

// A direct global -> LDS load of 16 bytes per lane: lane i's bytes land at lds_base + 16 i (lds_base
// wave-uniform, an LDS byte address). Written as inline assembly so that the compiler does not treat the
// loads as pending LDS writes, which makes it wait for every outstanding load before any LDS read or barrier;
// the kernel waits for them itself (wait_vmcnt), knowing which buffer each load fills.
__device__ __forceinline__ void lds_dma16(const void* src, uint32_t lds_base)
{
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(lds_base) : "m0", "memory");
}

// s_waitcnt with only a vmcnt limit (gfx9 encoding: vmcnt in bits 3:0 and 15:14, expcnt and lgkmcnt at max)
template <int V>
__device__ __forceinline__ void wait_vmcnt()
{
    __builtin_amdgcn_s_waitcnt((V & 0xF) | ((V >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// 16 bytes at LDS byte address p, which is 2-byte aligned and misaligned by mis = p % 16 (wave-uniform):
// two aligned 16-byte reads and a funnel shift.
__device__ __forceinline__ uint4 lds_read16_mis(const char* p, int mis)
{
    const uint4* b = reinterpret_cast<const uint4*>(p - mis);
    const uint4 lo = b[0], hi = b[1];
    uint32_t w[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
    if (mis & 8) {  // wave-uniform selects
#pragma unroll
        for (int i = 0; i < 6; i++) w[i] = w[i + 2];
    }
    if (mis & 4) {
#pragma unroll
        for (int i = 0; i < 5; i++) w[i] = w[i + 1];
    }
    const uint32_t sh = 8u * static_cast<uint32_t>(mis & 3);
    return make_uint4(__builtin_amdgcn_alignbyte(w[1], w[0], sh >> 3), __builtin_amdgcn_alignbyte(w[2], w[1], sh >> 3),
                      __builtin_amdgcn_alignbyte(w[3], w[2], sh >> 3), __builtin_amdgcn_alignbyte(w[4], w[3], sh >> 3));
}

template <int FMT, bool DUAL>
__global__ __launch_bounds__(64 * kKqTileWaves) void matvec_kq_tile(MatvecArgs a, int nseg)
{
    using G = KqGeom<FMT>;
    constexpr bool Q6 = FMT == SLHIP_FMT_Q6_K;
    constexpr int SEG = G::SEG_SB * G::BB;         // bytes of a row's segment
    constexpr int UNITS = SEG / 16;                // 16-byte units of it
    constexpr int LOADS = (UNITS + 63) / 64;       // load instructions per item and wave
    extern __shared__ uint32_t smem[];
    const int K = static_cast<int>(a.K);
    char* lds = reinterpret_cast<char*>(smem);
    const uint32_t zero_off = 4u * static_cast<uint32_t>(K);                 // 16 zero bytes after the planes
    float* xscale = reinterpret_cast<float*>(lds + zero_off + 16);            // [K / 32] 2^(e-6)
    float* xsum = xscale + K / 32;                                             // [K / 32]
    float* red = xsum + K / 32;                                                // [2][waves][16]
    char* wbuf = reinterpret_cast<char*>(red + 2 * kKqTileWaves * 16);        // [bufs][waves][G::ROW]
    const int lane = threadIdx.x & 63, wave = wave_id();
    const int n = lane & 15, q = lane >> 4;
    const int64_t tiles = (a.N + 15) / 16;

    // item (tile t, segment s) -> LDS buffer: wave w's row segment, 16-byte units on consecutive lanes
    auto issue = [&](int64_t t, int s, int buf) {
        const int64_t row0 = t * 16 + wave;
        const int64_t row = row0 < a.N ? row0 : a.N - 1;
        const bool up = DUAL && (s & 1);
        const int64_t off = row * a.wrow + static_cast<int64_t>(DUAL ? s >> 1 : s) * SEG;
        char* dst = wbuf + (buf * kKqTileWaves + wave) * G::ROW;
#pragma unroll
        for (int i = 0; i < LOADS; i++) {
            const int u = lane + 64 * i;
            if (64 * i + 64 > UNITS && u >= UNITS) continue;  // the last instruction's spare lanes
            lds_dma16((up ? a.wu : a.wg) + off + 16 * u,
                      __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(reinterpret_cast<uintptr_t>(dst + 1024 * i))));
        }
    };
    auto next_item = [&](int64_t& t, int& s) {
        if (++s == nseg) {
            s = 0;
            t += gridDim.x;
        }
    };

    int64_t lt = blockIdx.x;  // the item whose loads go out next
    int ls = 0;
    for (int b = 0; b < kKqBufs - 1; b++) {  // prologue: the first two items (past the end: the last tile again)
        issue(lt < tiles ? lt : tiles - 1, lt < tiles ? ls : 0, b);
        next_item(lt, ls);
    }
    // x digitized once: per 32-value block its exponent, sum and digit planes [4][K]
    for (int v4 = threadIdx.x; v4 < K / 4; v4 += 64 * kKqTileWaves) {  // whole waves (K % 256 == 0)
        float xv[4];
        kq_load_x(a, v4 / 64, xv);  // the lane's four values (v4 == 64 sb + lane)
        uint32_t pl[4];
        float down, sm;
        kq_digits(xv, pl, down, sm);
#pragma unroll
        for (int p = 0; p < 4; p++) reinterpret_cast<uint32_t*>(lds + p * K)[v4] = pl[p];
        if ((lane & 7) == 0) {
            xscale[v4 / 8] = down;
            xsum[v4 / 8] = sm;
        }
    }
    if (threadIdx.x < 4) smem[zero_off / 4 + threadIdx.x] = 0u;

    const int plane = n - 4 * q;  // this lane's slot n is digit plane `plane` of K-group q, or a zero slot
    const bool has_plane = plane >= 0 && plane < 4;
    const uint32_t a_base = has_plane ? static_cast<uint32_t>(plane * K) : zero_off;
    const uint32_t a_step = has_plane ? 1u : 0u;
    auto a_op = [&](int v) {  // A operand: 16 digits of plane `plane` from value v (or zeros)
        return as_i32x4(*reinterpret_cast<const uint4*>(lds + a_base + static_cast<uint32_t>(v) * a_step));
    };
    float accg = 0.0f, accu = 0.0f;

    // Q4_K: super-block `wave` of the segment. Lane group q holds code group q (sub-blocks 2q, 2q + 1: low and
    // high nibbles) of row n; two MFMAs per sub-block.
    auto compute_q4k = [&](const char* bufp, int seg, float& acc) {
        const int sb = seg * G::SEG_SB + wave;
        const char* row = bufp + n * G::ROW + wave * G::BB;
        const uint4 h = *reinterpret_cast<const uint4*>(row);
        const uint4 c0 = *reinterpret_cast<const uint4*>(row + 16 + 32 * q);
        const uint4 c1 = *reinterpret_cast<const uint4*>(row + 32 + 32 * q);
#pragma unroll
        for (int hi = 0; hi < 2; hi++) {
            i32x4_t c = {0, 0, 0, 0};
#pragma unroll
            for (int i = 0; i < 2; i++) {  // the sub-block's values 0-15, 16-31
                const uint4& w = i ? c1 : c0;
                const uint32_t S = hi ? 4 : 0;
                const uint4 b = make_uint4((w.x >> S) & 0x0F0F0F0Fu, (w.y >> S) & 0x0F0F0F0Fu,
                                           (w.z >> S) & 0x0F0F0F0Fu, (w.w >> S) & 0x0F0F0F0Fu);
                c = __builtin_amdgcn_mfma_i32_16x16x64_i8(a_op(sb * 256 + 64 * q + 32 * hi + 16 * i), as_i32x4(b), c,
                                                          0, 0, 0);
            }
            const int j = 2 * q + hi;
            float d0, m;
            q4k_scales(h, j, d0, m);
            acc = fmaf(d0, digits_dot(c, xscale[sb * 8 + j]), acc);
            acc = fmaf(-m, xsum[sb * 8 + j], acc);
        }
    };
    // Q6_K: half `hf` of super-block `wave / 2` (values 128 hf .. +127). In MFMA m lane group q takes the 16
    // values 128 hf + 32 k + 16 lh + 0..15, k = 2m + (q >> 1), lh = q & 1: low (k < 2) or high nibbles of
    // ql[64 hf + 32 (k & 1) + 16 lh ..] with bits 2k of qh[128 + 32 hf + 16 lh ..]; scale sc[8 hf + 2k + lh].
    auto compute_q6k = [&](const char* bufp, int seg, float& acc) {
        const int sbl = wave >> 1, hf = wave & 1, lh = q & 1;
        const int sb = seg * G::SEG_SB + sbl;
        const char* row = bufp + n * G::ROW + sbl * G::BB;
        const int mis = (sbl * G::BB) & 15;  // the super-block's offset from 16-byte alignment (rows are aligned)
        const uint4 ql = lds_read16_mis(row + 64 * hf + 32 * (q >> 1) + 16 * lh, mis);
        const uint4 qh = lds_read16_mis(row + 128 + 32 * hf + 16 * lh, mis);
        const float d = static_cast<float>(*reinterpret_cast<const _Float16*>(row + 208));
#pragma unroll
        for (int m = 0; m < 2; m++) {
            const int k = 2 * m + (q >> 1);
            const uint32_t hs = 2u * static_cast<uint32_t>(k);
            // q - 32 as a signed byte: (q + 128) - 32 cannot borrow across bytes, then the top bit flipped back
            auto code = [&](uint32_t l, uint32_t h) {
                const uint32_t q = ((m ? l >> 4 : l) & 0x0F0F0F0Fu) | (((h >> hs) & 0x03030303u) << 4);
                return ((q | 0x80808080u) - 0x20202020u) ^ 0x80808080u;
            };
            const uint4 b = make_uint4(code(ql.x, qh.x), code(ql.y, qh.y), code(ql.z, qh.z), code(ql.w, qh.w));
            const int v = sb * 256 + 128 * hf + 32 * k + 16 * lh;
            i32x4_t c = {0, 0, 0, 0};
            c = __builtin_amdgcn_mfma_i32_16x16x64_i8(a_op(v), as_i32x4(b), c, 0, 0, 0);
            const float sc = static_cast<float>(*reinterpret_cast<const int8_t*>(row + 192 + 8 * hf + 2 * k + lh));
            acc = fmaf(__fmul_rn(d, sc), digits_dot(c, xscale[v / 32]), acc);
        }
    };

    int64_t t = blockIdx.x;
    int s = 0, buf = 0;
    while (t < tiles) {  // block-uniform
        // this item's loads went out two items ago; the next item's may stay out
        wait_vmcnt<LOADS>();
        __syncthreads();  // the item is in LDS (every wave's row), and every wave is done with the buffer of
                          // the previous item, which now takes the item two ahead
        {
            const int pb = buf == 0 ? kKqBufs - 1 : buf - 1;
            issue(lt < tiles ? lt : tiles - 1, lt < tiles ? ls : 0, pb);
            next_item(lt, ls);
        }
        const char* bufp = wbuf + buf * kKqTileWaves * G::ROW;
        const int seg = DUAL ? s >> 1 : s;
        float& acc = DUAL && (s & 1) ? accu : accg;
        if (Q6)
            compute_q6k(bufp, seg, acc);
        else
            compute_q4k(bufp, seg, acc);
        if (s + 1 == nseg) {  // the tile is complete: the four lane groups of a row, then the waves
            float g = accg, u = accu;
            g += __shfl_xor(g, 16);
            g += __shfl_xor(g, 32);
            u += __shfl_xor(u, 16);
            u += __shfl_xor(u, 32);
            if (q == 0) {
                red[wave * 16 + n] = g;
                red[(kKqTileWaves + wave) * 16 + n] = u;
            }
            __syncthreads();
            const int64_t n0 = t * 16;
            if (wave == 0 && lane < 16 && n0 + n < a.N) {
                float ag[1] = {0.0f}, au[1] = {0.0f};
                for (int w = 0; w < kKqTileWaves; w++) {
                    ag[0] += red[w * 16 + n];
                    au[0] += red[(kKqTileWaves + w) * 16 + n];
                }
                store_row<1, DUAL>(a, n0 + n, ag, au);
            }
            accg = accu = 0.0f;
        }
        next_item(t, s);
        buf = buf + 1 == kKqBufs ? 0 : buf + 1;
    }
    wait_vmcnt<0>();  // no load may still be landing in LDS when the block ends
}

// ---- host dispatch --------------------------------------------------------------------------------

static int env_int(const char* name, int dflt)
{
    const char* s = getenv(name);
    return s && *s ? atoi(s) : dflt;
}

template <int WT, int TT, bool DUAL>
static int launch_nv(const MatvecArgs& a, int nv, int wpr, hipStream_t st)
{
    const int rpb = (kMvThreads / 64) / wpr;
    const dim3 grid(static_cast<unsigned>((a.N + rpb - 1) / rpb));
    const size_t lds = static_cast<size_t>(TT) * a.K * 4;
    switch (nv) {
    case 1: matvec_dense<WT, TT, 1, DUAL><<<grid, kMvThreads, lds, st>>>(a, wpr); break;
    case 2: matvec_dense<WT, TT, 2, DUAL><<<grid, kMvThreads, lds, st>>>(a, wpr); break;
    case 4: matvec_dense<WT, TT, 4, DUAL><<<grid, kMvThreads, lds, st>>>(a, wpr); break;
    case 8: matvec_dense<WT, TT, 8, DUAL><<<grid, kMvThreads, lds, st>>>(a, wpr); break;
    default: return fail(SLHIP_ERR_INVALID, "internal: matvec vector count %d", nv);
    }
    return check_launch("matvec_dense");
}

template <int WT, bool DUAL>
static int launch_tt(const MatvecArgs& a, int tt, int nv, int wpr, hipStream_t st)
{
    switch (tt) {
    case 1: return launch_nv<WT, 1, DUAL>(a, nv, wpr, st);
    case 2: return launch_nv<WT, 2, DUAL>(a, nv, wpr, st);
    case 4: return launch_nv<WT, 4, DUAL>(a, nv, wpr, st);
    case 8: return launch_nv<WT, 8, DUAL>(a, nv, wpr, st);
    default: return fail(SLHIP_ERR_INVALID, "internal: matvec token tile %d", tt);
    }
}

// Activation rows per launch: up to 8, within 64 KiB of staged f32 x.
static int token_tile(int64_t T, int64_t K)
{
    int tt = 8;
    while (tt > 1 && (tt / 2 >= T || static_cast<int64_t>(tt) * K * 4 > 65536)) tt /= 2;
    return tt;
}

template <int SK, int NT>
static void launch_mfma_lds(const MatvecArgs& a, bool dual, hipStream_t st)
{
    const dim3 grid(static_cast<unsigned>((a.N + 16 * NT - 1) / (16 * NT)));
    if (a.xt == SLHIP_F32) {
        if (dual) matvec_mfma_lds<true, true, SK, NT><<<grid, 64 * kMmWaves, 0, st>>>(a);
        else matvec_mfma_lds<false, true, SK, NT><<<grid, 64 * kMmWaves, 0, st>>>(a);
    } else {
        if (dual) matvec_mfma_lds<true, false, SK, NT><<<grid, 64 * kMmWaves, 0, st>>>(a);
        else matvec_mfma_lds<false, false, SK, NT><<<grid, 64 * kMmWaves, 0, st>>>(a);
    }
}

// Weight stage of the LDS-staged MFMA kernel (SLHIP_MATVEC_MFMA_SK: 256 or 512 values; 0 = operands
// loaded straight from global memory, also used when K is not a multiple of the stage) and 16-row tiles
// per block (SLHIP_MATVEC_MFMA_NT: 1 or 2; one with the 512-value stage).
static int mfma_stage() { return env_int("SLHIP_MATVEC_MFMA_SK", 256); }
// Default: one tile (finer blocks spread the 16-row tiles more evenly over the CUs), two only for f32 x above
// 12 tokens, where each x fragment's three-way bf16 split then feeds twice the weights. Measured at
// 14336 x 4096 (dual, us, one tile / two): f32 x T = 8 46.3 / 48.4, T = 12 47.7 / 48.9, T = 16 51.1 / 50.0;
// bf16 x T = 8 39.8 / 47.0, T = 16 42.1 / 47.7.
static int mfma_tiles(int64_t T, int xt)
{
    const int nt = env_int("SLHIP_MATVEC_MFMA_NT", 0);
    return nt == 1 || nt == 2 ? nt : (xt == SLHIP_F32 && T > 12 ? 2 : 1);
}

static int run_mfma(MatvecArgs a, bool dual, hipStream_t st)
{
    const dim3 grid(static_cast<unsigned>((a.N + 15) / 16));
    const int sk = mfma_stage(), nt = mfma_tiles(a.T, a.xt);
    for (int64_t t0 = 0; t0 < a.T; t0 += 16) {
        a.t0 = t0;
        if (sk == 512 && a.K % 512 == 0) {
            launch_mfma_lds<512, 1>(a, dual, st);  // two tiles would take 133 KB of LDS per block
        } else if (sk == 256 && a.K % 256 == 0) {
            nt == 2 ? launch_mfma_lds<256, 2>(a, dual, st) : launch_mfma_lds<256, 1>(a, dual, st);
        } else if (a.xt == SLHIP_F32) {
            if (dual) matvec_mfma<true, true><<<grid, 64 * kMmWaves, 0, st>>>(a);
            else matvec_mfma<false, true><<<grid, 64 * kMmWaves, 0, st>>>(a);
        } else {
            if (dual) matvec_mfma<true, false><<<grid, 64 * kMmWaves, 0, st>>>(a);
            else matvec_mfma<false, false><<<grid, 64 * kMmWaves, 0, st>>>(a);
        }
        const int r = check_launch("matvec_mfma");
        if (r != SLHIP_OK) return r;
    }
    return SLHIP_OK;
}

// Tokens from which bf16 weights take the matrix cores (SLHIP_MATVEC_MFMA_MIN_T; 0 disables): below it the
// VALU kernel is already at the HBM rate. Measured at 14336 x 4096 (dual, us, VALU / matrix cores) at T = 2:
// f32 x 41.6 / 44.3, bf16 x 45.1 / 40.0; at T = 3: f32 x 51.5 / 43.6.
static int mfma_min_tokens(int xt) { return env_int("SLHIP_MATVEC_MFMA_MIN_T", xt == SLHIP_BF16 ? 2 : 3); }

template <int WT>
static int run_dense(MatvecArgs a, bool dual, hipStream_t st)
{
    if constexpr (WT == SLHIP_BF16) {
        const int mt = mfma_min_tokens(a.xt);
        if (mt > 0 && a.T >= mt && a.K % 64 == 0) return run_mfma(a, dual, st);
    }
    constexpr int E = Vec<WT>::N;
    const int64_t nvr = a.K / E;
    int wpr = 1;
    while (wpr < 8 && nvr > static_cast<int64_t>(8) * 64 * wpr) wpr *= 2;
    const int forced = env_int("SLHIP_MATVEC_WPR", 0);
    if ((forced == 1 || forced == 2 || forced == 4 || forced == 8) && nvr <= static_cast<int64_t>(8) * 64 * forced)
        wpr = forced;
    const int64_t per = (nvr + 64 * wpr - 1) / (64 * wpr);
    const int nv = per <= 1 ? 1 : per <= 2 ? 2 : per <= 4 ? 4 : 8;
    const int tt = token_tile(a.T, a.K);
    for (int64_t t0 = 0; t0 < a.T; t0 += tt) {
        a.t0 = t0;
        const int r = dual ? launch_tt<WT, true>(a, tt, nv, wpr, st) : launch_tt<WT, false>(a, tt, nv, wpr, st);
        if (r != SLHIP_OK) return r;
    }
    return SLHIP_OK;
}

// Values and bytes per block of the quantized weight formats; {0, 0} for the others.
struct QGeom {
    int bs, bb;
};
static QGeom quant_geom(int fmt)
{
    switch (fmt) {
    case SLHIP_FMT_Q8_0: return {32, 34};
    case SLHIP_FMT_Q4_0: return {32, 18};
    case SLHIP_FMT_Q4_1: return {32, 20};
    case SLHIP_FMT_Q5_0: return {32, 22};
    case SLHIP_FMT_Q5_1: return {32, 24};
    case SLHIP_FMT_Q4_K: return {256, 144};
    case SLHIP_FMT_Q5_K: return {256, 176};
    case SLHIP_FMT_Q6_K: return {256, 210};
    case SLHIP_FMT_Q2_K: return {256, 84};
    case SLHIP_FMT_Q3_K: return {256, 110};
    default: return {0, 0};
    }
}

constexpr size_t kMaxLds = 160 * 1024;  // gfx950 LDS per workgroup

static int device_cus()
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

static size_t quant_lds(int tt, int64_t K, int64_t wrow, bool dual)
{
    const int64_t rowb = (wrow + 15) / 16 * 16;  // a row image, padded to whole 16-byte chunks
    return static_cast<size_t>(kMqThreads / 64) * (dual ? 2 : 1) * rowb + static_cast<size_t>(tt) * (K / 32) * 36 * 4 +
           static_cast<size_t>(tt) * (K / 32) * 4;
}

template <class Kern>
static int allow_lds(Kern kernel, size_t lds)
{
    if (lds <= 65536) return SLHIP_OK;
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
    return e == hipSuccess ? SLHIP_OK : fail(SLHIP_ERR_HIP, "matvec: %zu bytes of LDS refused: %s", lds, hipGetErrorString(e));
}

template <int FMT, int TT, int CH, bool DUAL, int U = 16>
static int launch_quant(const MatvecArgs& a, hipStream_t st)
{
    const size_t lds = quant_lds(TT, a.K, a.wrow, DUAL);
    auto kernel = matvec_quant<FMT, TT, CH, DUAL, U>;
    const int r = allow_lds(kernel, lds);
    if (r != SLHIP_OK) return r;
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, kMqThreads, lds) != hipSuccess || per_cu < 1)
        per_cu = 1;
    const int64_t blocks = (a.N + kMqThreads / 64 - 1) / (kMqThreads / 64);
    const int64_t resident = static_cast<int64_t>(device_cus()) * per_cu;
    const dim3 grid(static_cast<unsigned>(blocks < resident ? blocks : resident));
    kernel<<<grid, kMqThreads, lds, st>>>(a);
    return check_launch("matvec_quant");
}

template <int FMT, int TT, bool DUAL>
static int quant_ch(const MatvecArgs& a, int ch, hipStream_t st)
{
    if constexpr (FMT == SLHIP_FMT_Q6_K || FMT == SLHIP_FMT_Q3_K || FMT == SLHIP_FMT_Q2_K) {
        // rows not 16-byte multiples (210, 110 or 84 bytes per 256 values): narrower staging loads
        if (a.wrow % 16 != 0) {
            return a.wrow % 8 == 0   ? launch_quant<FMT, TT, 8, DUAL, 8>(a, st)
                   : a.wrow % 4 == 0 ? launch_quant<FMT, TT, 8, DUAL, 4>(a, st)
                                     : launch_quant<FMT, TT, 8, DUAL, 2>(a, st);
        }
    }
    switch (ch) {
    case 4: return launch_quant<FMT, TT, 4, DUAL>(a, st);
    case 8: return launch_quant<FMT, TT, 8, DUAL>(a, st);
    case 12: return launch_quant<FMT, TT, 12, DUAL>(a, st);
    default: return launch_quant<FMT, TT, 16, DUAL>(a, st);
    }
}

template <int FMT, bool DUAL>
static int quant_tt(const MatvecArgs& a, int tt, int ch, hipStream_t st)
{
    switch (tt) {
    case 1: return quant_ch<FMT, 1, DUAL>(a, ch, st);
    case 2: return quant_ch<FMT, 2, DUAL>(a, ch, st);
    case 4: return quant_ch<FMT, 4, DUAL>(a, ch, st);
    default: return quant_ch<FMT, 8, DUAL>(a, ch, st);
    }
}

template <int FMT, bool DUAL>
static int launch_kq_tile(const MatvecArgs& a, hipStream_t st)
{
    const size_t lds = kq_tile_lds<FMT>(a.K);
    auto kernel = matvec_kq_tile<FMT, DUAL>;
    const int r = allow_lds(kernel, lds);
    if (r != SLHIP_OK) return r;
    const int nseg = static_cast<int>(a.K / 256) / KqGeom<FMT>::SEG_SB * (DUAL ? 2 : 1);
    const int64_t tiles = (a.N + 15) / 16;
    const int64_t grid = tiles < device_cus() ? tiles : device_cus();
    kernel<<<dim3(static_cast<unsigned>(grid)), 64 * kKqTileWaves, lds, st>>>(a, nseg);
    return check_launch("matvec_kq_tile");
}

// Tokens from which the 32-value block formats (Q4_0, Q8_0, Q4_1, Q5_0, Q5_1) take the matrix cores
// (SLHIP_MATVEC_MQ_MIN_T; 0 disables). Measured with matvec_mq2 at [14336, 4096] (dual, f32 x, us, VALU /
// matrix cores): Q4_0 T = 2 28.1 / 44.1, T = 3 56.8 / 45.0; Q8_0 T = 2 32.5 / 46.2, T = 3 58.0 / 48.1.
static int mq_min_tokens() { return env_int("SLHIP_MATVEC_MQ_MIN_T", 3); }
// The same for the K-quants (SLHIP_MATVEC_KQ_MIN_T). With matvec_mq2, measured dual at [14336, 4096], f32 x
// (us, VALU / matrix cores): Q4_K T = 2 30.6 / 46.5, T = 3 60.6 / 49.0; Q6_K T = 3 94.2 / 62.5; Q3_K T = 3
// 78.0 / 61.2 (the VALU kernel's passes hold 2 and then 4 tokens): from three tokens.
static int kq_min_tokens() { return env_int("SLHIP_MATVEC_KQ_MIN_T", 3); }

// The several-token kernel with the stage moved straight to LDS and each lane scaling its own row
// (matvec_mq.hpp, matvec_mq_*.hip); SLHIP_MATVEC_MQ2=0 keeps matvec_mfma_q below, which also takes the
// launches mq2 does not fit.
int run_mq2_part0(int fmt, const MatvecArgs& a, bool dual, hipStream_t st);
int run_mq2_part1(int fmt, const MatvecArgs& a, bool dual, hipStream_t st);
int run_mq2_part2(int fmt, const MatvecArgs& a, bool dual, hipStream_t st);

static int run_mq2_any(int fmt, const MatvecArgs& a, bool dual, hipStream_t st)
{
    switch (fmt) {
    case SLHIP_FMT_Q4_0:
    case SLHIP_FMT_Q8_0:
    case SLHIP_FMT_Q4_1:
    case SLHIP_FMT_Q5_0:
    case SLHIP_FMT_Q5_1: return run_mq2_part0(fmt, a, dual, st);
    case SLHIP_FMT_Q4_K:
    case SLHIP_FMT_Q5_K: return run_mq2_part1(fmt, a, dual, st);
    default: return run_mq2_part2(fmt, a, dual, st);
    }
}

template <int FMT>
static int run_mfma_q(MatvecArgs a, bool dual, hipStream_t st)
{
    if (env_int("SLHIP_MATVEC_MQ2", 1)) {
        const int r = run_mq2_any(FMT, a, dual, st);
        if (r != SLHIP_ERR_UNSUPPORTED) return r;
    }
    const dim3 grid(static_cast<unsigned>((a.N + 15) / 16));
    for (int64_t t0 = 0; t0 < a.T; t0 += 16) {
        a.t0 = t0;
        if (a.xt == SLHIP_F32) {
            if (dual) matvec_mfma_q<FMT, true, true><<<grid, 64 * kMqWaves, 0, st>>>(a);
            else matvec_mfma_q<FMT, false, true><<<grid, 64 * kMqWaves, 0, st>>>(a);
        } else {
            if (dual) matvec_mfma_q<FMT, true, false><<<grid, 64 * kMqWaves, 0, st>>>(a);
            else matvec_mfma_q<FMT, false, false><<<grid, 64 * kMqWaves, 0, st>>>(a);
        }
        const int r = check_launch("matvec_mfma_q");
        if (r != SLHIP_OK) return r;
    }
    return SLHIP_OK;
}

template <int FMT>
static int run_quant(MatvecArgs a, bool dual, hipStream_t st)
{
    if constexpr (FMT == SLHIP_FMT_Q4_0 || FMT == SLHIP_FMT_Q8_0 || FMT == SLHIP_FMT_Q4_1 || FMT == SLHIP_FMT_Q5_0 ||
                  FMT == SLHIP_FMT_Q5_1 || FMT == SLHIP_FMT_Q4_K || FMT == SLHIP_FMT_Q5_K || FMT == SLHIP_FMT_Q6_K ||
                  FMT == SLHIP_FMT_Q2_K || FMT == SLHIP_FMT_Q3_K) {
        // several tokens: the matrix-core kernel, when K splits into whole stages (and the rows into its loads)
        const int mt = Fmt<FMT>::K ? kq_min_tokens() : mq_min_tokens();
        const uintptr_t al = reinterpret_cast<uintptr_t>(a.wg) | reinterpret_cast<uintptr_t>(a.wu);
        if (mt > 0 && a.T >= mt && a.K % (MqGeom<FMT>::SKB * 32) == 0 && al % MqGeom<FMT>::UB == 0)
            return run_mfma_q<FMT>(a, dual, st);
    }
    if constexpr (FMT == SLHIP_FMT_Q4_K || FMT == SLHIP_FMT_Q6_K) {
        // one token: the matrix-core kernel, when K splits into whole segments and its LDS fits
        if (a.T == 1 && a.K % (256 * KqGeom<FMT>::SEG_SB) == 0 && kq_tile_lds<FMT>(a.K) <= kMaxLds &&
            env_int("SLHIP_KQ_MFMA", 1))
            return dual ? launch_kq_tile<FMT, true>(a, st) : launch_kq_tile<FMT, false>(a, st);
    }
    int tt = Fmt<FMT>::K && dual ? 4 : 8;  // the K-quant sub-block decode at 8 tokens of a pair spills
    while (tt > 1 && (tt / 2 >= a.T || quant_lds(tt, a.K, a.wrow, dual) > kMaxLds)) tt /= 2;
    if (quant_lds(tt, a.K, a.wrow, dual) > kMaxLds)
        return fail(SLHIP_ERR_UNSUPPORTED, "matvec: K = %lld does not fit in LDS for this format", static_cast<long long>(a.K));
    const int64_t per_lane = ((dual ? 2 : 1) * (a.wrow / 16) + 63) / 64;
    const int ch = per_lane <= 4 ? 4 : per_lane <= 8 ? 8 : per_lane <= 12 ? 12 : 16;
    for (int64_t t0 = 0; t0 < a.T; t0 += tt) {
        a.t0 = t0;
        const int r = dual ? quant_tt<FMT, true>(a, tt, ch, st) : quant_tt<FMT, false>(a, tt, ch, st);
        if (r != SLHIP_OK) return r;
    }
    return SLHIP_OK;
}

// Whether a (dual) matvec over rows of K values of `fmt` can run: for the block formats, whether one token's
// staged x and the row images of a block's waves fit in LDS.
bool matvec_fits(int fmt, int64_t K, bool dual)
{
    const QGeom qg = quant_geom(fmt);
    if (qg.bs == 0) return true;
    if (K % qg.bs != 0) return false;
    return quant_lds(1, K, K / qg.bs * qg.bb, dual) <= kMaxLds;
}

static int matvec_common(int fmt, int dtype_x, int dtype_y, const void* x, int64_t x_stride, int64_t T, int64_t K,
                         const void* wg, const void* wu, int64_t N, void* y, int64_t y_stride, int act, bool dual,
                         slhip_stream stream, const float* bias = nullptr)
{
    const char* name = dual ? "dual_matvec" : "matvec";
    if (T < 0 || K < 0 || N < 0) return fail(SLHIP_ERR_INVALID, "%s: negative shape", name);
    if (T == 0 || N == 0) return SLHIP_OK;
    if (K == 0) return fail(SLHIP_ERR_INVALID, "%s: K must be positive", name);
    if (!x || !wg || !y || (dual && !wu)) return fail(SLHIP_ERR_INVALID, "%s: null pointer", name);
    if (dual && (act < SLHIP_ACT_SILU || act > SLHIP_ACT_GELU_ERF))
        return fail(SLHIP_ERR_INVALID, "%s: bad activation %d", name, act);
    if ((dtype_x != SLHIP_F32 && dtype_x != SLHIP_BF16) || (dtype_y != SLHIP_F32 && dtype_y != SLHIP_BF16))
        return fail(SLHIP_ERR_UNSUPPORTED, "%s: activations and outputs are f32 or bf16", name);
    if (x_stride < K || y_stride < N) return fail(SLHIP_ERR_INVALID, "%s: a row stride is smaller than the row", name);
    const bool dense = fmt == SLHIP_FMT_F32 || fmt == SLHIP_FMT_F16 || fmt == SLHIP_FMT_BF16;
    const QGeom qg = quant_geom(fmt);
    if (!dense && qg.bs == 0) return fail(SLHIP_ERR_UNSUPPORTED, "%s: weight format %d not supported", name, fmt);
    if (dense ? K % 8 != 0 : K % 256 != 0)
        return fail(SLHIP_ERR_UNSUPPORTED, "%s: K = %lld must be a multiple of %d for this weight format", name,
                    static_cast<long long>(K), dense ? 8 : 256);
    if (!aligned16(wg) || (dual && !aligned16(wu)) || !aligned16(x) || (x_stride % 8) != 0)
        return fail(SLHIP_ERR_UNSUPPORTED, "%s: weights and x rows must be 16-byte aligned (x stride a multiple of 8)",
                    name);
    if (dense && static_cast<int64_t>(K) * 4 > 65536)
        return fail(SLHIP_ERR_UNSUPPORTED, "%s: K = %lld above the staged-activation limit 16384", name,
                    static_cast<long long>(K));
    if (N > 0x7FFFFFFF || T > 0x7FFFFFFF) return fail(SLHIP_ERR_UNSUPPORTED, "%s: shape too large", name);
    const int64_t wrow = dense ? K * (fmt == SLHIP_FMT_F32 ? 4 : 2) : K / qg.bs * qg.bb;
    if (wrow % 16 != 0 && fmt != SLHIP_FMT_Q6_K && fmt != SLHIP_FMT_Q2_K && fmt != SLHIP_FMT_Q3_K)
        // (only the K-quants of 210, 84 and 110 bytes per 256 values can be)
        return fail(SLHIP_ERR_UNSUPPORTED, "%s: rows of %lld bytes are not a multiple of 16 for this weight format",
                    name, static_cast<long long>(wrow));
    MatvecArgs a{x, x_stride, static_cast<const char*>(wg), static_cast<const char*>(wu), wrow, y, y_stride,
                 T, K, N, 0, dtype_x, dtype_y, act, dual ? nullptr : bias};
    hipStream_t st = to_stream(stream);
    switch (fmt) {
    case SLHIP_FMT_F32: return run_dense<SLHIP_F32>(a, dual, st);
    case SLHIP_FMT_F16: return run_dense<SLHIP_F16>(a, dual, st);
    case SLHIP_FMT_BF16: return run_dense<SLHIP_BF16>(a, dual, st);
    case SLHIP_FMT_Q8_0: return run_quant<SLHIP_FMT_Q8_0>(a, dual, st);
    case SLHIP_FMT_Q4_0: return run_quant<SLHIP_FMT_Q4_0>(a, dual, st);
    case SLHIP_FMT_Q4_1: return run_quant<SLHIP_FMT_Q4_1>(a, dual, st);
    case SLHIP_FMT_Q5_0: return run_quant<SLHIP_FMT_Q5_0>(a, dual, st);
    case SLHIP_FMT_Q5_1: return run_quant<SLHIP_FMT_Q5_1>(a, dual, st);
    case SLHIP_FMT_Q4_K: return run_quant<SLHIP_FMT_Q4_K>(a, dual, st);
    case SLHIP_FMT_Q5_K: return run_quant<SLHIP_FMT_Q5_K>(a, dual, st);
    case SLHIP_FMT_Q2_K: return run_quant<SLHIP_FMT_Q2_K>(a, dual, st);
    case SLHIP_FMT_Q3_K: return run_quant<SLHIP_FMT_Q3_K>(a, dual, st);
    default: return run_quant<SLHIP_FMT_Q6_K>(a, dual, st);
    }
}

}  // namespace slhip

using namespace slhip;

extern "C" SLHIP_API int slhip_matvec(int fmt, int dtype_x, int dtype_y, const void* x, int64_t x_stride, int64_t T,
                                      int64_t K, const void* w, int64_t N, void* y, int64_t y_stride,
                                      slhip_stream stream)
{
    return matvec_common(fmt, dtype_x, dtype_y, x, x_stride, T, K, w, nullptr, N, y, y_stride, 0, false, stream);
}

extern "C" SLHIP_API int slhip_matvec_bias(int fmt, int dtype_x, int dtype_y, const void* x, int64_t x_stride, int64_t T,
                                           int64_t K, const void* w, int64_t N, const float* bias, void* y,
                                           int64_t y_stride, slhip_stream stream)
{
    return matvec_common(fmt, dtype_x, dtype_y, x, x_stride, T, K, w, nullptr, N, y, y_stride, 0, false, stream, bias);
}

extern "C" SLHIP_API int slhip_dual_matvec(int act, int fmt, int dtype_x, int dtype_y, const void* x, int64_t x_stride,
                                           int64_t T, int64_t K, const void* w_gate, const void* w_up, int64_t N,
                                           void* y, int64_t y_stride, slhip_stream stream)
{
    return matvec_common(fmt, dtype_x, dtype_y, x, x_stride, T, K, w_gate, w_up, N, y, y_stride, act, true, stream);
}
