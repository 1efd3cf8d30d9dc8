#pragma once
// The several-token (dual) matvec on GGUF block-format weights with f32 or bf16 activations (the float-rows
// numerics: the MatMul carries f32_activations, or its row count is outside the integer-dot rule), on the bf16
// matrix cores: matvec_mq2.
//
// A block of 8 waves takes a 16-row tile (a gate/up pair of tiles) and 16 tokens. Stages of SKB 32-value
// blocks of the tile's rows move HBM -> LDS by global_load_lds (double-buffered; one vmcnt(0) ahead of the
// barrier that publishes a stage), at a row pitch of 32 mod 64 bytes; each wave takes BPW blocks of a stage.
// v_mfma_f32_16x16x32_bf16 multiplies the tokens' x (A: lane l holds token l % 16, values 8 (l / 16) .. + 7;
// f32 x as three bf16 parts h + m + l == x exactly, bf16 x as is) with the block's codes as exact bf16 (B:
// lane l holds row l % 16, the same values), so lane l's sums are tokens 4 (l / 16) + i of row l % 16: each
// lane decodes its own row's block scale once and scales with one fma per output. Formats whose blocks hold
// two 16-value scale groups (Q6_K, Q3_K, Q2_K) take two chains, the other half's codes masked to zero. The
// block minimum terms (Q4_K / Q5_K -dmin mn sum(x), Q4_1 / Q5_1 +m sum(x), Q2_K -dmin m per half) of a wave's
// 4 blocks are a 16 x 16 x 4 product (tokens x blocks . blocks x rows): one v_mfma_f32_16x16x4f32 per matrix
// (two for Q2_K's halves) per stage. The waves' partial sums meet in LDS at the end.
//
// Arithmetic against the reference (MatMulOp's f32 dot of dequantized rows): every product code x part is
// exact and the sums are f32, so the result is the f32 evaluation of sum(scale * code * x) + min terms in
// another order: within f32 accumulation of those terms.
#include "lds_dma.hpp"
#include "mq.hpp"

namespace slhip {

constexpr int kMq2Waves = 8;

// The multipliers of block sj (32 values) of a row image, for the value halves (a0: values 0..15, a1:
// 16..31; equal for the 32-value scale formats), and its minimum coefficients per half (m0, m1; the min term
// is m * sum(x) over the half, or over the whole block with m0 when the format has one minimum per block).
// row: the row's stage bytes; sbo: the K-quant super-block's first byte in it; off: a 32-value block's first
// byte. Layouts of Quant.cs:242-405 and Quant.KQuants.cs (ggml's).
template <int FMT>
__device__ __forceinline__ void mq2_scales(const uint8_t* row, int sbo, int sj, int off, float& a0, float& a1, float& m0,
                                           float& m1)
{
    auto h16 = [&](int o) { return static_cast<float>(*reinterpret_cast<const _Float16*>(row + o)); };
    auto u16 = [&](int o) { return static_cast<uint32_t>(*reinterpret_cast<const uint16_t*>(row + o)); };
    m0 = m1 = 0.0f;
    if constexpr (FMT == SLHIP_FMT_Q4_K || FMT == SLHIP_FMT_Q5_K) {
        const uint32_t* w = reinterpret_cast<const uint32_t*>(row + sbo);  // 16-byte aligned super-block
        const uint32_t hx = w[0], hy = w[1], hz = w[2], hw = w[3];
        const int j = sj & 3, sh = 8 * j;
        uint32_t sc, mn;
        if (sj < 4) {
            sc = (hy >> sh) & 63u;
            mn = (hz >> sh) & 63u;
        } else {
            sc = ((hw >> sh) & 0xFu) | (((hy >> sh) >> 6 & 3u) << 4);
            mn = (((hw >> sh) >> 4) & 0xFu) | (((hz >> sh) >> 6 & 3u) << 4);
        }
        a0 = a1 = __fmul_rn(f16_lo(hx), static_cast<float>(sc));
        m0 = -__fmul_rn(f16_hi(hx), static_cast<float>(mn));
    } else if constexpr (FMT == SLHIP_FMT_Q6_K) {
        const float d = h16(sbo + 208);
        const uint32_t s = u16(sbo + 192 + 2 * sj);
        a0 = __fmul_rn(d, static_cast<float>(static_cast<int8_t>(s & 0xFFu)));
        a1 = __fmul_rn(d, static_cast<float>(static_cast<int8_t>(s >> 8)));
    } else if constexpr (FMT == SLHIP_FMT_Q3_K) {
        const float d = h16(sbo + 108);
        const int s0 = 2 * sj, w = s0 >> 2, b0 = s0 & 3;
        const uint32_t a = u16(sbo + 96 + 4 * (w & 1) + b0);
        const uint32_t h = u16(sbo + 104 + b0);
        const uint32_t lo = w < 2 ? (a & 0x0F0Fu) : ((a >> 4) & 0x0F0Fu);
        const uint32_t sc = lo | (((h >> (2 * w)) & 0x0303u) << 4);
        a0 = __fmul_rn(d, static_cast<float>(static_cast<int>(sc & 0xFFu) - 32));
        a1 = __fmul_rn(d, static_cast<float>(static_cast<int>(sc >> 8) - 32));
    } else if constexpr (FMT == SLHIP_FMT_Q2_K) {
        const float d = h16(sbo + 80), dm = h16(sbo + 82);
        const uint32_t v = u16(sbo + 2 * sj);
        a0 = __fmul_rn(d, static_cast<float>(v & 0xFu));
        a1 = __fmul_rn(d, static_cast<float>((v >> 8) & 0xFu));
        m0 = -__fmul_rn(dm, static_cast<float>((v >> 4) & 0xFu));
        m1 = -__fmul_rn(dm, static_cast<float>(v >> 12));
    } else {
        a0 = a1 = h16(off);
        if constexpr (Fmt<FMT>::M) m0 = h16(off + 2);  // Q4_1, Q5_1: + m sum(x)
    }
}

// The codes of block sj (32 values) of a row image, lane group g's eight (values 8g .. 8g + 7), as exact bf16.
template <int FMT>
__device__ __forceinline__ uint4 mq2_codes(const uint8_t* row, int sbo, int sj, int off, int g)
{
    if constexpr (FMT == SLHIP_FMT_Q4_K || FMT == SLHIP_FMT_Q5_K) return q4k_codes<FMT == SLHIP_FMT_Q5_K>(row, sbo, sj, g);
    else if constexpr (FMT == SLHIP_FMT_Q2_K || FMT == SLHIP_FMT_Q3_K) return q23k_codes<FMT == SLHIP_FMT_Q3_K>(row, sbo, sj, g);
    else if constexpr (FMT == SLHIP_FMT_Q6_K) return q6k_codes(row, sbo, sj, g);
    else return mq_codes<FMT>(row, off, g);
}

// 32-value blocks per stage: the block formats' stage of matvec_mfma_q, halved for f32 x when that stage holds
// 32 blocks (the x of the next stage waits in registers: 8 f32 per block and lane, two sets).
template <int FMT, bool XF32>
constexpr int mq2_blocks()
{
    return XF32 && MqGeom<FMT>::SKB == 32 ? 16 : MqGeom<FMT>::SKB;
}

// 16-row tiles per block with f32 x: two for the 32-value block formats, so that each block splits x into
// its three bf16 parts (and reads it) once for 32 rows -- [14336, 4096] pairs at 16 tokens, µs: Q4_0 51 -> 40,
// Q8_0 56 -> 45, Q4_1 52 -> 37, Q5_0 59 -> 51, Q5_1 55 -> 46; and for Q2_K / Q3_K with their group scales
// folded into the codes (Q2_K 52.7 -> 48.3, Q3_K 58.0 -> 56.7); one for Q4_K / Q5_K / Q6_K, whose extra
// decode state then spills (Q4_K 52 -> 55, Q6_K 70 -> 102).
template <int FMT>
constexpr int kMq2Tiles = (FMT == SLHIP_FMT_Q8_0 || FMT == SLHIP_FMT_Q4_0 || FMT == SLHIP_FMT_Q4_1 || FMT == SLHIP_FMT_Q5_0 ||
                           FMT == SLHIP_FMT_Q5_1 || FMT == SLHIP_FMT_Q2_K || FMT == SLHIP_FMT_Q3_K) ? 2 : 1;

template <int FMT, bool DUAL, bool XF32, int TN>
__global__ __launch_bounds__(64 * kMq2Waves) __attribute__((amdgpu_waves_per_eu(TN == 2 ? 4 : 1))) void matvec_mq2(MatvecArgs a)
{
    constexpr int NM = DUAL ? 2 : 1;
    constexpr int G = NM * TN;  // row groups: 16 rows of one matrix; group q = tile (q / NM), matrix (q % NM)
    constexpr int SKB = mq2_blocks<FMT, XF32>();
    constexpr int RB = MqGeom<FMT>::RB * SKB / MqGeom<FMT>::SKB;
    constexpr int UB = RB % 16 == 0 ? 16 : 4;  // bytes per staging load (global_load_lds: 16 or 4)
    constexpr int PITCH = stage_pitch(RB, UB);
    constexpr int SPR = PITCH / UB;
    constexpr int MS = (16 * SPR + 63) / 64 * 64;  // slots per matrix: whole waves
    constexpr int SLOTS = G * MS;
    constexpr int NT = 64 * kMq2Waves;
    constexpr int LPT = (SLOTS + NT - 1) / NT;
    constexpr int BPW = SKB / kMq2Waves;  // blocks per wave and stage
    constexpr bool KQ = FMT == SLHIP_FMT_Q4_K || FMT == SLHIP_FMT_Q5_K;
    constexpr bool K6 = FMT == SLHIP_FMT_Q6_K || FMT == SLHIP_FMT_Q2_K || FMT == SLHIP_FMT_Q3_K;  // 16-value groups
    constexpr bool Q2K = FMT == SLHIP_FMT_Q2_K;
    // Q2_K / Q3_K: the 16-value groups' scales folded into the codes (one MFMA chain per block, not two)
    constexpr bool FOLD = FMT == SLHIP_FMT_Q2_K || FMT == SLHIP_FMT_Q3_K;
    constexpr bool MIN = KQ || (Fmt<FMT>::M && !Fmt<FMT>::K) || Q2K;  // minimum terms
    constexpr int SBB = Fmt<FMT>::BB;
    constexpr int NP = XF32 ? 3 : 1;  // bf16 parts of x
    static_assert(RB % UB == 0 && SKB % kMq2Waves == 0, "stage shape");
    static_assert(!MIN || BPW <= 4, "the minimum terms take the wave's blocks as one 16 x 16 x 4 product");
    // per buffer: the stage, and at least half the cross-wave reduction's [wave][matrix][lane] sums
    constexpr int RED_WORDS = kMq2Waves * G * 64 * 4 / 2;
    constexpr int STW = SLOTS * UB / 4 > RED_WORDS ? SLOTS * UB / 4 : RED_WORDS;
    __shared__ __align__(16) uint32_t stage[2][STW];
    auto rowp = [&](int b, int m, int rr) -> const uint8_t* {
        return reinterpret_cast<const uint8_t*>(&stage[b][0]) + m * MS * UB + rr * PITCH;
    };
    const int lane = threadIdx.x & 63;
    const int wave = wave_id();
    const int r = lane & 15, g = lane >> 4;
    const int64_t n0 = static_cast<int64_t>(blockIdx.x) * 16 * TN;
    int64_t tok = a.t0 + r;
    tok = tok < a.T ? tok : a.T - 1;
    const int ns = static_cast<int>(a.K / (SKB * 32));

    // load slot q = threadIdx + NT i: matrix q / MS, row rr, piece c (padding slots reload a real piece)
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
            if (NT * i + 64 * wave >= SLOTS) break;  // wave-uniform
            if (NT * (i + 1) > SLOTS && static_cast<int>(threadIdx.x) + NT * i >= SLOTS) continue;
            char* base = reinterpret_cast<char*>(&stage[b][0]) + UB * (NT * i + 64 * wave);
            const char* mat = (((NT * i + 64 * wave) / MS) % NM ? a.wu : a.wg) + static_cast<int64_t>(s) * RB;
            load_to_lds<UB>(mat, src[i], base);
        }
    };
    // x of the wave's blocks of a stage: lane (g, token r) holds values 8g .. 8g + 7 of each
    struct Xs {
        float4 f[BPW][2];
        uint4 b[BPW];
    };
    auto fetch_x = [&](Xs& x, int s) {
#pragma unroll
        for (int j = 0; j < BPW; j++) {
            const int64_t k0 = (static_cast<int64_t>(s) * SKB + wave * BPW + j) * 32 + 8 * g;
            if constexpr (XF32) {
                const float* xr = static_cast<const float*>(a.x) + tok * a.xs + k0;
                x.f[j][0] = *reinterpret_cast<const float4*>(xr);
                x.f[j][1] = *reinterpret_cast<const float4*>(xr + 4);
            } else {
                x.b[j] = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(a.x) + tok * a.xs + k0);
            }
        }
    };
    f32x4_t acc[G];
#pragma unroll
    for (int m = 0; m < G; m++) acc[m] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

    auto compute = [&](int b, const Xs& x) {
        const int sbo = (KQ || K6) ? ((wave * BPW) >> 3) * SBB : 0;
        float xs0[BPW], xs1[BPW];  // the token's x sums of each block (Q2_K: of each half)
        float mn0[G][BPW], mn1[G][BPW];  // the row's minimum coefficients of each block
#pragma unroll
        for (int j = 0; j < BPW; j++) {
            const int blk = wave * BPW + j;
            const int sj = blk & 7;  // K-quant 32-value block in its super-block
            const int off = blk * Fmt<FMT>::BB;
            uint4 P[NP];
            float v[8];
            if constexpr (XF32) {
                v[0] = x.f[j][0].x; v[1] = x.f[j][0].y; v[2] = x.f[j][0].z; v[3] = x.f[j][0].w;
                v[4] = x.f[j][1].x; v[5] = x.f[j][1].y; v[6] = x.f[j][1].z; v[7] = x.f[j][1].w;
            } else {
                P[0] = x.b[j];
                Vec<SLHIP_BF16>::unpack(x.b[j], v);
            }
            const float ps8 = ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
            if constexpr (XF32) {
                // the split's guard against non-finite x (whose remainders would be NaN) only when some lane's
                // eight values have a non-finite (or overflowing) sum: a wave-uniform test
                if (__builtin_amdgcn_ballot_w64(!(fabsf(ps8) <= 3.4028235e38f)) == 0) split3_finite(v, P[0], P[1], P[NP - 1]);
                else split3(v, P[0], P[1], P[NP - 1]);
            }
            if constexpr (MIN) {
                float ps = ps8;
                if constexpr (Q2K) {  // per 16-value half: lane groups {0, 1} and {2, 3}
                    const float p01 = ps + __shfl_xor(ps, 16);
                    const float other = __shfl_xor(p01, 32);
                    xs0[j] = g < 2 ? p01 : other;
                    xs1[j] = g < 2 ? other : p01;
                } else {
                    ps += __shfl_xor(ps, 16);
                    ps += __shfl_xor(ps, 32);
                    xs0[j] = ps;
                }
            }
#pragma unroll
            for (int m = 0; m < G; m++) {
                const uint8_t* rw = rowp(b, m, r);
                const f32x4_t z = {0.0f, 0.0f, 0.0f, 0.0f};
                if constexpr (FOLD) {
                    // Q2_K / Q3_K: the 16-value groups' scales folded into the codes, one chain per block
                    float d;
                    const uint4 C = q23k_codes_scaled<FMT == SLHIP_FMT_Q3_K>(rw, sbo, sj, g, d);
                    if constexpr (MIN) {
                        float a0, a1, m0, m1;
                        mq2_scales<FMT>(rw, sbo, sj, off, a0, a1, m0, m1);
                        mn0[m][j] = m0;
                        mn1[m][j] = m1;
                    }
                    f32x4_t c = z;
#pragma unroll
                    for (int p = 0; p < NP; p++)
                        c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(P[p]), as_bf16x8(C), c, 0, 0, 0);
#pragma unroll
                    for (int i = 0; i < 4; i++) acc[m][i] = fmaf(d, c[i], acc[m][i]);
                    continue;
                }
                const uint4 C = mq2_codes<FMT>(rw, sbo, sj, off, g);
                float a0, a1, m0, m1;
                mq2_scales<FMT>(rw, sbo, sj, off, a0, a1, m0, m1);
                if constexpr (MIN) {
                    mn0[m][j] = m0;
                    mn1[m][j] = m1;
                }
                if constexpr (K6) {
                    const uint32_t keep = g < 2 ? ~0u : 0u;
                    const uint4 C0 = make_uint4(C.x & keep, C.y & keep, C.z & keep, C.w & keep);
                    const uint4 C1 = make_uint4(C.x & ~keep, C.y & ~keep, C.z & ~keep, C.w & ~keep);
                    f32x4_t c0 = z, c1 = z;
#pragma unroll
                    for (int p = 0; p < NP; p++) {
                        c0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(P[p]), as_bf16x8(C0), c0, 0, 0, 0);
                        c1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(P[p]), as_bf16x8(C1), c1, 0, 0, 0);
                    }
#pragma unroll
                    for (int i = 0; i < 4; i++) acc[m][i] = fmaf(a1, c1[i], fmaf(a0, c0[i], acc[m][i]));
                } else {
                    f32x4_t c = z;
#pragma unroll
                    for (int p = 0; p < NP; p++)
                        c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(P[p]), as_bf16x8(C), c, 0, 0, 0);
#pragma unroll
                    for (int i = 0; i < 4; i++) acc[m][i] = fmaf(a0, c[i], acc[m][i]);
                }
            }
        }
        if constexpr (MIN) {
            // lane (r, g): token r's sum of block g (A) and row r's minimum of block g (B)
            // (with two blocks per wave, lane groups 2 and 3 contribute zero)
            auto pick = [&](const float* v) {
                float o = g == 0 ? v[0] : 0.0f;
                if (BPW > 1) o = g == 1 ? v[1 % BPW] : o;
                if (BPW > 2) o = g == 2 ? v[2 % BPW] : o;
                if (BPW > 3) o = g == 3 ? v[3 % BPW] : o;
                return o;
            };
            const float xa = pick(xs0);
#pragma unroll
            for (int m = 0; m < G; m++) {
                acc[m] = __builtin_amdgcn_mfma_f32_16x16x4f32(xa, pick(mn0[m]), acc[m], 0, 0, 0);
                if constexpr (Q2K) acc[m] = __builtin_amdgcn_mfma_f32_16x16x4f32(pick(xs1), pick(mn1[m]), acc[m], 0, 0, 0);
            }
        }
    };

    constexpr int kWaitLoads = 0x0F70;  // vmcnt(0)
    Xs xa, xb;
    fetch(0, 0);
    fetch_x(xa, 0);
    __builtin_amdgcn_s_waitcnt(kWaitLoads);
    __syncthreads();
    for (int s = 0; s < ns; s += 2) {  // two stages per iteration: the x register sets alternate statically
        if (s + 1 < ns) {
            fetch(1, s + 1);
            fetch_x(xb, s + 1);
        }
        compute(0, xa);
        __builtin_amdgcn_s_waitcnt(kWaitLoads);
        __syncthreads();
        if (s + 1 >= ns) break;
        if (s + 2 < ns) {
            fetch(0, s + 2);
            fetch_x(xa, s + 2);
        }
        compute(1, xb);
        __builtin_amdgcn_s_waitcnt(kWaitLoads);
        __syncthreads();
    }
    // the waves' partial sums meet in the (now idle) stage memory: [wave][group][lane]
    f32x4_t* red = reinterpret_cast<f32x4_t*>(&stage[0][0]);
#pragma unroll
    for (int m = 0; m < G; m++) red[(wave * G + m) * 64 + lane] = acc[m];
    __syncthreads();
    if (wave >= TN) return;
    // wave tl finishes tile tl: row n0 + 16 tl + r, tokens 4g + i
    const int tl = wave;
    f32x4_t sg = red[(tl * NM) * 64 + lane], su = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    if (DUAL) su = red[(tl * NM + 1) * 64 + lane];
#pragma unroll
    for (int w = 1; w < kMq2Waves; w++) {
        sg += red[(w * G + tl * NM) * 64 + lane];
        if (DUAL) su += red[(w * G + tl * NM + 1) * 64 + lane];
    }
    const int64_t n = n0 + 16 * tl + r;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int64_t t = a.t0 + 4 * g + i;
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

// Whether matvec_mq2 takes this launch: K whole stages, rows whole staging loads, offsets below 2^31.
template <int FMT, bool XF32>
inline bool mq2_fits_x(const MatvecArgs& a)
{
    constexpr int SKB = mq2_blocks<FMT, XF32>();
    constexpr int RB = MqGeom<FMT>::RB * SKB / MqGeom<FMT>::SKB, UB = RB % 16 == 0 ? 16 : 4;
    return a.K % (SKB * 32) == 0 && a.wrow % UB == 0 && a.N * a.wrow < (int64_t{1} << 31);
}

template <int FMT>
inline bool mq2_fits(const MatvecArgs& a)
{
    return a.xt == SLHIP_F32 ? mq2_fits_x<FMT, true>(a) : mq2_fits_x<FMT, false>(a);
}

template <int FMT>
int run_mq2(MatvecArgs a, bool dual, hipStream_t st)
{
    constexpr int TN = kMq2Tiles<FMT>;
    const dim3 grid1(static_cast<unsigned>((a.N + 15) / 16)), gridx(static_cast<unsigned>((a.N + 16 * TN - 1) / (16 * TN)));
    for (int64_t t0 = 0; t0 < a.T; t0 += 16) {
        a.t0 = t0;
        if (a.xt == SLHIP_F32) {
            if (dual) matvec_mq2<FMT, true, true, TN><<<gridx, 64 * kMq2Waves, 0, st>>>(a);
            else matvec_mq2<FMT, false, true, TN><<<gridx, 64 * kMq2Waves, 0, st>>>(a);
        } else {
            if (dual) matvec_mq2<FMT, true, false, 1><<<grid1, 64 * kMq2Waves, 0, st>>>(a);
            else matvec_mq2<FMT, false, false, 1><<<grid1, 64 * kMq2Waves, 0, st>>>(a);
        }
        const int r = check_launch("matvec_mq2");
        if (r != SLHIP_OK) return r;
    }
    return SLHIP_OK;
}

// instantiated in matvec_mq_*.hip, one group of formats per unit; SLHIP_ERR_UNSUPPORTED when the launch does
// not fit (the caller then takes matvec_mfma_q)
int run_mq2_part0(int fmt, const MatvecArgs& a, bool dual, hipStream_t st);
int run_mq2_part1(int fmt, const MatvecArgs& a, bool dual, hipStream_t st);
int run_mq2_part2(int fmt, const MatvecArgs& a, bool dual, hipStream_t st);

}  // namespace slhip
