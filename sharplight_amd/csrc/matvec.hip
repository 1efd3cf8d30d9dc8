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
//   * the epilogue (activation, product, output rounding) runs on the reduced sums; lane l stores token l.
// Rows past N and lanes past the row end work on clamped indices and store the same values as their
// owners, so every lane issues the same memory operations (a divergent branch around loads makes the
// compiler wait for all outstanding ones).
#include "act.hpp"
#include "common.hpp"

#include <stdlib.h>

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
};

constexpr int kMvThreads = 512;

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

    // Stage x rows t0 .. t0+TT-1 (rows past T repeat row T-1) as f32, eight 16-byte loads per lane per pass.
    {
        const int per_row = static_cast<int>(a.K / 4);  // float4 units per staged row
        const int units = TT * per_row;
        for (int base = 0; base < units; base += 8 * kMvThreads) {
            float4 v[8];
#pragma unroll
            for (int q = 0; q < 8; q++) {
                int u = base + q * kMvThreads + static_cast<int>(threadIdx.x);
                u = u < units ? u : units - 1;
                const int t = u / per_row;
                const int c = u - t * per_row;
                int64_t tok = a.t0 + t;
                tok = tok < a.T ? tok : a.T - 1;
                if (a.xt == SLHIP_F32) {
                    v[q] = *reinterpret_cast<const float4*>(static_cast<const float*>(a.x) + tok * a.xs + c * 4);
                } else {
                    const uint2 b = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(a.x) + tok * a.xs + c * 4);
                    v[q] = make_float4(bf16_lo(b.x), bf16_hi(b.x), bf16_lo(b.y), bf16_hi(b.y));
                }
            }
#pragma unroll
            for (int q = 0; q < 8; q++) {
                int u = base + q * kMvThreads + static_cast<int>(threadIdx.x);
                u = u < units ? u : units - 1;
                reinterpret_cast<float4*>(xsh)[u] = v[q];
            }
        }
    }
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

    // Lane l stores token min(l, TT - 1), clamped to the last real token.
    const int tl = lane < TT ? lane : TT - 1;
    float g = ag[0], u = au[0];
#pragma unroll
    for (int t = 1; t < TT; t++) {
        g = tl == t ? ag[t] : g;
        u = tl == t ? au[t] : u;
    }
    float out = g;
    if (DUAL) {
        const float act = a.act == SLHIP_ACT_SILU        ? activate<SLHIP_ACT_SILU>(g)
                          : a.act == SLHIP_ACT_GELU_TANH ? activate<SLHIP_ACT_GELU_TANH>(g)
                                                         : activate<SLHIP_ACT_GELU_ERF>(g);
        out = act * u;
    }
    int64_t tok = a.t0 + tl;
    tok = tok < a.T ? tok : a.T - 1;
    if (a.yt == SLHIP_F32)
        static_cast<float*>(a.y)[tok * a.ys + n] = out;
    else
        static_cast<uint16_t*>(a.y)[tok * a.ys + n] = static_cast<uint16_t>(f32_to_bf16_bits(out));
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

template <int WT>
static int run_dense(MatvecArgs a, bool dual, hipStream_t st)
{
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

static int matvec_common(int fmt, int dtype_x, int dtype_y, const void* x, int64_t x_stride, int64_t T, int64_t K,
                         const void* wg, const void* wu, int64_t N, void* y, int64_t y_stride, int act, bool dual,
                         slhip_stream stream)
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
    if (fmt != SLHIP_FMT_F32 && fmt != SLHIP_FMT_F16 && fmt != SLHIP_FMT_BF16)
        return fail(SLHIP_ERR_UNSUPPORTED, "%s: weight format %d not supported", name, fmt);
    const int E = fmt == SLHIP_FMT_F32 ? 4 : 8;
    if (K % E != 0 || K % 4 != 0)
        return fail(SLHIP_ERR_UNSUPPORTED, "%s: K = %lld must be a multiple of %d for this weight format", name,
                    static_cast<long long>(K), E);
    if (!aligned16(wg) || (dual && !aligned16(wu)) || reinterpret_cast<uintptr_t>(x) % (dtype_x == SLHIP_F32 ? 16 : 8) ||
        (x_stride % 4) != 0)
        return fail(SLHIP_ERR_UNSUPPORTED, "%s: weights must be 16-byte aligned and x rows 4-element aligned", name);
    if (static_cast<int64_t>(K) * 4 > 65536)
        return fail(SLHIP_ERR_UNSUPPORTED, "%s: K = %lld above the staged-activation limit 16384", name,
                    static_cast<long long>(K));
    if (N > 0x7FFFFFFF || T > 0x7FFFFFFF) return fail(SLHIP_ERR_UNSUPPORTED, "%s: shape too large", name);
    MatvecArgs a{x, x_stride, static_cast<const char*>(wg), static_cast<const char*>(wu),
                 K * (fmt == SLHIP_FMT_F32 ? 4 : 2), y, y_stride, T, K, N, 0, dtype_x, dtype_y, act};
    hipStream_t st = to_stream(stream);
    if (fmt == SLHIP_FMT_F32) return run_dense<SLHIP_F32>(a, dual, st);
    if (fmt == SLHIP_FMT_F16) return run_dense<SLHIP_F16>(a, dual, st);
    return run_dense<SLHIP_BF16>(a, dual, st);
}

}  // namespace slhip

using namespace slhip;

extern "C" SLHIP_API int slhip_matvec(int fmt, int dtype_x, int dtype_y, const void* x, int64_t x_stride, int64_t T,
                                      int64_t K, const void* w, int64_t N, void* y, int64_t y_stride,
                                      slhip_stream stream)
{
    return matvec_common(fmt, dtype_x, dtype_y, x, x_stride, T, K, w, nullptr, N, y, y_stride, 0, false, stream);
}

extern "C" SLHIP_API int slhip_dual_matvec(int act, int fmt, int dtype_x, int dtype_y, const void* x, int64_t x_stride,
                                           int64_t T, int64_t K, const void* w_gate, const void* w_up, int64_t N,
                                           void* y, int64_t y_stride, slhip_stream stream)
{
    return matvec_common(fmt, dtype_x, dtype_y, x, x_stride, T, K, w_gate, w_up, N, y, y_stride, act, true, stream);
}
