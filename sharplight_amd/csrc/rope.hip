// Rotary position embedding with the per-head q/k RMSNorm of Qwen3-style blocks fused in front, for up
// to four tensors (q and k of a layer) that share one position vector, in one launch.
//
// Semantics follow the reference CPU provider's RopeOp (src/Sharplight.Cpu/RopeOp.cs:28-183) run on the
// output of RowOp RmsNorm (RowOp.cs:63-77), which is what the Vulkan lowerer fuses into its rope kernel
// (src/Sharplight.Shaders/Lowering/GraphLowerer.Fusion.cs:618-630, Kernels/rope.slang:150-195):
//   inv_i = base^(-2i/dims) * freq_scale and theta = pos * inv_i (/ ff[i]) in f64;
//   c = (float)cos(theta) * attn_factor, s = (float)sin(theta) * attn_factor (cos/sin within 1 f32 ulp);
//   optional norm: x' = (x * (1/sqrt(sum(x^2)/D + eps))) * w;
//   neox pairs (i, i + dims/2), normal pairs (2i, 2i+1): y0 = x0*c - x1*s, y1 = x0*s + x1*c;
//   elements from dims to D are copied (normed when the norm is fused).
// The angles and their reduction are f64 because positions reach 32767 and more: an f32 argument would
// be off by ~1e-3 rad; sin/cos of the reduced angle (|r| <= pi/4) are evaluated in f32.
//
// Layout (vector path): a flat grid of independent waves. A wave owns one token and a group of 64/L
// whole head rows of one tensor, L = dims/2 / V lanes per head row (V = elements per 16-byte vector);
// lane c of a head holds pairs [c*V, c*V + V) as two 16-byte vectors, so loads and stores are fully
// used 16-byte accesses and the fused norm is a butterfly over the L lanes of a head. Each wave issues
// its loads and norm weights, then computes the token's dims/2 (cos, sin) pairs (f64 angle and
// reduction, f32 series) into its own LDS slice, one angle per lane, and never waits for another wave:
// recomputing the table per wave costs about one sincos per lane, far less than a block-wide barrier
// that holds every wave of a token until the table is ready.
#include "common.hpp"
#include "rope_math.hpp"

#include <stdlib.h>
#include <string.h>

#include <cmath>

namespace slhip {


constexpr int kMaxRopeTensors = 4;
constexpr int kMaxHalf = 512;  // dims <= 1024
constexpr int kArgInv = 128;   // inverse frequencies carried in the kernel arguments up to dims = 256
constexpr int kRopeWpb = 4;    // waves per block of the vector path

struct RopeTensorDev {
    const void* x;
    void* y;
    const float* w;
    int64_t heads, head0;  // head count, and index of the first head in the launch's head numbering
    int64_t xst, xsh, yst, ysh;
    int to_cache;          // y is a KV cache written at the rows of RopeArgs::rows
};

struct RopeArgs {
    RopeTensorDev t[kMaxRopeTensors];
    int nt;
    int64_t total_heads;
    int groups;                   // vector path: head groups per token, over all tensors
    int goff[kMaxRopeTensors];    // vector path: first head group of each tensor
    const int32_t* pos;
    const float* ff;
    int64_t T, D;
    int dims, neox, norm;
    float base, fs, af, eps;
    float inv_d;             // 1/D when D is a power of two (then q * inv_d == q / D exactly), else 0
    int inv_in_args;         // inv[] holds the inverse frequencies (dims/2 <= kArgInv)
    double l2b;              // log2(base) in f64, for dims/2 > kArgInv
    double inv[kArgInv];     // base^(-2i/dims) * freq_scale in f64, computed on the host
    CacheRowsDev rows;       // cache rows of the tensors with to_cache
    uint32_t* err;           // the device error record (cache rows outside the cache)
    int axes;                // position axes per token (positions [T, axes])
    int multi;               // sections in use: pairs (or elements) take their own axis
    int sec[4], interleaved, per_element;
};

// RopeOp.AxisOf (src/Sharplight.Cpu/RopeOp.cs:70-106) / rope.slang's axis_for_pair (Kernels/rope.slang:20-40).
__device__ __forceinline__ int axis_of(const RopeArgs& a, int i)
{
    const int sd = a.sec[0] + a.sec[1] + a.sec[2] + a.sec[3];
    const int sector = i % sd;
    if (a.interleaved) {
        if (sector % 3 == 1 && sector < 3 * a.sec[1]) return 1;
        if (sector % 3 == 2 && sector < 3 * a.sec[2]) return 2;
        return sector % 3 == 0 && sector < 3 * a.sec[0] ? 0 : 3;
    }
    if (sector < a.sec[0]) return 0;
    if (sector < a.sec[0] + a.sec[1]) return 1;
    return sector < a.sec[0] + a.sec[1] + a.sec[2] ? 2 : 3;
}

// The axes of pair i's first and second element (RopeOp.cs:54-66).
__device__ __forceinline__ int2 pair_axes(const RopeArgs& a, int i)
{
    if (!a.multi) return make_int2(0, 0);
    const int half = a.dims / 2;
    const int first = a.neox ? i : 2 * i, second = a.neox ? i + half : 2 * i + 1;
    return make_int2(axis_of(a, a.per_element ? first / 2 : i), axis_of(a, a.per_element ? second / 2 : i));
}

// Token t's positions of the four axes: an axis beyond the given ones reads axis 0 when there is one axis,
// else position 0 (RopeOp.cs:133-139).
__device__ __forceinline__ void token_positions(const RopeArgs& a, int64_t t, double* pp)
{
#pragma unroll
    for (int ax = 0; ax < 4; ax++)
        pp[ax] = ax < a.axes ? static_cast<double>(a.pos[t * a.axes + ax]) : a.axes == 1 ? static_cast<double>(a.pos[t * a.axes]) : 0.0;
}

// Entry i of token t's table: (c1, s1, c2, s2), the second pair for the pair's second element (the same
// angle unless per-element sections give it another axis). The inverse frequencies come from the host in
// f64 (std::pow, as RopeOp's Math.Pow) when dims/2 <= kArgInv; beyond that, exp2(log2(base) * (-2i/dims))
// in f64 (within ~2e-15 relative of pow: < 1e-10 rad at position 32767, far below the f32 result's
// resolution).
__device__ __forceinline__ float4 table_entry(const RopeArgs& a, const double* pp, int i)
{
    const double inv = a.inv_in_args ? a.inv[i] : exp2(a.l2b * (-2.0 * i / a.dims)) * static_cast<double>(a.fs);
    const int2 ax = pair_axes(a, i);
    double theta = pp[ax.x] * inv;
    if (a.ff) theta /= static_cast<double>(a.ff[i]);
    float s, c;
    sincos_f64_to_f32(theta, &s, &c);
    float s2 = s, c2 = c;
    if (ax.y != ax.x) {
        double theta2 = pp[ax.y] * inv;
        if (a.ff) theta2 /= static_cast<double>(a.ff[i]);
        sincos_f64_to_f32(theta2, &s2, &c2);
    }
    return make_float4(c * a.af, s * a.af, c2 * a.af, s2 * a.af);
}

// sin/cos of theta = p * inv (/ ff, only when the launch has frequency factors: FF) in f64, narrowed to f32.
template <bool FF>
__device__ __forceinline__ float2 angle_cs(double p, double inv, float ff)
{
    double theta = p * inv;
    if constexpr (FF) theta /= static_cast<double>(ff);
    float s, c;
    sincos_f64_to_f32(theta, &s, &c);
    return make_float2(c, s);
}

__device__ __forceinline__ int tensor_of(const RopeArgs& a, int64_t gh)
{
    int k = 0;
#pragma unroll
    for (int j = 1; j < kMaxRopeTensors; j++)
        if (j < a.nt && gh >= a.t[j].head0) k = j;
    return k;
}

typedef __attribute__((address_space(1))) float gfloat;

// A row of ones standing in for an absent norm weight.
struct OnesRow {
    float v[2 * kArgInv];
};
constexpr OnesRow make_ones_row()
{
    OnesRow r{};
    for (int i = 0; i < 2 * kArgInv; i++) r.v[i] = 1.0f;
    return r;
}
__constant__ OnesRow kOnesRow = make_ones_row();

// Sum of squares of 2V values held as V/2 packed bf16 words per vector: each v_dot2 adds two exact products.
template <int DTI, int V>
__device__ __forceinline__ float sum_squares(const uint4& r0, const uint4& r1, const float* f)
{
    float q = 0.f;
    if constexpr (DTI == SLHIP_BF16) {
        const uint32_t w[8] = {r0.x, r0.y, r0.z, r0.w, r1.x, r1.y, r1.z, r1.w};
        float q1 = 0.f;
#pragma unroll
        for (int i = 0; i < 8; i += 2) {
            q = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w[i]), __builtin_bit_cast(bf16x2_t, w[i]), q, false);
            q1 = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w[i + 1]), __builtin_bit_cast(bf16x2_t, w[i + 1]), q1, false);
        }
        q += q1;
    } else {
        float q1 = 0.f;
#pragma unroll
        for (int e = 0; e < 2 * V; e += 2) {
            q = fmaf(f[e], f[e], q);
            q1 = fmaf(f[e + 1], f[e + 1], q1);
        }
        q += q1;
    }
    return q;
}

// Vector path. Grid: x = head group, y = block of kRopeWpb tokens. The group (and so the tensor) is uniform
// over the block, and the token needs no division: every wave issues few scalar instructions, which matters
// because a CU's scalar unit is shared by all of its waves. Blocks are dispatched x first, so the waves in
// flight cover whole tokens of contiguous memory.
//
// The wave's table holds, per rotation pair i of its token, (c1 w0, s1 w1, s2 w0, c2 w1) with w0, w1 the norm
// weights of the pair's two elements (1 without a weight) and (c2, s2) the angle of the second element's
// axis (the first's unless per-element sections differ): the norm's weight multiply is folded into the
// table, so a lane applies y0 = f0 T.x - f1 T.y, y1 = f0 T.z + f1 T.w to its scaled values f = x * scale.
// (The CPU provider rounds x*scale*w before the rotation; folding changes the rounding of each product by
// at most an f32 ulp, well inside the parity tolerance.)
template <int DTI, int DTO, int L, bool MULTI, bool FF>
__global__ __launch_bounds__(64 * kRopeWpb) void rope_vec(RopeArgs a)
{
    using VI = Vec<DTI>;
    constexpr int V = VI::N;
    constexpr int HPW = 64 / L;             // head rows per wave
    constexpr int HALF = L * V;             // dims / 2
    constexpr int NE = (HALF + 63) / 64;    // table entries per lane
    static_assert(HALF <= kArgInv, "the vector path takes its inverse frequencies from the arguments");
    __shared__ float4 cs[kRopeWpb][kArgInv];
    const uint32_t t = blockIdx.y * kRopeWpb + wave_id();
    if (t >= static_cast<uint32_t>(a.T)) return;
    const int lane = threadIdx.x & 63;
    const int wv = threadIdx.x >> 6;
    const int gi = blockIdx.x;
    int k = 0;
#pragma unroll
    for (int j = 1; j < kMaxRopeTensors; j++) k = (j < a.nt && gi >= a.goff[j]) ? j : k;
    const RopeTensorDev& tt = a.t[k];
    const void* xp = tt.x;
    void* yp = tt.y;
    const float* wp = tt.w;
    const int64_t heads = tt.heads, xs = tt.xst, xh = tt.xsh, ys = tt.yst, yh = tt.ysh;
    const int64_t h = static_cast<int64_t>(gi - a.goff[k]) * HPW + lane / L;
    const int c = lane % L;
    const bool active = h < heads;
    const int e0 = a.neox ? c * V : 2 * c * V;
    const int e1 = a.neox ? HALF + c * V : 2 * c * V + V;
    // Lanes past the tensor's last head read that head (and store nothing), so every load below is
    // unconditional: a load under a divergent branch makes the compiler wait for it at the join.
    const int64_t hl = active ? h : heads - 1;
    const char* xrow = static_cast<const char*>(xp) + static_cast<int64_t>(t) * xs * VI::BYTES;  // wave-uniform
    const uint32_t xo0 = static_cast<uint32_t>((hl * xh + e0) * VI::BYTES);
    const uint32_t xo1 = static_cast<uint32_t>((hl * xh + e1) * VI::BYTES);

    // Table inputs first: entries lane (+ 64), NE per lane. Vector-memory loads complete in order, so a table
    // input loaded after the row's data would make the f64 table wait for the HBM data instead of overlapping
    // it; and the code stays free of branches up to the table, because the compiler waits for outstanding
    // loads where divergent paths join. A norm without weight reads a row of ones (exact).
    double p = 0.0, pp[4];
    if constexpr (MULTI)
        token_positions(a, t, pp);
    else
        p = static_cast<double>(a.pos[t]);
    // (Global-address-space pointers: a generic pointer would make these flat loads, which also hold the
    // LDS counter that the table's synchronization waits on.)
    const gfloat* wsrc = (a.norm && wp) ? (const gfloat*)wp : (const gfloat*)kOnesRow.v;
    const gfloat* ffp = (const gfloat*)(FF ? a.ff : kOnesRow.v);
    int ie[NE];
    double inv[NE];
    float ffv[NE], w0[NE], w1[NE];
#pragma unroll
    for (int n = 0; n < NE; n++) {
        ie[n] = lane + 64 * n < HALF ? lane + 64 * n : HALF - 1;
        inv[n] = a.inv[ie[n]];
        ffv[n] = ffp[ie[n]];
        const int j0 = a.neox ? ie[n] : 2 * ie[n];
        const int j1 = a.neox ? ie[n] + HALF : 2 * ie[n] + 1;
        w0[n] = wsrc[j0];
        w1[n] = wsrc[j1];
    }
    const uint4 r0 = load_nt(xrow + xo0);
    const uint4 r1 = load_nt(xrow + xo1);
    // Keeps the instruction scheduler from sinking the loads below the f64 work (it would, to save
    // registers), which would leave the table's latency unhidden.
    __builtin_amdgcn_sched_barrier(0);
    // The output row: the token itself, or its KV-cache row (scalar loads of its sequence row and block
    // table entry, only needed by the stores).
    CacheRow cr{static_cast<int64_t>(t), 0, 0, 0, 0, 0};
    if (tt.to_cache) cr = cache_row(a.rows, t);
    // Lanes past dims/2 rewrite the last entry with the same value.
#pragma unroll
    for (int n = 0; n < NE; n++) {
        float2 v1, v2;
        if constexpr (MULTI) {
            const int2 ax = pair_axes(a, ie[n]);
            v1 = angle_cs<FF>(pp[ax.x], inv[n], ffv[n]);
            v2 = ax.y == ax.x ? v1 : angle_cs<FF>(pp[ax.y], inv[n], ffv[n]);
        } else {
            v1 = v2 = angle_cs<FF>(p, inv[n], ffv[n]);
        }
        const float cf = a.af;
        // entry c V + e at e L + c: the L lanes of a head read one vector of entries each step, L
        // consecutive 16-byte entries (no bank conflicts; entry-major the L reads were 16 V bytes apart)
        const int slot = (ie[n] % V) * L + ie[n] / V;
        cs[wv][slot] = make_float4((v1.x * cf) * w0[n], (v1.y * cf) * w1[n], (v2.y * cf) * w0[n], (v2.x * cf) * w1[n]);
    }
    wave_lds_sync();
    if (!active) return;

    float f[2 * V];
    VI::unpack(r0, f);
    VI::unpack(r1, f + V);
    if (a.norm) {
        const float q = group_sum<L>(sum_squares<DTI, V>(r0, r1, f));
        const float m = a.inv_d > 0.f ? q * a.inv_d : q / static_cast<float>(a.D);
        const float sq = sqrtf(m + a.eps);
        float scale = recip_nr(sq);
        // recip_nr equals 1/sq on [2^-125, 2^125]; outside it (a zero, infinite or extreme sum) the division.
        // The test is wave-uniform, so the division is not evaluated on the common path.
        const bool in_range = sq >= 0x1p-125f && sq <= 0x1p125f;
        if (__builtin_amdgcn_ballot_w64(!in_range) != 0) {
            if (!in_range) scale = 1.0f / sq;
        }
#pragma unroll
        for (int e = 0; e < 2 * V; e++) f[e] *= scale;
    }
    const float4* ct = &cs[wv][c];  // entry c V + e at e L + c
    float o[2 * V];
    if (a.neox) {  // wave-uniform: one loop per pair layout, no per-element selects
#pragma unroll
        for (int e = 0; e < V; e++) {
            const float4 cv = ct[e * L];
            o[e] = f[e] * cv.x - f[V + e] * cv.y;
            o[V + e] = f[e] * cv.z + f[V + e] * cv.w;
        }
    } else {
#pragma unroll
        for (int e = 0; e < V; e++) {
            const float4 cv = ct[e * L];
            o[2 * e] = f[2 * e] * cv.x - f[2 * e + 1] * cv.y;
            o[2 * e + 1] = f[2 * e] * cv.z + f[2 * e + 1] * cv.w;
        }
    }
    if (cr.row >= 0) {  // wave-uniform: a row outside the cache is skipped and reported
        char* yr = static_cast<char*>(yp) + (cr.row * ys + h * yh) * Vec<DTO>::BYTES;
        store_packed<DTO, V>(yr + e0 * Vec<DTO>::BYTES, o);
        store_packed<DTO, V>(yr + e1 * Vec<DTO>::BYTES, o + V);
    } else if (lane == 0) {
        raise_cache_error(a.err, cr, t);
    }
}

// General path (any D, dims <= D, strides, alignment): one block per token, one wave per head row,
// scalar loads.
template <int DTI, int DTO>
__global__ __launch_bounds__(256) void rope_scalar(RopeArgs a)
{
    __shared__ float4 cs[kMaxHalf];
    const int64_t t = blockIdx.x;
    const int half = a.dims / 2;
    double pp[4];
    token_positions(a, t, pp);
    for (int i = threadIdx.x; i < half; i += blockDim.x) cs[i] = table_entry(a, pp, i);
    __syncthreads();
    const int lane = threadIdx.x & 63;
    for (int64_t gh = threadIdx.x >> 6; gh < a.total_heads; gh += blockDim.x >> 6) {
        const RopeTensorDev& tt = a.t[tensor_of(a, gh)];  // gh is wave-uniform: scalar loads
        const int64_t h = gh - tt.head0;
        int64_t orow = t;
        if (tt.to_cache) {
            const CacheRow cr = cache_row(a.rows, t);
            if (cr.row < 0) {  // skipped and reported, once per token and tensor
                if (lane == 0 && h == 0) raise_cache_error(a.err, cr, t);
                continue;
            }
            orow = cr.row;
        }
        const void* xr = static_cast<const char*>(tt.x) + (t * tt.xst + h * tt.xsh) * Vec<DTI>::BYTES;
        void* yr = static_cast<char*>(tt.y) + (orow * tt.yst + h * tt.ysh) * Vec<DTO>::BYTES;
        float scale = 1.0f;
        if (a.norm) {
            float q = 0.f;
            for (int64_t i = lane; i < a.D; i += 64) {
                float v = Vec<DTI>::load1(xr, i);
                q = fmaf(v, v, q);
            }
            scale = 1.0f / sqrtf(wave_sum(q) / static_cast<float>(a.D) + a.eps);
        }
        auto val = [&](int64_t i) {
            float v = Vec<DTI>::load1(xr, i);
            if (a.norm) {
                v *= scale;
                if (tt.w) v *= tt.w[i];
            }
            return v;
        };
        for (int i = lane; i < half; i += 64) {
            const int i0 = a.neox ? i : 2 * i;
            const int i1 = a.neox ? i + half : 2 * i + 1;
            const float x0 = val(i0), x1 = val(i1);
            const float4 cv = cs[i];
            Vec<DTO>::store1(yr, i0, x0 * cv.x - x1 * cv.y);
            Vec<DTO>::store1(yr, i1, x0 * cv.w + x1 * cv.z);
        }
        for (int64_t i = a.dims + lane; i < a.D; i += 64) Vec<DTO>::store1(yr, i, val(i));
    }
}

template <int DTI, int DTO, int L>
static int launch_vec(RopeArgs& a, hipStream_t st)
{
    if constexpr (L * Vec<DTI>::N > kArgInv) {
        return 1;  // dims/2 beyond the argument table: the general path
    } else {
        constexpr int HPW = 64 / L;
        int groups = 0;
        for (int j = 0; j < a.nt; j++) {
            a.goff[j] = groups;
            groups += static_cast<int>((a.t[j].heads + HPW - 1) / HPW);
        }
        a.groups = groups;
        const int64_t blocks = (a.T + kRopeWpb - 1) / kRopeWpb;
        if (blocks > 65535) return 1;  // beyond the grid's y extent: the general path
        const dim3 grid(static_cast<unsigned>(groups), static_cast<unsigned>(blocks));
        const bool multi = a.multi || a.axes > 1;
        if (a.ff) {
            if (multi) rope_vec<DTI, DTO, L, true, true><<<grid, 64 * kRopeWpb, 0, st>>>(a);
            else rope_vec<DTI, DTO, L, false, true><<<grid, 64 * kRopeWpb, 0, st>>>(a);
        } else {
            if (multi) rope_vec<DTI, DTO, L, true, false><<<grid, 64 * kRopeWpb, 0, st>>>(a);
            else rope_vec<DTI, DTO, L, false, false><<<grid, 64 * kRopeWpb, 0, st>>>(a);
        }
        return check_launch("rope_vec");
    }
}

template <int DTI, int DTO>
static int dispatch(RopeArgs& a, bool vec_ok, hipStream_t st)
{
    constexpr int V = Vec<DTI>::N;
    const int half = a.dims / 2;
    const int L = half % V == 0 ? half / V : 0;
    if (vec_ok && a.inv_in_args && L >= 1 && L <= 64 && (L & (L - 1)) == 0 && a.total_heads < (int64_t{1} << 30)) {
        int st_vec;
        switch (L) {
        case 1: st_vec = launch_vec<DTI, DTO, 1>(a, st); break;
        case 2: st_vec = launch_vec<DTI, DTO, 2>(a, st); break;
        case 4: st_vec = launch_vec<DTI, DTO, 4>(a, st); break;
        case 8: st_vec = launch_vec<DTI, DTO, 8>(a, st); break;
        case 16: st_vec = launch_vec<DTI, DTO, 16>(a, st); break;
        case 32: st_vec = launch_vec<DTI, DTO, 32>(a, st); break;
        default: st_vec = launch_vec<DTI, DTO, 64>(a, st); break;
        }
        if (st_vec != 1) return st_vec;
    }
    rope_scalar<DTI, DTO><<<dim3(static_cast<unsigned>(a.T)), 256, 0, st>>>(a);
    return check_launch("rope_scalar");
}

}  // namespace slhip

using namespace slhip;

extern "C" SLHIP_API int slhip_rope(int dtype_in, int dtype_out, const slhip_rope_tensor* tensors, int n_tensors,
                                    const int32_t* pos, const float* ff, int64_t T, int64_t D,
                                    const slhip_rope_cfg* cfg, slhip_stream stream)
{
    if (!cfg) return fail(SLHIP_ERR_INVALID, "rope: cfg is null");
    if (n_tensors < 1 || n_tensors > kMaxRopeTensors || !tensors)
        return fail(SLHIP_ERR_INVALID, "rope: between 1 and %d tensors per launch", kMaxRopeTensors);
    if (T < 0 || D <= 0) return fail(SLHIP_ERR_INVALID, "rope: bad shape T=%lld D=%lld", (long long)T, (long long)D);
    int dims = cfg->dims <= 0 ? static_cast<int>(D) : cfg->dims;
    if (dims > D || (dims & 1)) return fail(SLHIP_ERR_INVALID, "Rope dims %d invalid for head size %lld.", dims, (long long)D);
    if (dims / 2 > kMaxHalf) return fail(SLHIP_ERR_UNSUPPORTED, "rope: dims %d above %d", dims, 2 * kMaxHalf);
    if (T == 0) return SLHIP_OK;
    if (!pos) return fail(SLHIP_ERR_INVALID, "rope: positions are required");
    if (T > 0x7FFFFFFF) return fail(SLHIP_ERR_UNSUPPORTED, "rope: more than 2^31-1 tokens");
    if (!(dtype_in == SLHIP_F32 || dtype_in == SLHIP_BF16) ||
        !(dtype_out == SLHIP_F32 || dtype_out == SLHIP_F16 || dtype_out == SLHIP_BF16))
        return fail(SLHIP_ERR_UNSUPPORTED, "rope: dtype pair (%d -> %d) not supported", dtype_in, dtype_out);
    if (!(cfg->base > 0.0f)) return fail(SLHIP_ERR_INVALID, "rope: base must be positive");

    RopeArgs a{};
    a.nt = n_tensors;
    a.pos = pos;
    a.ff = ff;
    a.T = T;
    a.D = D;
    a.dims = dims;
    a.neox = cfg->neox ? 1 : 0;
    a.norm = cfg->norm ? 1 : 0;
    a.base = cfg->base;
    a.fs = cfg->freq_scale;
    a.af = cfg->attn_factor;
    a.eps = cfg->eps;
    a.inv_d = (D & (D - 1)) == 0 ? 1.0f / static_cast<float>(D) : 0.0f;
    a.l2b = std::log2(static_cast<double>(cfg->base));
    a.axes = cfg->pos_axes <= 0 ? 1 : cfg->pos_axes;
    if (a.axes > 4) return fail(SLHIP_ERR_INVALID, "rope: at most 4 position axes (got %d)", a.axes);
    for (int k = 0; k < 4; k++) {
        if (cfg->sections[k] < 0) return fail(SLHIP_ERR_INVALID, "rope: negative section");
        a.sec[k] = cfg->sections[k];
    }
    a.multi = a.sec[0] > 0 || a.sec[1] > 0 || a.sec[2] > 0;
    a.interleaved = cfg->interleaved ? 1 : 0;
    a.per_element = cfg->per_element ? 1 : 0;
    a.inv_in_args = dims / 2 <= kArgInv;
    if (a.inv_in_args)
        for (int i = 0; i < dims / 2; i++)
            a.inv[i] = std::pow(static_cast<double>(cfg->base), -2.0 * i / dims) * static_cast<double>(cfg->freq_scale);
    const int vin = dtype_in == SLHIP_F32 ? 4 : 8;
    const int bout = dtype_out == SLHIP_F32 ? 4 : 2;
    const int64_t oalign = vin * bout < 16 ? vin * bout : 16;
    bool vec_ok = dims == D;
    int64_t heads = 0;
    const slhip_cache_rows* rows = nullptr;
    for (int i = 0; i < n_tensors; i++) {
        const slhip_rope_tensor& s = tensors[i];
        if (!s.x || !s.y || s.heads < 0) return fail(SLHIP_ERR_INVALID, "rope: tensor %d is incomplete", i);
        if (s.heads > 1 && (s.x_stride_h < D || s.y_stride_h < D))
            return fail(SLHIP_ERR_INVALID, "rope: tensor %d head stride is smaller than D", i);
        if (cfg->norm == 0 && s.norm_w) return fail(SLHIP_ERR_INVALID, "rope: norm weight given without cfg->norm");
        if (s.rows) {
            if (rows && memcmp(rows, s.rows, sizeof *rows) != 0)
                return fail(SLHIP_ERR_INVALID, "rope: the cache tensors of one launch must share their rows");
            if (!rows) {
                const int e = make_cache_rows(s.rows, T, &a.rows);
                if (e) return e;
                const int ee = error_word(&a.err);
                if (ee) return ee;
            }
            rows = s.rows;
        }
        a.t[i] = RopeTensorDev{s.x, s.y, s.norm_w, s.heads, heads, s.x_stride_t, s.x_stride_h, s.y_stride_t, s.y_stride_h,
                               s.rows ? 1 : 0};
        heads += s.heads;
        vec_ok = vec_ok && aligned16(s.x) && s.x_stride_t % vin == 0 && s.x_stride_h % vin == 0 &&
                 reinterpret_cast<uintptr_t>(s.y) % oalign == 0 && (s.y_stride_t * bout) % oalign == 0 &&
                 (s.y_stride_h * bout) % oalign == 0 && (!s.norm_w || aligned16(s.norm_w));
    }
    a.total_heads = heads;
    if (heads == 0) return SLHIP_OK;
    hipStream_t st = to_stream(stream);
    if (dtype_in == SLHIP_BF16) {
        if (dtype_out == SLHIP_BF16) return dispatch<SLHIP_BF16, SLHIP_BF16>(a, vec_ok, st);
        if (dtype_out == SLHIP_F16) return dispatch<SLHIP_BF16, SLHIP_F16>(a, vec_ok, st);
        return dispatch<SLHIP_BF16, SLHIP_F32>(a, vec_ok, st);
    }
    if (dtype_out == SLHIP_BF16) return dispatch<SLHIP_F32, SLHIP_BF16>(a, vec_ok, st);
    if (dtype_out == SLHIP_F16) return dispatch<SLHIP_F32, SLHIP_F16>(a, vec_ok, st);
    return dispatch<SLHIP_F32, SLHIP_F32>(a, vec_ok, st);
}
