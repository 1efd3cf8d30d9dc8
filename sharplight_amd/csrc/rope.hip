// Rotary position embedding with the per-head q/k RMSNorm of Qwen3-style blocks fused in front, for up
// to four tensors (q and k of a layer) that share one position vector, in one launch.
//
// Semantics follow the reference CPU provider's RopeOp (src/Sharplight.Cpu/RopeOp.cs:28-183) run on the
// output of RowOp RmsNorm (RowOp.cs:63-77), which is what the Vulkan lowerer fuses into its rope kernel
// (src/Sharplight.Shaders/Lowering/GraphLowerer.Fusion.cs:618-630, Kernels/rope.slang:150-195):
//   inv_i = base^(-2i/dims) * freq_scale and theta = pos * inv_i (/ ff[i]) in f64;
//   c = (float)cos(theta) * attn_factor, s = (float)sin(theta) * attn_factor;
//   optional norm: x' = (x * (1/sqrt(sum(x^2)/D + eps))) * w;
//   neox pairs (i, i + dims/2), normal pairs (2i, 2i+1): y0 = x0*c - x1*s, y1 = x0*s + x1*c;
//   elements from dims to D are copied (normed when the norm is fused).
// The angles are f64 because positions reach 32767 and more: an f32 argument would be off by ~1e-3 rad.
//
// Layout: one block per group of tokens. The block computes each token's dims/2 (cos, sin) pairs once
// in LDS (f64 sincos of f64 angles; the inverse frequencies come from the host in f64), shared by every
// head of every tensor; the first loads are issued before that work so their latency overlaps it. Each
// head row is handled by L lanes (L = dims/2 / V, V = elements per 16-byte vector): lane c of a head
// holds pairs [c*V, c*V + V) as two 16-byte vectors, so a wave covers 64/L whole heads with fully used
// 16-byte loads and stores, and the fused norm is a butterfly over the L lanes of the head.
#include "common.hpp"
#include "rope_math.hpp"

#include <stdlib.h>

#include <cmath>

namespace slhip {

constexpr int kMaxRopeTensors = 4;
constexpr int kMaxHalf = 512;    // dims <= 1024
constexpr int kArgInv = 128;     // inverse frequencies passed from the host when dims/2 <= this
constexpr int kTableEntries = 1024;  // (cos, sin) pairs per block: tokens_per_block * dims/2

struct RopeTensorDev {
    const void* x;
    void* y;
    const float* w;
    int64_t heads, head0;  // head count, and index of the first head in the launch's head numbering
    int64_t xst, xsh, yst, ysh;
};

struct RopeArgs {
    RopeTensorDev t[kMaxRopeTensors];
    int nt;
    int64_t total_heads;
    const int32_t* pos;
    const float* ff;
    int64_t T, D;
    int dims, neox, norm, tpb;  // tpb: tokens per block
    float base, fs, af, eps;
    int host_inv;              // inv[] holds base^(-2i/dims)*freq_scale, computed on the host in f64
    double inv[kArgInv];
};

// The block's (cos, sin) tables in LDS, one per token t0 .. t0+tpb-1; every thread must call it.
// HOST_INV: the inverse frequencies are in a.inv (always so on the vector path).
template <bool HOST_INV>
__device__ __forceinline__ void build_table(const RopeArgs& a, int64_t t0, float2* cs)
{
    const int half = a.dims / 2;
    for (int e = threadIdx.x; e < a.tpb * half; e += blockDim.x) {
        const int tl = e / half, i = e - tl * half;
        const int64_t t = t0 + tl;
        if (t >= a.T) continue;
        const double inv = (HOST_INV || a.host_inv)
                               ? a.inv[i]
                               : pow(static_cast<double>(a.base), -2.0 * i / a.dims) * static_cast<double>(a.fs);
        double theta = static_cast<double>(a.pos[t]) * inv;
        if (a.ff) theta /= static_cast<double>(a.ff[i]);
        double s, c;
        sincos_f64(theta, &s, &c);
        cs[e] = make_float2(static_cast<float>(c) * a.af, static_cast<float>(s) * a.af);
    }
    __syncthreads();
}

__device__ __forceinline__ int tensor_of(const RopeArgs& a, int64_t gh)
{
    int k = 0;
#pragma unroll
    for (int j = 1; j < kMaxRopeTensors; j++)
        if (j < a.nt && gh >= a.t[j].head0) k = j;
    return k;
}

// Work item `idx` of the block: token t0 + idx / lpt, head (idx % lpt) / L, chunk idx % L.
template <int DTI, int L>
struct RopeItem {
    int64_t t;
    int tl, c, k;
    int64_t h;
    __device__ __forceinline__ RopeItem(const RopeArgs& a, int64_t t0, int idx)
    {
        const int lpt = static_cast<int>(a.total_heads) * L;
        tl = idx / lpt;
        const int rem = idx - tl * lpt;
        const int64_t gh = rem / L;
        c = rem - static_cast<int>(gh) * L;
        t = t0 + tl;
        k = tensor_of(a, gh);
        h = gh - a.t[k].head0;
    }
};

template <int DTI, int DTO, int L>
__global__ __launch_bounds__(1024) void rope_vec(RopeArgs a)
{
    using VI = Vec<DTI>;
    constexpr int V = VI::N;
    __shared__ float2 cs[kTableEntries];
    const int half = a.dims / 2;
    const int64_t t0 = static_cast<int64_t>(blockIdx.x) * a.tpb;
    const int items = a.tpb * static_cast<int>(a.total_heads) * L;

    // element offsets of a lane's two vectors: neox (cV, half + cV); normal (2cV, 2cV + V)
    auto offsets = [&](int c, int& e0, int& e1) {
        e0 = a.neox ? c * V : 2 * c * V;
        e1 = a.neox ? half + c * V : 2 * c * V + V;
    };
    auto in_row = [&](const RopeItem<DTI, L>& it) {
        const RopeTensorDev& tt = a.t[it.k];
        return static_cast<const char*>(tt.x) + (it.t * tt.xst + it.h * tt.xsh) * VI::BYTES;
    };

    // The first item's loads are issued before the table is built, so their latency overlaps the f64 work.
    int idx = threadIdx.x;
    uint4 r0 = make_uint4(0, 0, 0, 0), r1 = r0;
    if (idx < items) {
        RopeItem<DTI, L> it(a, t0, idx);
        if (it.t < a.T) {
            int e0, e1;
            offsets(it.c, e0, e1);
            const char* xr = in_row(it);
            r0 = load_nt(xr + e0 * VI::BYTES);
            r1 = load_nt(xr + e1 * VI::BYTES);
        }
    }
    build_table<true>(a, t0, cs);

    for (bool first = true; idx < items; idx += blockDim.x, first = false) {
        RopeItem<DTI, L> it(a, t0, idx);
        if (it.t >= a.T) continue;
        const RopeTensorDev& tt = a.t[it.k];
        int e0, e1;
        offsets(it.c, e0, e1);
        if (!first) {
            const char* xr = in_row(it);
            r0 = load_nt(xr + e0 * VI::BYTES);
            r1 = load_nt(xr + e1 * VI::BYTES);
        }
        char* yr = static_cast<char*>(tt.y) + (it.t * tt.yst + it.h * tt.ysh) * Vec<DTO>::BYTES;
        float f[2 * V];
        VI::unpack(r0, f);
        VI::unpack(r1, f + V);
        if (a.norm) {
            float q = 0.f;
#pragma unroll
            for (int e = 0; e < 2 * V; e++) q = fmaf(f[e], f[e], q);
            q = group_sum<L>(q);
            const float scale = 1.0f / sqrtf(q / static_cast<float>(a.D) + a.eps);
#pragma unroll
            for (int e = 0; e < 2 * V; e++) f[e] *= scale;
            if (tt.w) {
#pragma unroll
                for (int hv = 0; hv < 2; hv++) {
                    const float4* wp = reinterpret_cast<const float4*>(tt.w + (hv ? e1 : e0));
#pragma unroll
                    for (int q4 = 0; q4 < V / 4; q4++) {
                        float4 w4 = wp[q4];
                        f[hv * V + 4 * q4 + 0] *= w4.x;
                        f[hv * V + 4 * q4 + 1] *= w4.y;
                        f[hv * V + 4 * q4 + 2] *= w4.z;
                        f[hv * V + 4 * q4 + 3] *= w4.w;
                    }
                }
            }
        }
        const float2* ct = cs + it.tl * half + it.c * V;
        float o[2 * V];
        if (a.neox) {
#pragma unroll
            for (int e = 0; e < V; e++) {
                const float2 cv = ct[e];
                const float x0 = f[e], x1 = f[V + e];
                o[e] = x0 * cv.x - x1 * cv.y;
                o[V + e] = x0 * cv.y + x1 * cv.x;
            }
        } else {
#pragma unroll
            for (int e = 0; e < V; e++) {
                const float2 cv = ct[e];
                const float x0 = f[2 * e], x1 = f[2 * e + 1];
                o[2 * e] = x0 * cv.x - x1 * cv.y;
                o[2 * e + 1] = x0 * cv.y + x1 * cv.x;
            }
        }
        store_packed<DTO, V>(yr + e0 * Vec<DTO>::BYTES, o);
        store_packed<DTO, V>(yr + e1 * Vec<DTO>::BYTES, o + V);
    }
}

// General path (any D, dims <= D, strides, alignment): one wave per head row, scalar loads.
template <int DTI, int DTO>
__global__ __launch_bounds__(256) void rope_scalar(RopeArgs a)
{
    __shared__ float2 cs[kTableEntries];
    const int64_t t = blockIdx.x;  // one token per block (tpb == 1)
    build_table<false>(a, t, cs);
    const int lane = threadIdx.x & 63;
    const int half = a.dims / 2;
    for (int64_t gh = threadIdx.x >> 6; gh < a.total_heads; gh += blockDim.x >> 6) {
        const int k = tensor_of(a, gh);
        const RopeTensorDev& tt = a.t[k];
        const int64_t h = gh - tt.head0;
        const void* xr = static_cast<const char*>(tt.x) + (t * tt.xst + h * tt.xsh) * Vec<DTI>::BYTES;
        void* yr = static_cast<char*>(tt.y) + (t * tt.yst + h * tt.ysh) * Vec<DTO>::BYTES;
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
            const float2 cv = cs[i];
            Vec<DTO>::store1(yr, i0, x0 * cv.x - x1 * cv.y);
            Vec<DTO>::store1(yr, i1, x0 * cv.y + x1 * cv.x);
        }
        for (int64_t i = a.dims + lane; i < a.D; i += 64) Vec<DTO>::store1(yr, i, val(i));
    }
}

static int env_int(const char* name, int dflt)
{
    const char* s = getenv(name);
    return s && *s ? atoi(s) : dflt;
}

template <int DTI, int DTO>
static int dispatch(RopeArgs a, bool vec_ok, hipStream_t st)
{
    constexpr int V = Vec<DTI>::N;
    const int half = a.dims / 2;
    if (vec_ok && a.host_inv && half % V == 0) {
        const int L = half / V;
        if (L <= 64 && (L & (L - 1)) == 0) {
            const int64_t lpt = a.total_heads * L;  // lanes per token
            // Tokens per block: as many as keep the block at <= 512 lanes (>= 1), within the LDS table.
            int tpb = lpt >= 512 ? 1 : static_cast<int>(512 / lpt);
            int forced = env_int("SLHIP_ROPE_TPB", 0);
            if (forced > 0) tpb = forced;
            while (tpb > 1 && (tpb * half > kTableEntries || tpb * lpt > 1024)) tpb--;
            a.tpb = tpb;
            const int64_t lanes = tpb * lpt;
            const int threads = static_cast<int>(lanes >= 1024 ? 1024 : ((lanes + 63) / 64) * 64);
            dim3 grid(static_cast<unsigned>((a.T + tpb - 1) / tpb));
            switch (L) {
            case 1: rope_vec<DTI, DTO, 1><<<grid, threads, 0, st>>>(a); break;
            case 2: rope_vec<DTI, DTO, 2><<<grid, threads, 0, st>>>(a); break;
            case 4: rope_vec<DTI, DTO, 4><<<grid, threads, 0, st>>>(a); break;
            case 8: rope_vec<DTI, DTO, 8><<<grid, threads, 0, st>>>(a); break;
            case 16: rope_vec<DTI, DTO, 16><<<grid, threads, 0, st>>>(a); break;
            case 32: rope_vec<DTI, DTO, 32><<<grid, threads, 0, st>>>(a); break;
            default: rope_vec<DTI, DTO, 64><<<grid, threads, 0, st>>>(a); break;
            }
            return check_launch("rope_vec");
        }
    }
    a.tpb = 1;
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
    if (!(dtype_in == SLHIP_F32 || dtype_in == SLHIP_BF16) || !(dtype_out == SLHIP_F32 || dtype_out == SLHIP_BF16))
        return fail(SLHIP_ERR_UNSUPPORTED, "rope: dtype pair (%d -> %d) not supported", dtype_in, dtype_out);

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
    // Inverse frequencies in f64 on the host, as RopeOp's constructor computes them (RopeOp.cs:47-52).
    a.host_inv = dims / 2 <= kArgInv;
    if (a.host_inv)
        for (int i = 0; i < dims / 2; i++) a.inv[i] = std::pow(static_cast<double>(a.base), -2.0 * i / dims) * static_cast<double>(a.fs);
    const int vin = dtype_in == SLHIP_F32 ? 4 : 8;
    const int bout = dtype_out == SLHIP_F32 ? 4 : 2;
    const int64_t oalign = vin * bout < 16 ? vin * bout : 16;
    bool vec_ok = dims == D;
    int64_t heads = 0;
    for (int i = 0; i < n_tensors; i++) {
        const slhip_rope_tensor& s = tensors[i];
        if (!s.x || !s.y || s.heads < 0) return fail(SLHIP_ERR_INVALID, "rope: tensor %d is incomplete", i);
        if (s.heads > 1 && (s.x_stride_h < D || s.y_stride_h < D))
            return fail(SLHIP_ERR_INVALID, "rope: tensor %d head stride is smaller than D", i);
        if (cfg->norm == 0 && s.norm_w) return fail(SLHIP_ERR_INVALID, "rope: norm weight given without cfg->norm");
        a.t[i] = RopeTensorDev{s.x, s.y, s.norm_w, s.heads, heads, s.x_stride_t, s.x_stride_h, s.y_stride_t, s.y_stride_h};
        heads += s.heads;
        vec_ok = vec_ok && aligned16(s.x) && s.x_stride_t % vin == 0 && s.x_stride_h % vin == 0 &&
                 reinterpret_cast<uintptr_t>(s.y) % oalign == 0 && (s.y_stride_t * bout) % oalign == 0 &&
                 (s.y_stride_h * bout) % oalign == 0 && (!s.norm_w || aligned16(s.norm_w));
    }
    a.total_heads = heads;
    if (heads == 0) return SLHIP_OK;
    hipStream_t st = to_stream(stream);
    if (dtype_in == SLHIP_BF16 && dtype_out == SLHIP_BF16) return dispatch<SLHIP_BF16, SLHIP_BF16>(a, vec_ok, st);
    if (dtype_in == SLHIP_F32 && dtype_out == SLHIP_F32) return dispatch<SLHIP_F32, SLHIP_F32>(a, vec_ok, st);
    if (dtype_in == SLHIP_BF16 && dtype_out == SLHIP_F32) return dispatch<SLHIP_BF16, SLHIP_F32>(a, vec_ok, st);
    return dispatch<SLHIP_F32, SLHIP_BF16>(a, vec_ok, st);
}
