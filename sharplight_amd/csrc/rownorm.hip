// Row normalization kernels: RMSNorm, L2Norm and LayerNorm over the last axis, each with an optional
// residual add fused in front (the Add+RmsNorm unit). Bandwidth-bound: one HBM read of every input and
// one write of every output.
//
// Semantics follow the reference CPU provider (src/Sharplight.Cpu/RowOp.cs:63-113):
//   RMS:   scale = 1/sqrt(sum(h^2)/D + eps), y = (h*scale)*w
//   L2:    scale = 1/sqrt(sum(h^2) + eps),   y = h*scale
//   LAYER: mean = sum(h)/D, inv = 1/sqrt(sum((h-mean)^2)/D + eps), y = ((h-mean)*inv)*w + b
// with h = x + res in f32 when a residual is given, written back as the updated residual stream (the
// pass-1 output of the fused unit, src/Sharplight.Shaders/Lowering/RowNormKernelSource.cs:5-9).
//
// Layout: a row is split over a "row group" of WPR wavefronts (64*WPR lanes). Lane t of the group owns
// the 16-byte vectors t, t + 64*WPR, t + 2*64*WPR, ... (NV of them), so every load and store
// instruction of a wave covers 1 KiB of consecutive bytes. The row stays in VGPRs between the
// reduction and the scaling pass. Reductions are a butterfly within the wave, then (WPR > 1) one LDS
// exchange between the group's waves. A block holds 256/(64*WPR) row groups (or one group of up to
// 16 waves). The GEMM activation copies of the normalized row (f16 values; E4M3 codes with one f32
// scale per 128 values) are written from the same f32 values as y: a 128-value group of the E4M3 rows is
// the 16 (bf16 input) or 32 (f32 input) consecutive lanes holding it, so its amax is a butterfly max over
// those lanes. 2-byte rows whose length is a multiple of 4 but not of 8 use the same kernel with 8-byte
// vectors. Rows that fit neither (odd lengths, unaligned pointers or strides, or D beyond 8*64*16
// vectors) take a scalar block-per-row kernel.
#include "common.hpp"

#include <stdlib.h>

namespace slhip {

struct RowNormArgs {
    const void* x;
    const void* res;
    const float* w;
    const float* b;
    void* y;
    void* h;
    int64_t rows;
    int64_t D;
    int64_t xs, rs, ys, hs;  // row strides in elements
    float eps;
    int kind;
    void* y16;     // f16 copy of y, or null
    int64_t y16s;  // its row stride in elements
    void* yq;      // E4M3 rows (D codes, then D/128 f32 scales), or null
    int64_t yqs;   // their row stride in bytes
};

// Sum over a row group: a wave butterfly, then (several waves) one LDS exchange. Each call of a kernel passes
// its own LDS region, so no barrier is needed ahead of the writes.
template <int NG>  // number of row groups sharing the LDS exchange
__device__ __forceinline__ float group_reduce(float v, int wpr, int group, int wave_in_group, float* red)
{
    v = wave_sum(v);
    if (wpr == 1) return v;
    if ((threadIdx.x & 63) == 0) red[group * 16 + wave_in_group] = v;
    __syncthreads();
    float s = 0.f;
    for (int i = 0; i < wpr; i++) s += red[group * 16 + i];
    return s;
}

// The raw input vector of a lane: 16 bytes, or 8 bytes (four 2-byte values) for rows whose length is a
// multiple of 4 but not of 8.
template <int VB> struct RawVec;
template <> struct RawVec<16> {
    using T = uint4;
    __device__ static __forceinline__ T load(const void* p) { return load_nt(p); }
    __device__ static __forceinline__ void launder(T& r)
    {
        asm volatile("" : "+v"(r.x), "+v"(r.y), "+v"(r.z), "+v"(r.w));
    }
    template <int DT> __device__ static __forceinline__ void unpack(const T& r, float* f) { Vec<DT>::unpack(r, f); }
    template <int DT> __device__ static __forceinline__ T pack(const float* f) { return Vec<DT>::pack(f); }
};
template <> struct RawVec<8> {
    using T = uint2;
    __device__ static __forceinline__ T load(const void* p)
    {
        const u32x2 v = __builtin_nontemporal_load(static_cast<const u32x2*>(p));
        return make_uint2(v.x, v.y);
    }
    __device__ static __forceinline__ void launder(T& r) { asm volatile("" : "+v"(r.x), "+v"(r.y)); }
    template <int DT> __device__ static __forceinline__ void unpack(const T& r, float* f)
    {
        static_assert(Vec<DT>::BYTES == 2, "8-byte vectors hold 2-byte values");
        float t[8];
        Vec<DT>::unpack(make_uint4(r.x, r.y, 0u, 0u), t);
#pragma unroll
        for (int e = 0; e < 4; e++) f[e] = t[e];
    }
    template <int DT> __device__ static __forceinline__ T pack(const float* f)
    {
        const float t[8] = {f[0], f[1], f[2], f[3], 0.f, 0.f, 0.f, 0.f};
        const uint4 v = Vec<DT>::pack(t);
        return make_uint2(v.x, v.y);
    }
};

template <int DTI, int DTO, int NV, bool RES, bool Q, int VB>
__global__ __launch_bounds__(1024) void rownorm_vec(RowNormArgs a, int wpr)
{
    using VI = Vec<DTI>;
    using RV = RawVec<VB>;
    static_assert(VB == 16 || (VB == 8 && VI::BYTES == 2 && !Q), "8-byte vectors: 2-byte rows, no E4M3 copy");
    constexpr int E = VB / VI::BYTES;  // elements per input vector
    constexpr int G = 128 / E;  // lanes per 128-value E4M3 group
    __shared__ float red[2][4 * 16];  // one region per reduction

    const int lane = threadIdx.x & 63;
    const int wave = wave_id();
    const int group = wave / wpr;
    const int wig = wave - group * wpr;
    const int groups = blockDim.x / (64 * wpr);
    const int64_t row0 = static_cast<int64_t>(blockIdx.x) * groups + group;
    const int tpr = 64 * wpr;
    const int t = wig * 64 + lane;
    const int nvec = static_cast<int>(a.D / E);

    // Every load and store below is unconditional and each lane issues the same number of them: a lane
    // past the row's end works on the row's last vector and a group past the last row on the last row,
    // storing the same bytes as their owners, and masked values are kept out of the sums. (A memory
    // operation under a divergent branch makes the compiler wait for all outstanding ones afterwards.)
    // With E4M3 rows (D a multiple of 128) a lane past the end takes its place in the row's last 128-value
    // group instead, so that a whole group of such lanes repeats that group's codes and scale exactly.
    const int64_t row = row0 < a.rows ? row0 : a.rows - 1;
    int jv[NV];
    bool own[NV];
#pragma unroll
    for (int k = 0; k < NV; k++) {
        const int j = t + k * tpr;
        own[k] = j < nvec;
        jv[k] = own[k] ? j : Q ? nvec - G + (j & (G - 1)) : nvec - 1;
    }
    const char* xr = static_cast<const char*>(a.x) + row * a.xs * VI::BYTES;
    typename RV::T raw[NV], rraw[NV];
#pragma unroll
    for (int k = 0; k < NV; k++) raw[k] = RV::load(xr + static_cast<int64_t>(jv[k]) * VB);
    if (RES) {
        const char* rr = static_cast<const char*>(a.res) + row * a.rs * VI::BYTES;
#pragma unroll
        for (int k = 0; k < NV; k++) rraw[k] = RV::load(rr + static_cast<int64_t>(jv[k]) * VB);
    }
    // The norm weight is read with the row data, ahead of the reduction, rather than after it.
    float wv[NV][E];
    const bool has_w = a.w != nullptr, has_b = a.b != nullptr;
    constexpr bool W_EARLY = RES || DTI == SLHIP_F32;  // a packed row reads it after the reductions
    if (W_EARLY && has_w) {
#pragma unroll
        for (int k = 0; k < NV; k++) {
            const float4* wp = reinterpret_cast<const float4*>(a.w + static_cast<int64_t>(jv[k]) * E);
#pragma unroll
            for (int q4 = 0; q4 < E / 4; q4++) {
                const float4 w4 = wp[q4];
                wv[k][4 * q4 + 0] = w4.x;
                wv[k][4 * q4 + 1] = w4.y;
                wv[k][4 * q4 + 2] = w4.z;
                wv[k][4 * q4 + 3] = w4.w;
            }
        }
    }

    // Without a residual the row stays in registers as loaded (a 2-byte row in half the registers of its
    // f32 values) and is widened again in each pass; the empty asm statements stop the compiler from
    // keeping the widened values alive across the reductions instead. The registers saved double the
    // waves resident per SIMD, i.e. the bytes in flight, which is what a 2-stream norm lacks.
    constexpr bool PACKED = !RES && DTI != SLHIP_F32;
    auto launder = [&]() {
        if constexpr (PACKED) {
#pragma unroll
            for (int k = 0; k < NV; k++) RV::launder(raw[k]);
        }
    };
    float v[NV][E];
#pragma unroll
    for (int k = 0; k < NV; k++) {
        RV::template unpack<DTI>(raw[k], v[k]);
        if (RES) {
            float rf[E];
            RV::template unpack<DTI>(rraw[k], rf);
#pragma unroll
            for (int e = 0; e < E; e++) v[k][e] += rf[e];
        }
    }
    // In-place calls (y over x, h over res) are safe because no store is issued before every wave of the
    // block holds all of its loaded data: the first reduction consumes every loaded value of the wave (and,
    // with WPR > 1, ends in a block barrier), and every store comes after it. Lanes past the row's end then
    // store the bytes their owners store, computed from the same unmodified inputs. A group past the last
    // row (possible only with one wave per row, where no barrier orders it against the owning wave) stores
    // nothing: its test is wave-uniform, so the branch is scalar.
    const bool store_row = row0 < a.rows;
    auto store_h = [&]() {
        if (RES && a.h && store_row) {
            char* hr = static_cast<char*>(a.h) + row * a.hs * VI::BYTES;
#pragma unroll
            for (int k = 0; k < NV; k++) store_nt(hr + static_cast<int64_t>(jv[k]) * VB, RV::template pack<DTI>(v[k]));
        }
    };

    const float inv_d = 1.0f / static_cast<float>(a.D);
    float mean = 0.f, scale;
    if (a.kind == SLHIP_NORM_LAYER) {
        float s = 0.f;
#pragma unroll
        for (int k = 0; k < NV; k++)
#pragma unroll
            for (int e = 0; e < E; e++) s += own[k] ? v[k][e] : 0.0f;
        mean = group_reduce<4>(s, wpr, group, wig, red[0]) * inv_d;
        store_h();
        launder();
        float q = 0.f;
#pragma unroll
        for (int k = 0; k < NV; k++) {
            if constexpr (PACKED) RV::template unpack<DTI>(raw[k], v[k]);
#pragma unroll
            for (int e = 0; e < E; e++) {
                const float d = own[k] ? v[k][e] - mean : 0.0f;
                q = fmaf(d, d, q);
            }
        }
        const float var = group_reduce<4>(q, wpr, group, wig, red[1]) * inv_d;
        scale = 1.0f / sqrtf(var + a.eps);
    } else {
        float q = 0.f;
#pragma unroll
        for (int k = 0; k < NV; k++)
#pragma unroll
            for (int e = 0; e < E; e++) {
                const float x = own[k] ? v[k][e] : 0.0f;
                q = fmaf(x, x, q);
            }
        const float ss = group_reduce<4>(q, wpr, group, wig, red[1]);
        store_h();
        scale = a.kind == SLHIP_NORM_RMS ? 1.0f / sqrtf(ss * inv_d + a.eps) : 1.0f / sqrtf(ss + a.eps);
    }

    if (!store_row) return;
    launder();
    // Unpacked rows (f32, or with a residual) load the LayerNorm bias for every vector here, ahead of the
    // stores (a load used inside its own branch is waited for before the next vector's loads go out:
    // [197, 768] f32 3.40 -> 3.23 us); a packed row loads weight and bias per vector (both before either is
    // used), as the registers of all of them would cost the packed row its occupancy ([8192, 4096] bf16:
    // 29.4 -> 30.6 us).
    float bv[NV][E];
    if (!PACKED && has_b) {
#pragma unroll
        for (int k = 0; k < NV; k++) {
            const float4* bp = reinterpret_cast<const float4*>(a.b + static_cast<int64_t>(jv[k]) * E);
#pragma unroll
            for (int q4 = 0; q4 < E / 4; q4++) {
                const float4 b4 = bp[q4];
                bv[k][4 * q4 + 0] = b4.x;
                bv[k][4 * q4 + 1] = b4.y;
                bv[k][4 * q4 + 2] = b4.z;
                bv[k][4 * q4 + 3] = b4.w;
            }
        }
    }
    char* yr = static_cast<char*>(a.y) + row * a.ys * Vec<DTO>::BYTES;
    char* y16r = static_cast<char*>(a.y16) + row * a.y16s * 2;
    char* qr = static_cast<char*>(a.yq) + row * a.yqs;
#pragma unroll
    for (int k = 0; k < NV; k++) {
        // a packed row's weight and bias for this vector, both loads out before either is used
        if constexpr (!W_EARLY) {
            if (has_w) {
                const float4* wp = reinterpret_cast<const float4*>(a.w + static_cast<int64_t>(jv[k]) * E);
#pragma unroll
                for (int q4 = 0; q4 < E / 4; q4++) {
                    const float4 w4 = wp[q4];
                    wv[k][4 * q4 + 0] = w4.x;
                    wv[k][4 * q4 + 1] = w4.y;
                    wv[k][4 * q4 + 2] = w4.z;
                    wv[k][4 * q4 + 3] = w4.w;
                }
            }
        }
        if constexpr (PACKED) {
            if (has_b) {
                const float4* bp = reinterpret_cast<const float4*>(a.b + static_cast<int64_t>(jv[k]) * E);
#pragma unroll
                for (int q4 = 0; q4 < E / 4; q4++) {
                    const float4 b4 = bp[q4];
                    bv[k][4 * q4 + 0] = b4.x;
                    bv[k][4 * q4 + 1] = b4.y;
                    bv[k][4 * q4 + 2] = b4.z;
                    bv[k][4 * q4 + 3] = b4.w;
                }
            }
        }
        if constexpr (PACKED) RV::template unpack<DTI>(raw[k], v[k]);
        float o[E];
        if (a.kind == SLHIP_NORM_LAYER) {
#pragma unroll
            for (int e = 0; e < E; e++) o[e] = (v[k][e] - mean) * scale;
        } else {
#pragma unroll
            for (int e = 0; e < E; e++) o[e] = v[k][e] * scale;
        }
        if (has_w) {
#pragma unroll
            for (int e = 0; e < E; e++) o[e] *= wv[k][e];
        }
        if (has_b) {
#pragma unroll
            for (int e = 0; e < E; e++) o[e] += bv[k][e];
        }
        if (a.y) store_packed<DTO, E>(yr + static_cast<int64_t>(jv[k]) * E * Vec<DTO>::BYTES, o);
        if (a.y16) store_packed<SLHIP_F16, E>(y16r + static_cast<int64_t>(jv[k]) * E * 2, o);
        if (Q) {
            // quantize_fp8 on the group (src/Sharplight.Shaders/Kernels/gemm_fp8.slang:36-55): d = amax/448,
            // codes of o * (1/d); every lane of the group stores the same scale.
            float m = 0.0f;
#pragma unroll
            for (int e = 0; e < E; e++) m = fmaxf(m, fabsf(o[e]));
            m = group_max_nonneg<G>(m);  // m is not NaN: the first fmaxf with 0 drops quiet NaNs
            float d, id;
            e4m3_group_scale(m, d, id);
            char* qp = qr + static_cast<int64_t>(jv[k]) * E;
            if constexpr (E == 8)
                store_nt(qp, make_uint2(e4m3_pack4(o, id), e4m3_pack4(o + 4, id)));
            else
                store_nt(qp, e4m3_pack4(o, id));
            store_nt(qr + a.D + static_cast<int64_t>(jv[k] / G) * 4, __float_as_uint(d));
        }
    }
}

// Sums of R rows over their row groups at once: the same butterfly and the same LDS order per row as
// group_reduce, with one barrier for all R. Each call of a kernel passes its own LDS region, so no barrier
// is needed ahead of the writes.
template <int R>
__device__ __forceinline__ void group_reduce_rows(float* v, int wpr, int group, int wave_in_group, float* red)
{
#pragma unroll
    for (int i = 0; i < R; i++) v[i] = wave_sum(v[i]);
    if (wpr == 1) return;
    if ((threadIdx.x & 63) == 0) {
#pragma unroll
        for (int i = 0; i < R; i++) red[(group * 16 + wave_in_group) * R + i] = v[i];
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < R; i++) {
        float s = 0.f;
        for (int w = 0; w < wpr; w++) s += red[(group * 16 + w) * R + i];
        v[i] = s;
    }
}

// Two-byte rows without a residual or copies, R rows per row group: the group loads all R rows, reduces
// them together and then, per vector, reads the norm weight and bias once for the R rows. Each row's
// arithmetic (and so its result) is that of rownorm_vec; what changes is that the f32 weight and bias,
// which are 4x the row's bytes between them for a bf16 LayerNorm and come from the L2 for every row, are
// read once per R rows, and the block barriers of the reductions are shared by the R rows.
template <int DTI, int DTO, int NV, int R>
__global__ __launch_bounds__(1024) __attribute__((amdgpu_waves_per_eu(5))) void rownorm_rows(RowNormArgs a, int wpr)
{
    using VI = Vec<DTI>;
    using RV = RawVec<16>;
    static_assert(VI::BYTES == 2, "rows of 2-byte values");
    constexpr int E = 16 / VI::BYTES;
    __shared__ float red[2][4 * 16 * R];  // one region per reduction
    __shared__ float red3[4 * 16 * R * 3];  // LayerNorm: (sum, M2, count) per wave and row

    const int lane = threadIdx.x & 63;
    const int wave = wave_id();
    const int group = wave / wpr;
    const int wig = wave - group * wpr;
    const int groups = blockDim.x / (64 * wpr);
    const int64_t row0 = (static_cast<int64_t>(blockIdx.x) * groups + group) * R;
    const int tpr = 64 * wpr;
    const int t = wig * 64 + lane;
    const int nvec = static_cast<int>(a.D / E);

    // As in rownorm_vec: unconditional loads and stores, lanes past the row's end on its last vector, rows
    // past the last row on the last row (and storing nothing).
    int jv[NV];
    bool own[NV];
#pragma unroll
    for (int k = 0; k < NV; k++) {
        const int j = t + k * tpr;
        own[k] = j < nvec;
        jv[k] = own[k] ? j : nvec - 1;
    }
    int64_t row[R];
    RV::T raw[R][NV];
#pragma unroll
    for (int i = 0; i < R; i++) {
        row[i] = row0 + i < a.rows ? row0 + i : a.rows - 1;
        const char* xr = static_cast<const char*>(a.x) + row[i] * a.xs * VI::BYTES;
#pragma unroll
        for (int k = 0; k < NV; k++) raw[i][k] = RV::load(xr + static_cast<int64_t>(jv[k]) * 16);
    }
    const bool has_w = a.w != nullptr, has_b = a.b != nullptr;
    // the weight and bias of a vector are loaded once for the R rows (loading the next vector's ahead, or the
    // first one's with the rows, measured ~6% slower: the registers cost a wave per SIMD)
    auto load_wb = [&](int k, float* w8, float* b8) {
        if (has_w) {
            const float4* wp = reinterpret_cast<const float4*>(a.w + static_cast<int64_t>(jv[k]) * E);
#pragma unroll
            for (int q4 = 0; q4 < E / 4; q4++) {
                const float4 w4 = wp[q4];
                w8[4 * q4 + 0] = w4.x;
                w8[4 * q4 + 1] = w4.y;
                w8[4 * q4 + 2] = w4.z;
                w8[4 * q4 + 3] = w4.w;
            }
        }
        if (has_b) {
            const float4* bp = reinterpret_cast<const float4*>(a.b + static_cast<int64_t>(jv[k]) * E);
#pragma unroll
            for (int q4 = 0; q4 < E / 4; q4++) {
                const float4 b4 = bp[q4];
                b8[4 * q4 + 0] = b4.x;
                b8[4 * q4 + 1] = b4.y;
                b8[4 * q4 + 2] = b4.z;
                b8[4 * q4 + 3] = b4.w;
            }
        }
    };
    auto launder = [&]() {
#pragma unroll
        for (int i = 0; i < R; i++)
#pragma unroll
            for (int k = 0; k < NV; k++) RV::launder(raw[i][k]);
    };

    const float inv_d = 1.0f / static_cast<float>(a.D);
    float mean[R], scale[R];
    if (a.kind == SLHIP_NORM_LAYER) {
        // mean and variance with one exchange across the group's waves: each lane's count, sum and sum of
        // squared deviations about its own mean (from its registers), combined within the wave and then
        // across waves by the exact identity M2 = sum M2_p + n_p (m_p - m)^2 over the parts p (stable: no
        // difference of large sums); mean = sum x / D. Against two exchanges (sum, then the deviations about
        // the mean) on bf16 [8192, 4096]: 28.6 against 28.9 us, within the noise; kept for the one barrier.
        float S[R], M[R], n_w[R];
#pragma unroll
        for (int i = 0; i < R; i++) {
            float sl = 0.f, nl = 0.f;
#pragma unroll
            for (int k = 0; k < NV; k++) {
                float v[E];
                RV::template unpack<DTI>(raw[i][k], v);
#pragma unroll
                for (int e = 0; e < E; e++) sl += own[k] ? v[e] : 0.0f;
                nl += own[k] ? static_cast<float>(E) : 0.0f;
            }
            const float ml = nl > 0.f ? sl / nl : 0.0f;
            float ql = 0.f;
#pragma unroll
            for (int k = 0; k < NV; k++) {
                float v[E];
                RV::template unpack<DTI>(raw[i][k], v);
#pragma unroll
                for (int e = 0; e < E; e++) {
                    const float d = own[k] ? v[e] - ml : 0.0f;
                    ql = fmaf(d, d, ql);
                }
            }
            S[i] = wave_sum(sl);
            n_w[i] = wave_sum(nl);
            const float mw = n_w[i] > 0.f ? S[i] / n_w[i] : 0.0f;
            const float dm = ml - mw;
            M[i] = wave_sum(fmaf(nl * dm, dm, ql));
        }
        if (wpr > 1) {
            if (lane == 0) {
#pragma unroll
                for (int i = 0; i < R; i++) {
                    float* e3 = &red3[((group * 16 + wig) * R + i) * 3];
                    e3[0] = S[i];
                    e3[1] = M[i];
                    e3[2] = n_w[i];
                }
            }
            __syncthreads();
#pragma unroll
            for (int i = 0; i < R; i++) {
                float st = 0.f;
                for (int w = 0; w < wpr; w++) st += red3[((group * 16 + w) * R + i) * 3];
                const float m = st * inv_d;
                float mt = 0.f;
                for (int w = 0; w < wpr; w++) {
                    const float* e3 = &red3[((group * 16 + w) * R + i) * 3];
                    const float dm = e3[2] > 0.f ? e3[0] / e3[2] - m : 0.0f;
                    mt += fmaf(e3[2] * dm, dm, e3[1]);
                }
                S[i] = st;
                M[i] = mt;
            }
        }
        launder();
#pragma unroll
        for (int i = 0; i < R; i++) {
            mean[i] = S[i] * inv_d;
            scale[i] = 1.0f / sqrtf(M[i] * inv_d + a.eps);
        }
    } else {
        float q[R];
#pragma unroll
        for (int i = 0; i < R; i++) {
            mean[i] = 0.f;
            q[i] = 0.f;
#pragma unroll
            for (int k = 0; k < NV; k++) {
                float v[E];
                RV::template unpack<DTI>(raw[i][k], v);
#pragma unroll
                for (int e = 0; e < E; e++) {
                    const float x = own[k] ? v[e] : 0.0f;
                    q[i] = fmaf(x, x, q[i]);
                }
            }
        }
        group_reduce_rows<R>(q, wpr, group, wig, red[1]);
#pragma unroll
        for (int i = 0; i < R; i++)
            scale[i] = a.kind == SLHIP_NORM_RMS ? 1.0f / sqrtf(q[i] * inv_d + a.eps) : 1.0f / sqrtf(q[i] + a.eps);
    }
    if (row0 >= a.rows) return;
    launder();
#pragma unroll
    for (int k = 0; k < NV; k++) {
        float w8[E], b8[E];
        load_wb(k, w8, b8);
#pragma unroll
        for (int i = 0; i < R; i++) {
            if (row0 + i >= a.rows) break;  // wave-uniform
            float v[E], o[E];
            RV::template unpack<DTI>(raw[i][k], v);
            if (a.kind == SLHIP_NORM_LAYER) {
#pragma unroll
                for (int e = 0; e < E; e++) o[e] = (v[e] - mean[i]) * scale[i];
            } else {
#pragma unroll
                for (int e = 0; e < E; e++) o[e] = v[e] * scale[i];
            }
            if (has_w) {
#pragma unroll
                for (int e = 0; e < E; e++) o[e] *= w8[e];
            }
            if (has_b) {
#pragma unroll
                for (int e = 0; e < E; e++) o[e] += b8[e];
            }
            char* yr = static_cast<char*>(a.y) + row[i] * a.ys * Vec<DTO>::BYTES;
            store_packed<DTO, E>(yr + static_cast<int64_t>(jv[k]) * E * Vec<DTO>::BYTES, o);
        }
    }
}

// Two-byte rows without a residual or copies, persistent: a block is one row group of wpr waves that keeps
// its lanes' weight and bias vectors in registers for the whole launch (read from L2 once per block, where
// rownorm_rows reads them per row pair) and walks row pairs b, b + B, ... (B blocks, each with the same
// count `per`); the next pair's rows are loaded before the current pair is reduced and stored. The
// arithmetic per row is rownorm_rows's.
template <int DTI, int DTO, int NV>
__global__ __launch_bounds__(1024) void rownorm_rows_p(RowNormArgs a, int wpr, int64_t per)
{
    using VI = Vec<DTI>;
    using RV = RawVec<16>;
    static_assert(VI::BYTES == 2, "rows of 2-byte values");
    constexpr int E = 16 / VI::BYTES;
    constexpr int R = 2;
    __shared__ float red[2][16 * R];  // one region per reduction

    const int lane = threadIdx.x & 63;
    const int wave = wave_id();
    const int t = wave * 64 + lane;
    const int tpr = 64 * wpr;
    const int nvec = static_cast<int>(a.D / E);
    int jv[NV];
    bool own[NV];
#pragma unroll
    for (int k = 0; k < NV; k++) {
        const int j = t + k * tpr;
        own[k] = j < nvec;
        jv[k] = own[k] ? j : nvec - 1;
    }
    const bool has_w = a.w != nullptr, has_b = a.b != nullptr;
    float w[NV][E], b[NV][E];
#pragma unroll
    for (int k = 0; k < NV; k++) {
#pragma unroll
        for (int q4 = 0; q4 < E / 4; q4++) {
            const float4 w4 = has_w ? reinterpret_cast<const float4*>(a.w + static_cast<int64_t>(jv[k]) * E)[q4] : make_float4(1.f, 1.f, 1.f, 1.f);
            const float4 b4 = has_b ? reinterpret_cast<const float4*>(a.b + static_cast<int64_t>(jv[k]) * E)[q4] : make_float4(0.f, 0.f, 0.f, 0.f);
            w[k][4 * q4 + 0] = w4.x;
            w[k][4 * q4 + 1] = w4.y;
            w[k][4 * q4 + 2] = w4.z;
            w[k][4 * q4 + 3] = w4.w;
            b[k][4 * q4 + 0] = b4.x;
            b[k][4 * q4 + 1] = b4.y;
            b[k][4 * q4 + 2] = b4.z;
            b[k][4 * q4 + 3] = b4.w;
        }
    }
    const int64_t B = gridDim.x;
    const float inv_d = 1.0f / static_cast<float>(a.D);
    // rows past the last are loaded as the last row and not stored
    auto clamp_row = [&](int64_t r) { return r < a.rows ? r : a.rows - 1; };
    auto load_pair = [&](RV::T (&raw)[R][NV], int64_t pair) {
#pragma unroll
        for (int i = 0; i < R; i++) {
            const char* xr = static_cast<const char*>(a.x) + clamp_row(pair * R + i) * a.xs * VI::BYTES;
#pragma unroll
            for (int k = 0; k < NV; k++) raw[i][k] = RV::load(xr + static_cast<int64_t>(jv[k]) * 16);
        }
    };
    auto process = [&](RV::T (&raw)[R][NV], int64_t pair) {
        auto launder = [&]() {
#pragma unroll
            for (int i = 0; i < R; i++)
#pragma unroll
                for (int k = 0; k < NV; k++) RV::launder(raw[i][k]);
        };
        float mean[R], scale[R];
        if (a.kind == SLHIP_NORM_LAYER) {
            float s[R];
#pragma unroll
            for (int i = 0; i < R; i++) {
                s[i] = 0.f;
#pragma unroll
                for (int k = 0; k < NV; k++) {
                    float v[E];
                    RV::template unpack<DTI>(raw[i][k], v);
#pragma unroll
                    for (int e = 0; e < E; e++) s[i] += own[k] ? v[e] : 0.0f;
                }
            }
            group_reduce_rows<R>(s, wpr, 0, wave, red[0]);
            launder();
            float q[R];
#pragma unroll
            for (int i = 0; i < R; i++) {
                mean[i] = s[i] * inv_d;
                q[i] = 0.f;
#pragma unroll
                for (int k = 0; k < NV; k++) {
                    float v[E];
                    RV::template unpack<DTI>(raw[i][k], v);
#pragma unroll
                    for (int e = 0; e < E; e++) {
                        const float d = own[k] ? v[e] - mean[i] : 0.0f;
                        q[i] = fmaf(d, d, q[i]);
                    }
                }
            }
            group_reduce_rows<R>(q, wpr, 0, wave, red[1]);
#pragma unroll
            for (int i = 0; i < R; i++) scale[i] = 1.0f / sqrtf(q[i] * inv_d + a.eps);
        } else {
            float q[R];
#pragma unroll
            for (int i = 0; i < R; i++) {
                mean[i] = 0.f;
                q[i] = 0.f;
#pragma unroll
                for (int k = 0; k < NV; k++) {
                    float v[E];
                    RV::template unpack<DTI>(raw[i][k], v);
#pragma unroll
                    for (int e = 0; e < E; e++) {
                        const float x = own[k] ? v[e] : 0.0f;
                        q[i] = fmaf(x, x, q[i]);
                    }
                }
            }
            group_reduce_rows<R>(q, wpr, 0, wave, red[1]);
#pragma unroll
            for (int i = 0; i < R; i++)
                scale[i] = a.kind == SLHIP_NORM_RMS ? 1.0f / sqrtf(q[i] * inv_d + a.eps) : 1.0f / sqrtf(q[i] + a.eps);
        }
        launder();
#pragma unroll
        for (int i = 0; i < R; i++) {
            const int64_t r = pair * R + i;
            if (r >= a.rows) break;  // block-uniform
#pragma unroll
            for (int k = 0; k < NV; k++) {
                float v[E], o[E];
                RV::template unpack<DTI>(raw[i][k], v);
                if (a.kind == SLHIP_NORM_LAYER) {
#pragma unroll
                    for (int e = 0; e < E; e++) o[e] = (v[e] - mean[i]) * scale[i];
                } else {
#pragma unroll
                    for (int e = 0; e < E; e++) o[e] = v[e] * scale[i];
                }
                if (has_w) {
#pragma unroll
                    for (int e = 0; e < E; e++) o[e] *= w[k][e];
                }
                if (has_b) {
#pragma unroll
                    for (int e = 0; e < E; e++) o[e] += b[k][e];
                }
                char* yr = static_cast<char*>(a.y) + r * a.ys * Vec<DTO>::BYTES;
                store_packed<DTO, E>(yr + static_cast<int64_t>(jv[k]) * E * Vec<DTO>::BYTES, o);
            }
        }
    };
    RV::T A[R][NV], C[R][NV];
    int64_t pair = blockIdx.x;
    load_pair(A, pair);
    for (int64_t it = 0; it < per; it += 2) {  // two pairs per pass: the register sets alternate statically
        if (it + 1 < per) load_pair(C, pair + B);
        process(A, pair);
        if (it + 1 >= per) break;
        if (it + 2 < per) load_pair(A, pair + 2 * B);
        process(C, pair + B);
        pair += 2 * B;
    }
}

// Scalar fallback: one 256-thread block per row, re-reading the row from global memory (cache-resident)
// for each pass.
template <int DTI, int DTO>
__global__ __launch_bounds__(256) void rownorm_scalar(RowNormArgs a)
{
    using VI = Vec<DTI>;
    __shared__ float red[4];
    const int64_t row = blockIdx.x;
    const void* xr = static_cast<const char*>(a.x) + row * a.xs * VI::BYTES;
    const void* rr = a.res ? static_cast<const char*>(a.res) + row * a.rs * VI::BYTES : nullptr;
    void* hr = (a.res && a.h) ? static_cast<char*>(a.h) + row * a.hs * VI::BYTES : nullptr;
    void* yr = a.y ? static_cast<char*>(a.y) + row * a.ys * Vec<DTO>::BYTES : nullptr;
    void* y16r = a.y16 ? static_cast<char*>(a.y16) + row * a.y16s * 2 : nullptr;
    char* qr = a.yq ? static_cast<char*>(a.yq) + row * a.yqs : nullptr;
    const int64_t D = a.D;

    auto reduce = [&](float s) {
        s = wave_sum(s);
        __syncthreads();
        if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
        __syncthreads();
        return red[0] + red[1] + red[2] + red[3];
    };
    auto value = [&](int64_t i) {
        float v = VI::load1(xr, i);
        if (rr) v += VI::load1(rr, i);
        return v;
    };

    float mean = 0.f, scale;
    if (a.kind == SLHIP_NORM_LAYER) {
        float s = 0.f;
        for (int64_t i = threadIdx.x; i < D; i += 256) s += value(i);
        mean = reduce(s) / static_cast<float>(D);
        float q = 0.f;
        for (int64_t i = threadIdx.x; i < D; i += 256) {
            float d = value(i) - mean;
            q = fmaf(d, d, q);
        }
        scale = 1.0f / sqrtf(reduce(q) / static_cast<float>(D) + a.eps);
    } else {
        float q = 0.f;
        for (int64_t i = threadIdx.x; i < D; i += 256) {
            float v = value(i);
            q = fmaf(v, v, q);
        }
        float ss = reduce(q);
        scale = a.kind == SLHIP_NORM_RMS ? 1.0f / sqrtf(ss / static_cast<float>(D) + a.eps) : 1.0f / sqrtf(ss + a.eps);
    }
    auto normed = [&](float v, int64_t i) {
        float o = a.kind == SLHIP_NORM_LAYER ? (v - mean) * scale : v * scale;
        if (a.w) o *= a.w[i];
        if (a.b) o += a.b[i];
        return o;
    };
    // The E4M3 rows re-read the inputs, so they are written first and a barrier separates them from the
    // stores of y and h, which may overwrite x and res (in-place calls).
    if (qr) {  // one wave per 128-value group, two values per lane
        const int lane = threadIdx.x & 63;
        for (int64_t g = threadIdx.x >> 6; g < D / 128; g += 4) {
            const int64_t i0 = g * 128 + lane, i1 = i0 + 64;
            const float o0 = normed(value(i0), i0), o1 = normed(value(i1), i1);
            const float d = group_max<64>(fmaxf(fabsf(o0), fabsf(o1))) / 448.0f;
            const float id = d > 0.0f ? 1.0f / d : 0.0f;  // the division itself: this path is not hot
            qr[i0] = static_cast<char>(e4m3_code(o0 * id));
            qr[i1] = static_cast<char>(e4m3_code(o1 * id));
            if (lane == 0) *reinterpret_cast<float*>(qr + D + g * 4) = d;
        }
    }
    if (qr) __syncthreads();
    for (int64_t i = threadIdx.x; i < D; i += 256) {
        float v = value(i);
        if (hr) VI::store1(hr, i, v);
        const float o = normed(v, i);
        if (yr) Vec<DTO>::store1(yr, i, o);
        if (y16r) Vec<SLHIP_F16>::store1(y16r, i, o);
    }
}

// ---- host dispatch --------------------------------------------------------------------------------

static int env_int(const char* name, int dflt)
{
    const char* s = getenv(name);
    return s && *s ? atoi(s) : dflt;
}

template <int DTI, int DTO, bool RES, bool Q, int VB>
static int launch_vec(const RowNormArgs& a, int nv, int wpr, hipStream_t st)
{
    int groups = wpr >= 4 ? 1 : 4 / wpr;
    int threads = 64 * wpr * groups;
    dim3 grid(static_cast<unsigned>((a.rows + groups - 1) / groups));
    switch (nv) {
    case 1: rownorm_vec<DTI, DTO, 1, RES, Q, VB><<<grid, threads, 0, st>>>(a, wpr); break;
    case 2: rownorm_vec<DTI, DTO, 2, RES, Q, VB><<<grid, threads, 0, st>>>(a, wpr); break;
    case 3: rownorm_vec<DTI, DTO, 3, RES, Q, VB><<<grid, threads, 0, st>>>(a, wpr); break;
    case 4: rownorm_vec<DTI, DTO, 4, RES, Q, VB><<<grid, threads, 0, st>>>(a, wpr); break;
    case 5: rownorm_vec<DTI, DTO, 5, RES, Q, VB><<<grid, threads, 0, st>>>(a, wpr); break;
    case 6: rownorm_vec<DTI, DTO, 6, RES, Q, VB><<<grid, threads, 0, st>>>(a, wpr); break;
    case 8: rownorm_vec<DTI, DTO, 8, RES, Q, VB><<<grid, threads, 0, st>>>(a, wpr); break;
    default: return fail(SLHIP_ERR_INVALID, "internal: bad vector count %d", nv);
    }
    return check_launch("rownorm_vec");
}

template <int DTI, int DTO, int R>
static int launch_rows(const RowNormArgs& a, int nv, int wpr, hipStream_t st)
{
    int groups = wpr >= 4 ? 1 : 4 / wpr;
    int threads = 64 * wpr * groups;
    dim3 grid(static_cast<unsigned>((a.rows + groups * R - 1) / (groups * R)));
    switch (nv) {
    case 1: rownorm_rows<DTI, DTO, 1, R><<<grid, threads, 0, st>>>(a, wpr); break;
    case 2: rownorm_rows<DTI, DTO, 2, R><<<grid, threads, 0, st>>>(a, wpr); break;
    case 3: rownorm_rows<DTI, DTO, 3, R><<<grid, threads, 0, st>>>(a, wpr); break;
    case 4: rownorm_rows<DTI, DTO, 4, R><<<grid, threads, 0, st>>>(a, wpr); break;
    default: return fail(SLHIP_ERR_INVALID, "internal: bad vector count %d", nv);
    }
    return check_launch("rownorm_rows");
}

template <int DTI, int DTO>
static int launch_rows_p(const RowNormArgs& a, int64_t nvec, hipStream_t st)
{
    // the smallest row group whose lanes hold at most two vectors, then one block per group
    int wpr = 1;
    while (wpr < 16 && nvec > static_cast<int64_t>(2) * 64 * wpr) wpr *= 2;
    const int nv = static_cast<int>((nvec + 64 * wpr - 1) / (64 * wpr));
    const void* k = nv == 1 ? reinterpret_cast<const void*>(rownorm_rows_p<DTI, DTO, 1>)
                            : reinterpret_cast<const void*>(rownorm_rows_p<DTI, DTO, 2>);
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k, 64 * wpr, 0) != hipSuccess || per_cu < 1) per_cu = 1;
    static int cus = 0;
    if (!cus) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            cus <= 0)
            cus = 256;
    }
    const int64_t pairs = (a.rows + 1) / 2;
    const int64_t resident = static_cast<int64_t>(cus) * per_cu;
    const int64_t per = (pairs + resident - 1) / resident;
    const dim3 grid(static_cast<unsigned>((pairs + per - 1) / per));
    if (nv == 1) rownorm_rows_p<DTI, DTO, 1><<<grid, 64 * wpr, 0, st>>>(a, wpr, per);
    else rownorm_rows_p<DTI, DTO, 2><<<grid, 64 * wpr, 0, st>>>(a, wpr, per);
    return check_launch("rownorm_rows_p");
}

static bool aligned_to(const void* p, int n) { return reinterpret_cast<uintptr_t>(p) % n == 0; }

// Whether the rows fit the vector kernel with VB-byte input vectors: D a multiple of the vector's values,
// every pointer and row stride aligned to the accesses the kernel makes (inputs and h: VB bytes; y and the
// f16 copy: the values of one vector at the output width, at most 16 bytes; w and b: 16-byte loads), and
// at most 8 vectors per lane of a 16-wave row group.
template <int DTI, int DTO, int VB>
static bool vec_fits(const RowNormArgs& a)
{
    constexpr int E = VB / Vec<DTI>::BYTES;
    constexpr int OA = E * Vec<DTO>::BYTES < 16 ? E * Vec<DTO>::BYTES : 16;
    constexpr int HA = E * 2 < 16 ? E * 2 : 16;
    return a.D % E == 0 && a.D / E <= 8 * 64 * 16 && aligned_to(a.x, VB) && a.xs % E == 0 &&
           (!a.res || (aligned_to(a.res, VB) && a.rs % E == 0)) && (!a.h || (aligned_to(a.h, VB) && a.hs % E == 0)) &&
           aligned_to(a.y, OA) && (a.ys * Vec<DTO>::BYTES) % OA == 0 && aligned_to(a.y16, HA) &&
           (a.y16s * 2) % HA == 0 && aligned_to(a.yq, E) && a.yqs % E == 0 && (!a.w || aligned16(a.w)) &&
           (!a.b || aligned16(a.b));
}

template <int DTI, int DTO, int VB>
static int launch_fitting(const RowNormArgs& a, hipStream_t st)
{
    const int64_t nvec = a.D / (VB / Vec<DTI>::BYTES);
    // Row group sized for at most 64 bytes per lane and input (4 vectors of 16 bytes, 8 of 8): measured on
    // MI355X at [8192, 4096] bf16 (residual add) 4 vectors of 16 bytes beat 2 by ~2.5% and 8 (one wave per
    // row) by more; at [8192, 4100] five 8-byte vectors over four waves beat three over eight by 7%.
    // Widened further while the launch has fewer than ~4096 waves. Lanes take 1-6 or 8 vectors, so that a
    // row just beyond a power of two leaves fewer lanes idle.
    constexpr int LANE_VECS = 64 / VB;
    int wpr = 1;
    while (wpr < 16 && nvec > static_cast<int64_t>(LANE_VECS) * 64 * wpr) wpr *= 2;
    while (wpr < 16 && a.rows * wpr < 4096 && nvec >= static_cast<int64_t>(64) * wpr * 2) wpr *= 2;
    int forced = env_int("SLHIP_ROWNORM_WPR", 0);
    if (forced == 1 || forced == 2 || forced == 4 || forced == 8 || forced == 16) {
        if (nvec <= static_cast<int64_t>(8) * 64 * forced) wpr = forced;
    }
    int64_t per = (nvec + 64 * wpr - 1) / (64 * wpr);
    int nv = per == 7 ? 8 : static_cast<int>(per);
    if constexpr (VB == 16 && Vec<DTI>::BYTES == 2) {
        // two-byte rows without a residual or copies (SLHIP_ROWNORM_ROWS): 3 (default), RMS and L2 rows up to
        // 16384 values on persistent row groups holding their weight (bf16 [8192, 4096] RMSNorm 26.2 -> 25.5 us;
        // LayerNorm measured slower so, 27.9 -> 29.5: two block barriers per row pair on 4-wave groups, and
        // the bias's registers cost a wave per SIMD); 2 (and LayerNorm), two rows per row group up to 4 vectors
        // per lane (beyond that two rows' registers spill at 1024-thread blocks); 1, rownorm_vec
        const int r = env_int("SLHIP_ROWNORM_ROWS", 3);
        if (!a.res && !a.yq && !a.y16 && a.y && r == 3 && a.kind != SLHIP_NORM_LAYER && nvec <= 2 * 64 * 16)
            return launch_rows_p<DTI, DTO>(a, nvec, st);
        if (!a.res && !a.yq && !a.y16 && a.y && r >= 2 && nv <= 4) return launch_rows<DTI, DTO, 2>(a, nv, wpr, st);
    }
    if constexpr (VB == 16) {
        if (a.yq)
            return a.res ? launch_vec<DTI, DTO, true, true, VB>(a, nv, wpr, st)
                         : launch_vec<DTI, DTO, false, true, VB>(a, nv, wpr, st);
    }
    return a.res ? launch_vec<DTI, DTO, true, false, VB>(a, nv, wpr, st)
                 : launch_vec<DTI, DTO, false, false, VB>(a, nv, wpr, st);
}

template <int DTI, int DTO>
static int dispatch(const RowNormArgs& a, hipStream_t st)
{
    if (vec_fits<DTI, DTO, 16>(a)) return launch_fitting<DTI, DTO, 16>(a, st);
    // 2-byte rows of a length that is a multiple of 4 but not 8 (e.g. D = 4100) take 8-byte vectors; the
    // E4M3 copy needs D % 128 == 0 and so always fits 16-byte vectors when its pointers do.
    if constexpr (Vec<DTI>::BYTES == 2) {
        if (!a.yq && vec_fits<DTI, DTO, 8>(a)) return launch_fitting<DTI, DTO, 8>(a, st);
    }
    rownorm_scalar<DTI, DTO><<<dim3(static_cast<unsigned>(a.rows)), 256, 0, st>>>(a);
    return check_launch("rownorm_scalar");
}

}  // namespace slhip

using namespace slhip;

extern "C" SLHIP_API int slhip_rownorm_copies(int kind, int dtype_in, int dtype_out, const void* x, const void* res,
                                              const float* w, const float* b, void* y, void* h_out, int64_t rows,
                                              int64_t D, int64_t x_stride, int64_t res_stride, int64_t y_stride,
                                              int64_t h_stride, float eps, const slhip_norm_copies* copies,
                                              slhip_stream stream)
{
    void* y16 = copies ? copies->y16 : nullptr;
    void* yq = copies ? copies->yq : nullptr;
    if (kind < SLHIP_NORM_RMS || kind > SLHIP_NORM_LAYER) return fail(SLHIP_ERR_INVALID, "rownorm: bad kind %d", kind);
    if (rows < 0 || D < 0) return fail(SLHIP_ERR_INVALID, "rownorm: negative shape");
    if (rows == 0 || D == 0) return SLHIP_OK;
    if (!x) return fail(SLHIP_ERR_INVALID, "rownorm: x is required");
    if (!y && !y16 && !yq) return fail(SLHIP_ERR_INVALID, "rownorm: y or a copy of it is required");
    if (kind == SLHIP_NORM_L2 && w) return fail(SLHIP_ERR_INVALID, "rownorm: L2Norm takes no weight");
    if (kind != SLHIP_NORM_LAYER && b) return fail(SLHIP_ERR_INVALID, "rownorm: only LayerNorm takes a bias");
    if (x_stride < D || (y && y_stride < D) || (res && res_stride < D) || (res && h_out && h_stride < D) ||
        (y16 && copies->y16_stride < D))
        return fail(SLHIP_ERR_INVALID, "rownorm: a row stride is smaller than D");
    if (yq && D % 128 != 0)
        return fail(SLHIP_ERR_INVALID, "rownorm: E4M3 rows need a row length that is a multiple of 128 (D = %lld)",
                    static_cast<long long>(D));
    if (yq && copies->yq_stride < D + D / 32)
        return fail(SLHIP_ERR_INVALID, "rownorm: E4M3 row stride %lld is below D + D/32 = %lld bytes",
                    static_cast<long long>(copies->yq_stride), static_cast<long long>(D + D / 32));
    if (yq && (reinterpret_cast<uintptr_t>(yq) % 4 != 0 || copies->yq_stride % 4 != 0))
        return fail(SLHIP_ERR_INVALID, "rownorm: E4M3 rows must be 4-byte aligned (their f32 scales)");
    if (rows > 0x7FFFFFFF) return fail(SLHIP_ERR_UNSUPPORTED, "rownorm: more than 2^31-1 rows");
    RowNormArgs a{x, res, w, b, y, res ? h_out : nullptr, rows, D, x_stride, res_stride, y_stride, h_stride, eps, kind,
                  y16, y16 ? copies->y16_stride : 0, yq, yq ? copies->yq_stride : 0};
    hipStream_t st = to_stream(stream);
    if (dtype_in == SLHIP_F32 && dtype_out == SLHIP_F32) return dispatch<SLHIP_F32, SLHIP_F32>(a, st);
    if (dtype_in == SLHIP_BF16 && dtype_out == SLHIP_BF16) return dispatch<SLHIP_BF16, SLHIP_BF16>(a, st);
    if (dtype_in == SLHIP_BF16 && dtype_out == SLHIP_F32) return dispatch<SLHIP_BF16, SLHIP_F32>(a, st);
    if (dtype_in == SLHIP_F32 && dtype_out == SLHIP_BF16) return dispatch<SLHIP_F32, SLHIP_BF16>(a, st);
    return fail(SLHIP_ERR_UNSUPPORTED, "rownorm: dtype pair (%d -> %d) not supported", dtype_in, dtype_out);
}

extern "C" SLHIP_API int slhip_rownorm(int kind, int dtype_in, int dtype_out, const void* x, const void* res,
                                       const float* w, const float* b, void* y, void* h_out, int64_t rows, int64_t D,
                                       int64_t x_stride, int64_t res_stride, int64_t y_stride, int64_t h_stride,
                                       float eps, slhip_stream stream)
{
    if (!y && rows > 0 && D > 0) return fail(SLHIP_ERR_INVALID, "rownorm: x and y are required");
    return slhip_rownorm_copies(kind, dtype_in, dtype_out, x, res, w, b, y, h_out, rows, D, x_stride, res_stride,
                                y_stride, h_stride, eps, nullptr, stream);
}
