// Embedding gather with on-the-fly dequantization: y[i, :] = dequant(table[ids[i], :]).
//
// Semantics follow the reference CPU provider (GatherOp, src/Sharplight.Cpu/GatherOp.cs:22-75; decoders
// Quant.Dequantize, src/Sharplight.Cpu/Quant.cs:242-405, and Simd.StoreI8x16/StoreU8x16,
// src/Sharplight.Cpu/Simd.cs:699-753): value = fma(q, d, offset) with the block's f16 scale d and
//   Q8_0: q int8, offset 0       Q4_0: q nibble, offset -8d    Q5_0: q 5-bit, offset -16d
//   Q4_1: q nibble, offset m     Q5_1: q 5-bit, offset m       F16/BF16/F32: exact conversion
// and the 256-value K-quants and the IQ4 codebook formats as decode_k (quant.hpp) restates them
// (Quant.cs:407-446,500-624, Quant.KQuants.cs:36-107).
// Every product is exact in f32, so the f32 result is bit-exact; a bf16 output is that value rounded
// to nearest even (Simd.FloatToBFloat, Simd.cs:530-540). fma(q, d, 0) also fixes the sign of a zero
// (+0 for q = 0), as the reference's FMA does.
//
// Layout: a flat grid of work items, one wavefront each: an item is a chunk of one output row -- CB
// quantized blocks or STEPS output vectors per lane of a plain table (for the quantized formats about 1 KiB of block image, for the plain ones 4096 values) -- and each
// wave streams its item and exits; the waves of a block never synchronize with each other. Quantized
// chunks (blocks of 34, 18, 20, 22 or 24 bytes: only 2-byte aligned) are loaded with 16-byte loads into
// LDS, then each lane decodes VPL consecutive values per output vector, VPL = 16 bytes / output element
// size (8 for bf16, 4 for f32), so every store instruction writes one contiguous span. An id outside
// [0, V) zeroes its row and raises the device error record, reported by slhip_stream_sync.
#include "common.hpp"
#include "quant.hpp"

#include <stdlib.h>

#include <type_traits>

namespace slhip {

struct GatherArgs {
    const uint8_t* table;
    int64_t V, D, rb;  // rows, values per row, bytes per row
    const int32_t* ids;
    int64_t N;
    void* y;
    int64_t ys;  // output row stride in elements
    uint32_t* err;
    int64_t chunks;  // chunks per row
};

__device__ __forceinline__ void raise_index_error(uint32_t* err, int64_t id, int64_t V)
{
    raise_error(err, kErrGatherIndex, static_cast<uint32_t>(static_cast<uint64_t>(id)),
                static_cast<uint32_t>(static_cast<uint64_t>(id) >> 32), static_cast<uint32_t>(V), 0, 0, 0);
}

// One output vector: VPL values as dtype DTO (16 bytes).
template <int DTO, int VPL>
__device__ __forceinline__ void store_vec(void* y, int64_t elem, const float* f)
{
    store_packed<DTO, VPL>(static_cast<char*>(y) + elem * Vec<DTO>::BYTES, f);
}

// One quantized work item of a wave: where its chunk comes from and goes to.
struct QuantItem {
    const uint8_t* src;
    void* yrow;
    int64_t id;
    int nvec16, groups;
    bool live, ok, first_chunk;
};

template <int FMT, int DTO, int CB, int WPB, int RPW>
__global__ __launch_bounds__(64 * WPB) void gather_quant(GatherArgs a)
{
    constexpr int BB = Fmt<FMT>::BB;
    constexpr int BS = Fmt<FMT>::BS;                 // values per block
    constexpr int VPL = 16 / Vec<DTO>::BYTES;       // values per lane per output vector
    constexpr int LOADS = (CB * BB / 16 + 63) / 64;  // 16-byte loads per lane per chunk
    constexpr int STEPS = (CB * BS / VPL + 63) / 64;  // output vectors per lane per chunk
    constexpr int WORDS = CB * BB / 4 + 4;            // +pad for the 3-word reads at the end
    __shared__ __align__(16) uint32_t lds[WPB][WORDS];
    const int lane = threadIdx.x & 63;
    const int wave = wave_id();
    const int64_t total = a.N * a.chunks;
    const int64_t first = (static_cast<int64_t>(blockIdx.x) * WPB + wave) * RPW;
    if (first >= total) return;
    uint32_t* s = lds[wave];
    const int64_t nblocks = a.D / BS;

    // The wave's RPW consecutive items; every id is fetched up front (wave-uniform scalar loads), so the
    // dependent id latency is paid once per wave rather than once per item.
    QuantItem it[RPW];
#pragma unroll
    for (int j = 0; j < RPW; j++) {
        const int64_t item = first + j < total ? first + j : first;
        const int64_t row = a.chunks == 1 ? item : item / a.chunks;
        const int64_t chunk = item - row * a.chunks;
        const int64_t b0 = chunk * CB;
        const int nb = static_cast<int>(nblocks - b0 < CB ? nblocks - b0 : CB);
        const int64_t id = a.ids[row];
        it[j].live = first + j < total;
        it[j].ok = static_cast<uint64_t>(id) < static_cast<uint64_t>(a.V);
        it[j].first_chunk = chunk == 0;
        it[j].id = id;
        it[j].nvec16 = nb * BB / 16;  // chunk starts and lengths are multiples of 16 bytes
        it[j].groups = nb * BS / VPL;
        it[j].src = a.table + (it[j].ok ? id : 0) * a.rb + b0 * BB;  // a bad id reads row 0, stores zeros
        it[j].yrow = static_cast<char*>(a.y) + (row * a.ys + b0 * BS) * Vec<DTO>::BYTES;
    }

    // Two-stage pipeline: item j + 1's loads are issued before item j is decoded and stored. Loads and
    // LDS writes are branch-free (lanes past a chunk's end re-read and re-write its last 16 bytes): under
    // a divergent branch the compiler could not prove the loads complete on every path and would wait
    // for all outstanding memory operations -- the previous stores included -- before each later store.
    uint4 cur[LOADS], nxt[LOADS];
    int ic[LOADS];
#pragma unroll
    for (int k = 0; k < LOADS; k++) {
        const int i = lane + 64 * k < it[0].nvec16 ? lane + 64 * k : it[0].nvec16 - 1;
        cur[k] = load_nt(it[0].src + 16 * i);
    }
#pragma unroll
    for (int j = 0; j < RPW; j++) {
        if (j + 1 < RPW) {
#pragma unroll
            for (int k = 0; k < LOADS; k++) {
                const int i = lane + 64 * k < it[j + 1].nvec16 ? lane + 64 * k : it[j + 1].nvec16 - 1;
                nxt[k] = load_nt(it[j + 1].src + 16 * i);
            }
        }
        // A bad id's chunk (row 0 was read in its place) becomes all-zero bytes: scale 0 and code 0,
        // which every format decodes to +0.
        // (A mask, not a select of vectors: the compiler lowers the latter to a stack array.)
        const uint32_t keep = it[j].ok ? 0xFFFFFFFFu : 0u;
#pragma unroll
        for (int k = 0; k < LOADS; k++) {
            ic[k] = lane + 64 * k < it[j].nvec16 ? lane + 64 * k : it[j].nvec16 - 1;
            reinterpret_cast<uint4*>(s)[ic[k]] =
                make_uint4(cur[k].x & keep, cur[k].y & keep, cur[k].z & keep, cur[k].w & keep);
        }
        wave_lds_sync();
        // Every lane stores every step, so each item issues exactly STEPS stores on every path and the
        // compiler can wait for the next item's loads without waiting for these stores. Lanes past a
        // partial chunk's end (and a tail wave's dead item, which re-reads item 0) re-store identical
        // bytes at the last vector.
#pragma unroll
        for (int k = 0; k < STEPS; k++) {
            const int g = lane + 64 * k < it[j].groups ? lane + 64 * k : it[j].groups - 1;
            float f[VPL];
            decode<FMT, VPL>(s, g * VPL, f);
            store_vec<DTO, VPL>(it[j].live ? it[j].yrow : it[0].yrow, g * VPL, f);
        }
        wave_lds_sync();
        if (j + 1 < RPW) {
#pragma unroll
            for (int k = 0; k < LOADS; k++) cur[k] = nxt[k];
        }
    }
    if (lane == 0) {
#pragma unroll
        for (int j = 0; j < RPW; j++)
            if (it[j].live && !it[j].ok && it[j].first_chunk) raise_index_error(a.err, it[j].id, a.V);
    }
}

// f16 / bf16 / f32 tables: each lane converts VPL values per step straight from global memory.
template <int FMT, int DTO, int STEPS, int WPB>
__global__ __launch_bounds__(64 * WPB) void gather_plain(GatherArgs a)
{
    constexpr int IN_BYTES = FMT == SLHIP_FMT_F32 ? 4 : 2;
    constexpr int VPL = 16 / (IN_BYTES > Vec<DTO>::BYTES ? IN_BYTES : Vec<DTO>::BYTES);
    constexpr int LB = VPL * IN_BYTES;  // bytes loaded per lane per step: 8 or 16
    constexpr int CHUNK = 64 * STEPS * VPL;
    const int lane = threadIdx.x & 63;
    const int64_t item = static_cast<int64_t>(blockIdx.x) * WPB + (threadIdx.x >> 6);
    if (item >= a.N * a.chunks) return;
    const int64_t row = item / a.chunks;
    const int64_t chunk = item - row * a.chunks;
    const int64_t c0 = chunk * CHUNK;
    const int n = static_cast<int>(a.D - c0 < CHUNK ? a.D - c0 : CHUNK);
    const int groups = n / VPL;
    void* const yrow = static_cast<char*>(a.y) + (row * a.ys + c0) * Vec<DTO>::BYTES;
    const int64_t id = a.ids[row];
    if (static_cast<uint64_t>(id) >= static_cast<uint64_t>(a.V)) {
        if (lane == 0 && chunk == 0) raise_index_error(a.err, id, a.V);
        const float z[VPL] = {};
        for (int g = lane; g < groups; g += 64) store_vec<DTO, VPL>(yrow, g * VPL, z);
        return;
    }
    // Every load is issued before the first store, without branches (lanes past the chunk's end re-read
    // its last vector): with a load under a divergent branch the compiler waits for all outstanding
    // memory operations at each step, which serializes the loads behind the previous stores.
    const uint8_t* src = a.table + id * a.rb + c0 * IN_BYTES;
    uint32_t w[STEPS][LB / 4];
#pragma unroll
    for (int k = 0; k < STEPS; k++) {
        const int g = lane + 64 * k < groups ? lane + 64 * k : groups - 1;
        if constexpr (LB == 16) {
            const uint4 v = load_nt(src + 16 * g);
            w[k][0] = v.x;
            w[k][1] = v.y;
            w[k][2] = v.z;
            w[k][3] = v.w;
        } else {
            const u32x2 v = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(src + 8 * g));
            w[k][0] = v.x;
            w[k][1] = v.y;
        }
    }
    const bool full = groups == 64 * STEPS;  // wave-uniform
#pragma unroll
    for (int k = 0; k < STEPS; k++) {
        const int g = lane + 64 * k;
        float f[VPL];
#pragma unroll
        for (int e = 0; e < VPL; e++) {
            if (FMT == SLHIP_FMT_F32) f[e] = __uint_as_float(w[k][e]);
            else if (FMT == SLHIP_FMT_F16) f[e] = (e & 1) ? f16_hi(w[k][e >> 1]) : f16_lo(w[k][e >> 1]);
            else f[e] = (e & 1) ? bf16_hi(w[k][e >> 1]) : bf16_lo(w[k][e >> 1]);
        }
        if (full || g < groups) store_vec<DTO, VPL>(yrow, g * VPL, f);
    }
}

// General path: any alignment and D; one thread per value, byte loads.
template <int DTO>
__global__ __launch_bounds__(256) void gather_scalar(GatherArgs a, int fmt)
{
    const int64_t total = a.N * a.D;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < total;
         i += static_cast<int64_t>(gridDim.x) * 256) {
        const int64_t row = i / a.D, j = i - row * a.D;
        const int64_t id = a.ids[row];
        float v = 0.f;
        if (static_cast<uint64_t>(id) >= static_cast<uint64_t>(a.V)) {
            if (j == 0) raise_index_error(a.err, id, a.V);
        } else {
            const uint8_t* p = a.table + id * a.rb;
            auto h16 = [](const uint8_t* q) {
                return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(q[0] | (q[1] << 8))));
            };
            const int64_t blk = j / 32;
            const int k = static_cast<int>(j % 32);
            auto kv = [&](auto fmt_tag) {  // one value of a K-quant or codebook block
                constexpr int F = decltype(fmt_tag)::value;
                if constexpr (F == SLHIP_FMT_F8E4M3) return e4m3_value(p[j]);  // one byte per value: no 4-byte group
                if constexpr (F == SLHIP_FMT_F8E5M2) return e5m2_value(p[j]);
                const int64_t kb = j / Fmt<F>::BS;
                const int kk = static_cast<int>(j % Fmt<F>::BS);
                float f4[4];
                decode_k<F, 4>(GlobalBytes{p + kb * Fmt<F>::BB}, 0, kk & ~3, f4);
                return f4[kk & 3];
            };
            switch (fmt) {
            case SLHIP_FMT_Q2_K: v = kv(std::integral_constant<int, SLHIP_FMT_Q2_K>{}); break;
            case SLHIP_FMT_Q3_K: v = kv(std::integral_constant<int, SLHIP_FMT_Q3_K>{}); break;
            case SLHIP_FMT_Q4_K: v = kv(std::integral_constant<int, SLHIP_FMT_Q4_K>{}); break;
            case SLHIP_FMT_Q5_K: v = kv(std::integral_constant<int, SLHIP_FMT_Q5_K>{}); break;
            case SLHIP_FMT_Q6_K: v = kv(std::integral_constant<int, SLHIP_FMT_Q6_K>{}); break;
            case SLHIP_FMT_IQ4_NL: v = kv(std::integral_constant<int, SLHIP_FMT_IQ4_NL>{}); break;
            case SLHIP_FMT_IQ4_XS: v = kv(std::integral_constant<int, SLHIP_FMT_IQ4_XS>{}); break;
            case SLHIP_FMT_TQ1_0: v = kv(std::integral_constant<int, SLHIP_FMT_TQ1_0>{}); break;
            case SLHIP_FMT_TQ2_0: v = kv(std::integral_constant<int, SLHIP_FMT_TQ2_0>{}); break;
            case SLHIP_FMT_MXFP4: v = kv(std::integral_constant<int, SLHIP_FMT_MXFP4>{}); break;
            case SLHIP_FMT_NVFP4: v = kv(std::integral_constant<int, SLHIP_FMT_NVFP4>{}); break;
            case SLHIP_FMT_IQ2_XXS: v = kv(std::integral_constant<int, SLHIP_FMT_IQ2_XXS>{}); break;
            case SLHIP_FMT_IQ2_XS: v = kv(std::integral_constant<int, SLHIP_FMT_IQ2_XS>{}); break;
            case SLHIP_FMT_IQ2_S: v = kv(std::integral_constant<int, SLHIP_FMT_IQ2_S>{}); break;
            case SLHIP_FMT_IQ3_XXS: v = kv(std::integral_constant<int, SLHIP_FMT_IQ3_XXS>{}); break;
            case SLHIP_FMT_IQ3_S: v = kv(std::integral_constant<int, SLHIP_FMT_IQ3_S>{}); break;
            case SLHIP_FMT_IQ1_S: v = kv(std::integral_constant<int, SLHIP_FMT_IQ1_S>{}); break;
            case SLHIP_FMT_IQ1_M: v = kv(std::integral_constant<int, SLHIP_FMT_IQ1_M>{}); break;
            case SLHIP_FMT_Q1_0: v = kv(std::integral_constant<int, SLHIP_FMT_Q1_0>{}); break;
            case SLHIP_FMT_Q2_0: v = kv(std::integral_constant<int, SLHIP_FMT_Q2_0>{}); break;
            case SLHIP_FMT_Q2_0_G128: v = kv(std::integral_constant<int, SLHIP_FMT_Q2_0_G128>{}); break;
            case SLHIP_FMT_TERN1_G128: v = kv(std::integral_constant<int, SLHIP_FMT_TERN1_G128>{}); break;
            case SLHIP_FMT_NVFP4_GS: v = kv(std::integral_constant<int, SLHIP_FMT_NVFP4_GS>{}); break;
            case SLHIP_FMT_Q4Z_G32: v = kv(std::integral_constant<int, SLHIP_FMT_Q4Z_G32>{}); break;
            case SLHIP_FMT_Q4Z_G128: v = kv(std::integral_constant<int, SLHIP_FMT_Q4Z_G128>{}); break;
            case SLHIP_FMT_Q8Z_G32: v = kv(std::integral_constant<int, SLHIP_FMT_Q8Z_G32>{}); break;
            case SLHIP_FMT_Q8Z_G128: v = kv(std::integral_constant<int, SLHIP_FMT_Q8Z_G128>{}); break;
            case SLHIP_FMT_NF4_B64: v = kv(std::integral_constant<int, SLHIP_FMT_NF4_B64>{}); break;
            case SLHIP_FMT_FP4_B64: v = kv(std::integral_constant<int, SLHIP_FMT_FP4_B64>{}); break;
            case SLHIP_FMT_Q8A_G32: v = kv(std::integral_constant<int, SLHIP_FMT_Q8A_G32>{}); break;
            case SLHIP_FMT_Q2S_G128: v = kv(std::integral_constant<int, SLHIP_FMT_Q2S_G128>{}); break;
            case SLHIP_FMT_F8E4M3: v = kv(std::integral_constant<int, SLHIP_FMT_F8E4M3>{}); break;
            case SLHIP_FMT_F8E5M2: v = kv(std::integral_constant<int, SLHIP_FMT_F8E5M2>{}); break;
            case SLHIP_FMT_F8E4M3_B32: v = kv(std::integral_constant<int, SLHIP_FMT_F8E4M3_B32>{}); break;
            case SLHIP_FMT_F8E4M3_B128: v = kv(std::integral_constant<int, SLHIP_FMT_F8E4M3_B128>{}); break;
            case SLHIP_FMT_TRELLIS_V4K8_G128: v = kv(std::integral_constant<int, SLHIP_FMT_TRELLIS_V4K8_G128>{}); break;
            case SLHIP_FMT_TRELLIS_V4K6_G128: v = kv(std::integral_constant<int, SLHIP_FMT_TRELLIS_V4K6_G128>{}); break;
            case SLHIP_FMT_TRELLIS_V4K7_G128: v = kv(std::integral_constant<int, SLHIP_FMT_TRELLIS_V4K7_G128>{}); break;
            case SLHIP_FMT_TRELLIS_V2K5_G128: v = kv(std::integral_constant<int, SLHIP_FMT_TRELLIS_V2K5_G128>{}); break;
            case SLHIP_FMT_TRELLIS_V2K6_G128: v = kv(std::integral_constant<int, SLHIP_FMT_TRELLIS_V2K6_G128>{}); break;
            case SLHIP_FMT_TRELLIS_V2K7_G128: v = kv(std::integral_constant<int, SLHIP_FMT_TRELLIS_V2K7_G128>{}); break;
            case SLHIP_FMT_F32: {
                uint32_t u = p[4 * j] | (p[4 * j + 1] << 8) | (p[4 * j + 2] << 16) | (static_cast<uint32_t>(p[4 * j + 3]) << 24);
                v = __uint_as_float(u);
                break;
            }
            case SLHIP_FMT_F16: v = h16(p + 2 * j); break;
            case SLHIP_FMT_BF16: v = __uint_as_float(static_cast<uint32_t>(p[2 * j] | (p[2 * j + 1] << 8)) << 16); break;
            case SLHIP_FMT_Q8_0: {
                const uint8_t* b = p + blk * 34;
                v = __fmaf_rn(static_cast<float>(static_cast<int8_t>(b[2 + k])), h16(b), 0.0f);
                break;
            }
            default: {
                const int bb = fmt == SLHIP_FMT_Q4_0 ? 18 : fmt == SLHIP_FMT_Q4_1 ? 20 : fmt == SLHIP_FMT_Q5_0 ? 22 : 24;
                const int qs = fmt == SLHIP_FMT_Q4_0 ? 2 : fmt == SLHIP_FMT_Q4_1 ? 4 : fmt == SLHIP_FMT_Q5_0 ? 6 : 8;
                const uint8_t* b = p + blk * bb;
                const float d = h16(b);
                const uint32_t byte = b[qs + (k & 15)];
                uint32_t q = k < 16 ? (byte & 15u) : (byte >> 4);
                if (fmt == SLHIP_FMT_Q5_0 || fmt == SLHIP_FMT_Q5_1) {
                    const uint8_t* hq = b + (fmt == SLHIP_FMT_Q5_0 ? 2 : 4);
                    uint32_t qh = hq[0] | (hq[1] << 8) | (hq[2] << 16) | (static_cast<uint32_t>(hq[3]) << 24);
                    q |= ((qh >> k) & 1u) << 4;
                }
                float add = (fmt == SLHIP_FMT_Q4_1 || fmt == SLHIP_FMT_Q5_1) ? h16(b + 2)
                          : (fmt == SLHIP_FMT_Q4_0 ? -8.0f * d : -16.0f * d);
                v = __fmaf_rn(static_cast<float>(q), d, add);
                break;
            }
            }
        }
        Vec<DTO>::store1(a.y, row * a.ys + j, v);
    }
}

static int block_bytes(int fmt)
{
    switch (fmt) {
    case SLHIP_FMT_F32: return 4;
    case SLHIP_FMT_F16: case SLHIP_FMT_BF16: return 2;
    case SLHIP_FMT_Q8_0: return 34;
    case SLHIP_FMT_Q4_0: return 18;
    case SLHIP_FMT_Q4_1: return 20;
    case SLHIP_FMT_Q5_0: return 22;
    case SLHIP_FMT_Q5_1: return 24;
    case SLHIP_FMT_Q2_K: return 84;
    case SLHIP_FMT_Q3_K: return 110;
    case SLHIP_FMT_Q4_K: return 144;
    case SLHIP_FMT_Q5_K: return 176;
    case SLHIP_FMT_Q6_K: return 210;
    case SLHIP_FMT_IQ4_NL: return 18;
    case SLHIP_FMT_IQ4_XS: return 136;
    case SLHIP_FMT_TQ1_0: return 54;
    case SLHIP_FMT_TQ2_0: return 66;
    case SLHIP_FMT_MXFP4: return 17;
    case SLHIP_FMT_NVFP4: return 36;
    case SLHIP_FMT_IQ2_XXS: return 66;
    case SLHIP_FMT_IQ2_XS: return 74;
    case SLHIP_FMT_IQ2_S: return 82;
    case SLHIP_FMT_IQ3_XXS: return 98;
    case SLHIP_FMT_IQ3_S: return 110;
    case SLHIP_FMT_IQ1_S: return 50;
    case SLHIP_FMT_IQ1_M: return 56;
    case SLHIP_FMT_Q1_0: return 18;
    case SLHIP_FMT_Q2_0: return 18;
    case SLHIP_FMT_Q2_0_G128: return 34;
    case SLHIP_FMT_TERN1_G128: return 28;
    case SLHIP_FMT_NVFP4_GS: return 40;
    case SLHIP_FMT_Q4Z_G32: return 20;
    case SLHIP_FMT_Q4Z_G128: return 68;
    case SLHIP_FMT_Q8Z_G32: return 36;
    case SLHIP_FMT_Q8Z_G128: return 132;
    case SLHIP_FMT_NF4_B64: return 36;
    case SLHIP_FMT_FP4_B64: return 36;
    case SLHIP_FMT_Q8A_G32: return 36;
    case SLHIP_FMT_Q2S_G128: return 36;
    case SLHIP_FMT_F8E4M3: return 1;
    case SLHIP_FMT_F8E5M2: return 1;
    case SLHIP_FMT_F8E4M3_B32: return 36;
    case SLHIP_FMT_F8E4M3_B128: return 132;
    case SLHIP_FMT_TRELLIS_V4K8_G128: return 34;
    case SLHIP_FMT_TRELLIS_V4K6_G128: return 26;
    case SLHIP_FMT_TRELLIS_V4K7_G128: return 30;
    case SLHIP_FMT_TRELLIS_V2K5_G128: return 42;
    case SLHIP_FMT_TRELLIS_V2K6_G128: return 50;
    case SLHIP_FMT_TRELLIS_V2K7_G128: return 58;
    default: return -1;
    }
}

static int block_values(int fmt)
{
    switch (fmt) {
    case SLHIP_FMT_F32: case SLHIP_FMT_F16: case SLHIP_FMT_BF16: return 1;
    case SLHIP_FMT_Q8_0: case SLHIP_FMT_Q4_0: case SLHIP_FMT_Q4_1: case SLHIP_FMT_Q5_0: case SLHIP_FMT_Q5_1:
    case SLHIP_FMT_IQ4_NL: case SLHIP_FMT_MXFP4: return 32;
    case SLHIP_FMT_NVFP4: return 64;
    case SLHIP_FMT_Q1_0: case SLHIP_FMT_Q2_0_G128: case SLHIP_FMT_TERN1_G128: case SLHIP_FMT_Q4Z_G128: case SLHIP_FMT_Q8Z_G128: case SLHIP_FMT_Q2S_G128: case SLHIP_FMT_F8E4M3_B128:
    case SLHIP_FMT_TRELLIS_V4K8_G128: case SLHIP_FMT_TRELLIS_V4K6_G128: case SLHIP_FMT_TRELLIS_V4K7_G128:
    case SLHIP_FMT_TRELLIS_V2K5_G128: case SLHIP_FMT_TRELLIS_V2K6_G128: case SLHIP_FMT_TRELLIS_V2K7_G128: return 128;
    case SLHIP_FMT_Q2_0: case SLHIP_FMT_NVFP4_GS: case SLHIP_FMT_NF4_B64: case SLHIP_FMT_FP4_B64: return 64;
    case SLHIP_FMT_Q4Z_G32: case SLHIP_FMT_Q8Z_G32: case SLHIP_FMT_Q8A_G32: case SLHIP_FMT_F8E4M3_B32: return 32;
    case SLHIP_FMT_F8E4M3: case SLHIP_FMT_F8E5M2: return 1;
    default: return 256;
    }
}

static int env_int(const char* name, int dflt)
{
    const char* s = getenv(name);
    return s && *s ? atoi(s) : dflt;
}

// Work-item size (SLHIP_GATHER_ITEM = 0: small, 1: large) and waves per block (SLHIP_GATHER_WPB = 1 or 4).
// Default: large items (item_values() for the quantized formats, 8 vectors per lane of a plain table) in
// 4-wave blocks; two items per wave (SLHIP_GATHER_RPW = 2, the second item's loads issued before the first
// is decoded) measured 3-4% slower.
struct GatherShape {
    bool large;
    int wpb;
    int rpw;  // quantized work items per wave (SLHIP_GATHER_RPW = 1 or 2)
};

static GatherShape gather_shape()
{
    return GatherShape{env_int("SLHIP_GATHER_ITEM", 1) != 0, env_int("SLHIP_GATHER_WPB", 4) == 1 ? 1 : 4,
                       env_int("SLHIP_GATHER_RPW", 1) == 2 ? 2 : 1};
}

template <int FMT, int DTO, int CB, int WPB, int RPW>
static int launch_quant_shape(GatherArgs a, hipStream_t st)
{
    a.chunks = (a.D / Fmt<FMT>::BS + CB - 1) / CB;
    const int64_t waves = (a.N * a.chunks + RPW - 1) / RPW;
    const int64_t blocks = (waves + WPB - 1) / WPB;
    if (blocks > 0x7FFFFFFF) return fail(SLHIP_ERR_UNSUPPORTED, "gather: grid too large");
    gather_quant<FMT, DTO, CB, WPB, RPW><<<static_cast<unsigned>(blocks), 64 * WPB, 0, st>>>(a);
    return check_launch("gather_quant");
}

// Values per work item for a format: the smallest of 1024, 2048 and 4096 values whose block image is at least
// 1 KiB and a whole number of 16-byte vectors (4096 otherwise). Measured on MI355X at 16384 x 4096 from a
// 151936-row table: ~1 KiB of random row bytes per wave beats 2 and 4 KiB by 1-3% (Q8_0 at 1024 values:
// 36.4 against 37.4 us at 4096; Q4_0 at 2048: 31.3-31.6 against 31.8), while smaller items lose (~0.5 KiB:
// Q4_0 at 1024 values 31.9 us, and 512-value items ~35% slower: each wave pays a dependent id load).
template <int FMT>
constexpr int item_values()
{
    constexpr int BS = Fmt<FMT>::BS, BB = Fmt<FMT>::BB;
    for (int v = 1024; v < 4096; v *= 2)
        if (v % BS == 0 && (v / BS * BB) % 16 == 0 && v / BS * BB >= 1024) return v;
    return 4096;
}

template <int FMT, int DTO>
static int launch_quant(const GatherArgs& a, hipStream_t st)
{
    constexpr int CB = item_values<FMT>() / Fmt<FMT>::BS, CBS = 512 / Fmt<FMT>::BS;
    const GatherShape g = gather_shape();
    if constexpr ((CBS * Fmt<FMT>::BB) % 16 == 0) {
        if (!g.large)
            return g.wpb == 1 ? launch_quant_shape<FMT, DTO, CBS, 1, 1>(a, st) : launch_quant_shape<FMT, DTO, CBS, 4, 1>(a, st);
    }
    if (g.rpw == 2) return launch_quant_shape<FMT, DTO, CB, 4, 2>(a, st);
    return g.wpb == 1 ? launch_quant_shape<FMT, DTO, CB, 1, 1>(a, st) : launch_quant_shape<FMT, DTO, CB, 4, 1>(a, st);
}

template <int FMT, int DTO, int STEPS, int WPB>
static int launch_plain_shape(GatherArgs a, hipStream_t st)
{
    constexpr int IN_BYTES = FMT == SLHIP_FMT_F32 ? 4 : 2;
    constexpr int VPL = 16 / (IN_BYTES > Vec<DTO>::BYTES ? IN_BYTES : Vec<DTO>::BYTES);
    constexpr int CHUNK = 64 * STEPS * VPL;
    a.chunks = (a.D + CHUNK - 1) / CHUNK;
    const int64_t blocks = (a.N * a.chunks + WPB - 1) / WPB;
    if (blocks > 0x7FFFFFFF) return fail(SLHIP_ERR_UNSUPPORTED, "gather: grid too large");
    gather_plain<FMT, DTO, STEPS, WPB><<<static_cast<unsigned>(blocks), 64 * WPB, 0, st>>>(a);
    return check_launch("gather_plain");
}

template <int FMT, int DTO>
static int launch_plain(const GatherArgs& a, hipStream_t st)
{
    const GatherShape g = gather_shape();
    if (g.large) return g.wpb == 1 ? launch_plain_shape<FMT, DTO, 8, 1>(a, st) : launch_plain_shape<FMT, DTO, 8, 4>(a, st);
    return g.wpb == 1 ? launch_plain_shape<FMT, DTO, 1, 1>(a, st) : launch_plain_shape<FMT, DTO, 1, 4>(a, st);
}

template <int DTO>
static int dispatch(int fmt, GatherArgs a, hipStream_t st)
{
    // Vector paths: 16-byte row starts (rows are multiples of 16 bytes and the table is 16-byte aligned),
    // whole output vectors (D a multiple of 8 values) at 16-byte aligned output rows.
    const bool vec_ok = a.rb % 16 == 0 && aligned16(a.table) && a.D % 8 == 0 && aligned16(a.y) &&
                        (a.ys * Vec<DTO>::BYTES) % 16 == 0;
    if (vec_ok) {
        switch (fmt) {
        case SLHIP_FMT_Q8_0: return launch_quant<SLHIP_FMT_Q8_0, DTO>(a, st);
        case SLHIP_FMT_Q4_0: return launch_quant<SLHIP_FMT_Q4_0, DTO>(a, st);
        case SLHIP_FMT_Q4_1: return launch_quant<SLHIP_FMT_Q4_1, DTO>(a, st);
        case SLHIP_FMT_Q5_0: return launch_quant<SLHIP_FMT_Q5_0, DTO>(a, st);
        case SLHIP_FMT_Q5_1: return launch_quant<SLHIP_FMT_Q5_1, DTO>(a, st);
        case SLHIP_FMT_Q2_K: return launch_quant<SLHIP_FMT_Q2_K, DTO>(a, st);
        case SLHIP_FMT_Q3_K: return launch_quant<SLHIP_FMT_Q3_K, DTO>(a, st);
        case SLHIP_FMT_Q4_K: return launch_quant<SLHIP_FMT_Q4_K, DTO>(a, st);
        case SLHIP_FMT_Q5_K: return launch_quant<SLHIP_FMT_Q5_K, DTO>(a, st);
        case SLHIP_FMT_Q6_K: return launch_quant<SLHIP_FMT_Q6_K, DTO>(a, st);
        case SLHIP_FMT_IQ4_NL: return launch_quant<SLHIP_FMT_IQ4_NL, DTO>(a, st);
        case SLHIP_FMT_IQ4_XS: return launch_quant<SLHIP_FMT_IQ4_XS, DTO>(a, st);
        case SLHIP_FMT_TQ1_0: return launch_quant<SLHIP_FMT_TQ1_0, DTO>(a, st);
        case SLHIP_FMT_TQ2_0: return launch_quant<SLHIP_FMT_TQ2_0, DTO>(a, st);
        case SLHIP_FMT_MXFP4: return launch_quant<SLHIP_FMT_MXFP4, DTO>(a, st);
        case SLHIP_FMT_NVFP4: return launch_quant<SLHIP_FMT_NVFP4, DTO>(a, st);
        case SLHIP_FMT_IQ2_XXS: return launch_quant<SLHIP_FMT_IQ2_XXS, DTO>(a, st);
        case SLHIP_FMT_IQ2_XS: return launch_quant<SLHIP_FMT_IQ2_XS, DTO>(a, st);
        case SLHIP_FMT_IQ2_S: return launch_quant<SLHIP_FMT_IQ2_S, DTO>(a, st);
        case SLHIP_FMT_IQ3_XXS: return launch_quant<SLHIP_FMT_IQ3_XXS, DTO>(a, st);
        case SLHIP_FMT_IQ3_S: return launch_quant<SLHIP_FMT_IQ3_S, DTO>(a, st);
        case SLHIP_FMT_IQ1_S: return launch_quant<SLHIP_FMT_IQ1_S, DTO>(a, st);
        case SLHIP_FMT_IQ1_M: return launch_quant<SLHIP_FMT_IQ1_M, DTO>(a, st);
        case SLHIP_FMT_Q1_0: return launch_quant<SLHIP_FMT_Q1_0, DTO>(a, st);
        case SLHIP_FMT_Q2_0: return launch_quant<SLHIP_FMT_Q2_0, DTO>(a, st);
        case SLHIP_FMT_Q2_0_G128: return launch_quant<SLHIP_FMT_Q2_0_G128, DTO>(a, st);
        case SLHIP_FMT_TERN1_G128: return launch_quant<SLHIP_FMT_TERN1_G128, DTO>(a, st);
        case SLHIP_FMT_NVFP4_GS: return launch_quant<SLHIP_FMT_NVFP4_GS, DTO>(a, st);
        case SLHIP_FMT_Q4Z_G32: return launch_quant<SLHIP_FMT_Q4Z_G32, DTO>(a, st);
        case SLHIP_FMT_Q4Z_G128: return launch_quant<SLHIP_FMT_Q4Z_G128, DTO>(a, st);
        case SLHIP_FMT_Q8Z_G32: return launch_quant<SLHIP_FMT_Q8Z_G32, DTO>(a, st);
        case SLHIP_FMT_Q8Z_G128: return launch_quant<SLHIP_FMT_Q8Z_G128, DTO>(a, st);
        case SLHIP_FMT_NF4_B64: return launch_quant<SLHIP_FMT_NF4_B64, DTO>(a, st);
        case SLHIP_FMT_FP4_B64: return launch_quant<SLHIP_FMT_FP4_B64, DTO>(a, st);
        case SLHIP_FMT_Q8A_G32: return launch_quant<SLHIP_FMT_Q8A_G32, DTO>(a, st);
        case SLHIP_FMT_Q2S_G128: return launch_quant<SLHIP_FMT_Q2S_G128, DTO>(a, st);
        case SLHIP_FMT_F8E4M3: return launch_quant<SLHIP_FMT_F8E4M3, DTO>(a, st);
        case SLHIP_FMT_F8E5M2: return launch_quant<SLHIP_FMT_F8E5M2, DTO>(a, st);
        case SLHIP_FMT_F8E4M3_B32: return launch_quant<SLHIP_FMT_F8E4M3_B32, DTO>(a, st);
        case SLHIP_FMT_F8E4M3_B128: return launch_quant<SLHIP_FMT_F8E4M3_B128, DTO>(a, st);
        case SLHIP_FMT_TRELLIS_V4K8_G128: return launch_quant<SLHIP_FMT_TRELLIS_V4K8_G128, DTO>(a, st);
        case SLHIP_FMT_TRELLIS_V4K6_G128: return launch_quant<SLHIP_FMT_TRELLIS_V4K6_G128, DTO>(a, st);
        case SLHIP_FMT_TRELLIS_V4K7_G128: return launch_quant<SLHIP_FMT_TRELLIS_V4K7_G128, DTO>(a, st);
        case SLHIP_FMT_TRELLIS_V2K5_G128: return launch_quant<SLHIP_FMT_TRELLIS_V2K5_G128, DTO>(a, st);
        case SLHIP_FMT_TRELLIS_V2K6_G128: return launch_quant<SLHIP_FMT_TRELLIS_V2K6_G128, DTO>(a, st);
        case SLHIP_FMT_TRELLIS_V2K7_G128: return launch_quant<SLHIP_FMT_TRELLIS_V2K7_G128, DTO>(a, st);
        case SLHIP_FMT_F16: return launch_plain<SLHIP_FMT_F16, DTO>(a, st);
        case SLHIP_FMT_BF16: return launch_plain<SLHIP_FMT_BF16, DTO>(a, st);
        case SLHIP_FMT_F32: return launch_plain<SLHIP_FMT_F32, DTO>(a, st);
        default: break;
        }
    }
    const int64_t blocks = (a.N * a.D + 255) / 256;
    const unsigned g2 = static_cast<unsigned>(blocks < 65536 ? blocks : 65536);
    gather_scalar<DTO><<<g2, 256, 0, st>>>(a, fmt);
    return check_launch("gather_scalar");
}

}  // namespace slhip

using namespace slhip;

extern "C" SLHIP_API int slhip_gather(int format, const void* table, int64_t V, int64_t D, const int32_t* ids,
                                      int64_t N, int dtype_out, void* y, int64_t y_stride, slhip_stream stream)
{
    const int bb = block_bytes(format);
    if (bb < 0) return fail(SLHIP_ERR_UNSUPPORTED, "gather: table format %d not supported", format);
    if (V < 0 || D < 0 || N < 0) return fail(SLHIP_ERR_INVALID, "gather: negative shape");
    const int bs = block_values(format);
    if (D % bs != 0) return fail(SLHIP_ERR_INVALID, "gather: row length %lld is not a multiple of the block size %d", (long long)D, bs);
    if (N == 0 || D == 0) return SLHIP_OK;
    if (!table || !ids || !y) return fail(SLHIP_ERR_INVALID, "gather: null tensor");
    if (N > 1 && y_stride < D) return fail(SLHIP_ERR_INVALID, "gather: output row stride is smaller than D");
    if (dtype_out != SLHIP_F32 && dtype_out != SLHIP_BF16)
        return fail(SLHIP_ERR_UNSUPPORTED, "gather: output dtype %d not supported", dtype_out);
    uint32_t* err = nullptr;
    int stc = error_word(&err);
    if (stc) return stc;
    GatherArgs a{static_cast<const uint8_t*>(table), V, D, D / bs * bb, ids, N, y, N > 1 ? y_stride : D, err, 1};
    hipStream_t st = to_stream(stream);
    return dtype_out == SLHIP_BF16 ? dispatch<SLHIP_BF16>(format, a, st) : dispatch<SLHIP_F32>(format, a, st);
}
