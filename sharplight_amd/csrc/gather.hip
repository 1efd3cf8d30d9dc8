// Embedding gather with on-the-fly dequantization: y[i, :] = dequant(table[ids[i], :]).
//
// Semantics follow the reference CPU provider (GatherOp, src/Sharplight.Cpu/GatherOp.cs:22-75; decoders
// Quant.Dequantize, src/Sharplight.Cpu/Quant.cs:242-405, and Simd.StoreI8x16/StoreU8x16,
// src/Sharplight.Cpu/Simd.cs:699-753): value = fma(q, d, offset) with the block's f16 scale d and
//   Q8_0: q int8, offset 0       Q4_0: q nibble, offset -8d    Q5_0: q 5-bit, offset -16d
//   Q4_1: q nibble, offset m     Q5_1: q 5-bit, offset m       F16/BF16/F32: exact conversion
// Every product is exact in f32, so the f32 result is bit-exact; a bf16 output is that value rounded
// to nearest even (Simd.FloatToBFloat, Simd.cs:530-540). fma(q, d, 0) also fixes the sign of a zero
// (+0 for q = 0), as the reference's FMA does.
//
// Layout: one wavefront per output row (4 per block). Quantized rows are staged through LDS in chunks
// of up to 128 blocks with 16-byte loads (block rows are only 2-byte aligned: 34, 18, 20, 22 or 24
// bytes), then each lane decodes 8 consecutive values -- a quarter block -- from LDS and writes them
// with one 16-byte (bf16) or two 16-byte (f32) stores, so every global access of a wave is a fully
// used 1 KiB span. f16/bf16/f32 tables stream straight from global memory. An id outside [0, V) zeroes
// its row and raises the device's index-error word, reported by slhip_stream_sync.
#include "common.hpp"

namespace slhip {

constexpr int kChunkBlocks = 128;  // 32-value blocks staged per wave and chunk (4096 values)
constexpr int kWaves = 4;

struct GatherArgs {
    const uint8_t* table;
    int64_t V, D, rb;  // rows, values per row, bytes per row
    const int32_t* ids;
    int64_t N;
    void* y;
    int64_t ys;  // output row stride in elements
    uint32_t* err;
};

template <int FMT> struct Fmt;
template <> struct Fmt<SLHIP_FMT_Q8_0> { static constexpr int BB = 34; };
template <> struct Fmt<SLHIP_FMT_Q4_0> { static constexpr int BB = 18; };
template <> struct Fmt<SLHIP_FMT_Q4_1> { static constexpr int BB = 20; };
template <> struct Fmt<SLHIP_FMT_Q5_0> { static constexpr int BB = 22; };
template <> struct Fmt<SLHIP_FMT_Q5_1> { static constexpr int BB = 24; };

__device__ __forceinline__ uint32_t lds_u16(const uint32_t* s, int off)
{
    uint32_t w = s[off >> 2];
    return (off & 2) ? (w >> 16) : (w & 0xFFFFu);
}

// 8 bytes at an even LDS byte offset, as two little-endian words.
__device__ __forceinline__ uint2 lds_u64(const uint32_t* s, int off)
{
    const int i = off >> 2;
    const uint32_t sh = (off & 3) * 8;
    const uint32_t w0 = s[i], w1 = s[i + 1], w2 = s[i + 2];
    return make_uint2(__builtin_amdgcn_alignbit(w1, w0, sh), __builtin_amdgcn_alignbit(w2, w1, sh));
}

__device__ __forceinline__ uint32_t lds_u32(const uint32_t* s, int off)
{
    const int i = off >> 2;
    const uint32_t sh = (off & 3) * 8;
    return __builtin_amdgcn_alignbit(s[i + 1], s[i], sh);
}

__device__ __forceinline__ float half_at(const uint32_t* s, int off)
{
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(lds_u16(s, off))));
}

// Decodes values [8*sub, 8*sub + 8) of the block at LDS byte offset `o`.
template <int FMT> __device__ __forceinline__ void decode8(const uint32_t* s, int o, int sub, float* f);

template <> __device__ __forceinline__ void decode8<SLHIP_FMT_Q8_0>(const uint32_t* s, int o, int sub, float* f)
{
    const float d = half_at(s, o);
    const uint2 q = lds_u64(s, o + 2 + 8 * sub);
#pragma unroll
    for (int e = 0; e < 4; e++) {
        f[e] = __fmaf_rn(static_cast<float>(static_cast<int8_t>(q.x >> (8 * e))), d, 0.0f);
        f[4 + e] = __fmaf_rn(static_cast<float>(static_cast<int8_t>(q.y >> (8 * e))), d, 0.0f);
    }
}

// Nibble blocks: values j < 16 are the low nibbles of qs[j], j >= 16 the high nibbles of qs[j - 16].
template <int QS, int QH, bool HAS_M, int OFF>
__device__ __forceinline__ void decode_nibbles(const uint32_t* s, int o, int sub, float* f)
{
    const float d = half_at(s, o);
    const float add = HAS_M ? half_at(s, o + 2) : static_cast<float>(OFF) * d;
    const uint2 q = lds_u64(s, o + QS + 8 * (sub & 1));
    const int shift = (sub >> 1) * 4;
    uint32_t qh = 0;
    if (QH >= 0) qh = lds_u32(s, o + QH) >> (8 * (sub & 1) + 16 * (sub >> 1));
#pragma unroll
    for (int e = 0; e < 8; e++) {
        uint32_t byte = (e < 4 ? q.x >> (8 * e) : q.y >> (8 * (e - 4))) & 0xFFu;
        uint32_t v = (byte >> shift) & 15u;
        if (QH >= 0) v |= ((qh >> e) & 1u) << 4;
        f[e] = __fmaf_rn(static_cast<float>(v), d, add);
    }
}

template <> __device__ __forceinline__ void decode8<SLHIP_FMT_Q4_0>(const uint32_t* s, int o, int sub, float* f)
{
    decode_nibbles<2, -1, false, -8>(s, o, sub, f);
}
template <> __device__ __forceinline__ void decode8<SLHIP_FMT_Q4_1>(const uint32_t* s, int o, int sub, float* f)
{
    decode_nibbles<4, -1, true, 0>(s, o, sub, f);
}
template <> __device__ __forceinline__ void decode8<SLHIP_FMT_Q5_0>(const uint32_t* s, int o, int sub, float* f)
{
    decode_nibbles<6, 2, false, -16>(s, o, sub, f);
}
template <> __device__ __forceinline__ void decode8<SLHIP_FMT_Q5_1>(const uint32_t* s, int o, int sub, float* f)
{
    decode_nibbles<8, 4, true, 0>(s, o, sub, f);
}

__device__ __forceinline__ void raise_index_error(uint32_t* err, int64_t id, int64_t V)
{
    if (atomicCAS(err, 0u, 1u) == 0u) {
        err[1] = static_cast<uint32_t>(static_cast<uint64_t>(id));
        err[2] = static_cast<uint32_t>(static_cast<uint64_t>(id) >> 32);
        err[3] = static_cast<uint32_t>(V);
    }
}

template <int DTO> __device__ __forceinline__ void store8(void* y, int64_t elem, const float* f)
{
    store_packed<DTO, 8>(static_cast<char*>(y) + elem * Vec<DTO>::BYTES, f);
}

template <int FMT, int DTO>
__global__ __launch_bounds__(256) void gather_quant(GatherArgs a)
{
    constexpr int BB = Fmt<FMT>::BB;
    constexpr int WORDS = (kChunkBlocks * BB) / 4 + 4;  // +pad for the 3-word reads at the end
    __shared__ uint32_t lds[kWaves][WORDS];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    uint32_t* s = lds[wave];
    const int64_t nblocks = a.D / 32;
    for (int64_t r0 = static_cast<int64_t>(blockIdx.x) * kWaves; r0 < a.N; r0 += static_cast<int64_t>(gridDim.x) * kWaves) {
        const int64_t row = r0 + wave;
        const bool live = row < a.N;
        int64_t id = live ? a.ids[row] : 0;
        const bool bad = live && static_cast<uint64_t>(id) >= static_cast<uint64_t>(a.V);
        if (bad && lane == 0) raise_index_error(a.err, id, a.V);
        const uint8_t* src = a.table + (bad ? 0 : id) * a.rb;
        for (int64_t b0 = 0; b0 < nblocks; b0 += kChunkBlocks) {
            const int nb = static_cast<int>(nblocks - b0 < kChunkBlocks ? nblocks - b0 : kChunkBlocks);
            const int nvec16 = nb * BB / 16;  // chunk starts and lengths are multiples of 16 bytes
            if (live && !bad) {
                const uint8_t* g = src + b0 * BB;
                for (int i = lane; i < nvec16; i += 64) reinterpret_cast<uint4*>(s)[i] = load_nt(g + 16 * i);
            }
            __syncthreads();
            if (live) {
                for (int v = lane; v < nb * 4; v += 64) {
                    float f[8];
                    if (bad) {
#pragma unroll
                        for (int e = 0; e < 8; e++) f[e] = 0.f;
                    } else {
                        decode8<FMT>(s, (v >> 2) * BB, v & 3, f);
                    }
                    store8<DTO>(a.y, row * a.ys + (b0 * 32 + v * 8), f);
                }
            }
            __syncthreads();
        }
    }
}

// f16 / bf16 / f32 tables: 8 values per lane per step straight from global memory.
template <int FMT, int DTO>
__global__ __launch_bounds__(256) void gather_plain(GatherArgs a)
{
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int64_t nv8 = a.D / 8;
    for (int64_t row = static_cast<int64_t>(blockIdx.x) * kWaves + wave; row < a.N;
         row += static_cast<int64_t>(gridDim.x) * kWaves) {
        const int64_t id = a.ids[row];
        const bool bad = static_cast<uint64_t>(id) >= static_cast<uint64_t>(a.V);
        if (bad && lane == 0) raise_index_error(a.err, id, a.V);
        const uint8_t* src = a.table + (bad ? 0 : id) * a.rb;
        for (int64_t v = lane; v < nv8; v += 64) {
            float f[8];
            if (bad) {
#pragma unroll
                for (int e = 0; e < 8; e++) f[e] = 0.f;
            } else if (FMT == SLHIP_FMT_F32) {
                uint4 p0 = load_nt(src + 32 * v), p1 = load_nt(src + 32 * v + 16);
                Vec<SLHIP_F32>::unpack(p0, f);
                Vec<SLHIP_F32>::unpack(p1, f + 4);
            } else if (FMT == SLHIP_FMT_F16) {
                Vec<SLHIP_F16>::unpack(load_nt(src + 16 * v), f);
            } else {
                Vec<SLHIP_BF16>::unpack(load_nt(src + 16 * v), f);
            }
            store8<DTO>(a.y, row * a.ys + v * 8, f);
        }
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
            switch (fmt) {
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
    default: return -1;
    }
}

template <int DTO>
static int dispatch(int fmt, const GatherArgs& a, hipStream_t st)
{
    const int64_t rows_blocks = (a.N + kWaves - 1) / kWaves;
    const unsigned grid = static_cast<unsigned>(rows_blocks < 0x7FFFFFFF ? rows_blocks : 0x7FFFFFFF);
    const bool vec_ok = a.rb % 16 == 0 && aligned16(a.table) && a.D % 8 == 0 && aligned16(a.y) &&
                        (a.ys * Vec<DTO>::BYTES) % 16 == 0;
    if (vec_ok) {
        switch (fmt) {
        case SLHIP_FMT_Q8_0: gather_quant<SLHIP_FMT_Q8_0, DTO><<<grid, 256, 0, st>>>(a); return check_launch("gather_quant");
        case SLHIP_FMT_Q4_0: gather_quant<SLHIP_FMT_Q4_0, DTO><<<grid, 256, 0, st>>>(a); return check_launch("gather_quant");
        case SLHIP_FMT_Q4_1: gather_quant<SLHIP_FMT_Q4_1, DTO><<<grid, 256, 0, st>>>(a); return check_launch("gather_quant");
        case SLHIP_FMT_Q5_0: gather_quant<SLHIP_FMT_Q5_0, DTO><<<grid, 256, 0, st>>>(a); return check_launch("gather_quant");
        case SLHIP_FMT_Q5_1: gather_quant<SLHIP_FMT_Q5_1, DTO><<<grid, 256, 0, st>>>(a); return check_launch("gather_quant");
        case SLHIP_FMT_F16: gather_plain<SLHIP_FMT_F16, DTO><<<grid, 256, 0, st>>>(a); return check_launch("gather_plain");
        case SLHIP_FMT_BF16: gather_plain<SLHIP_FMT_BF16, DTO><<<grid, 256, 0, st>>>(a); return check_launch("gather_plain");
        case SLHIP_FMT_F32: gather_plain<SLHIP_FMT_F32, DTO><<<grid, 256, 0, st>>>(a); return check_launch("gather_plain");
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
    const int bs = format >= SLHIP_FMT_Q8_0 ? 32 : 1;
    if (D % bs != 0) return fail(SLHIP_ERR_INVALID, "gather: row length %lld is not a multiple of the block size %d", (long long)D, bs);
    if (N == 0 || D == 0) return SLHIP_OK;
    if (!table || !ids || !y) return fail(SLHIP_ERR_INVALID, "gather: null tensor");
    if (N > 1 && y_stride < D) return fail(SLHIP_ERR_INVALID, "gather: output row stride is smaller than D");
    if (dtype_out != SLHIP_F32 && dtype_out != SLHIP_BF16)
        return fail(SLHIP_ERR_UNSUPPORTED, "gather: output dtype %d not supported", dtype_out);
    uint32_t* err = nullptr;
    int stc = index_error_word(&err);
    if (stc) return stc;
    GatherArgs a{static_cast<const uint8_t*>(table), V, D, D / bs * bb, ids, N, y, N > 1 ? y_stride : D, err};
    hipStream_t st = to_stream(stream);
    return dtype_out == SLHIP_BF16 ? dispatch<SLHIP_BF16>(format, a, st) : dispatch<SLHIP_F32>(format, a, st);
}
