// Standalone elementwise ops: the broadcasting binary ops (StandardOps.BinaryNames) and the one-operand ops
// (StandardOps.UnaryNames, Scale, Clip) that the lowerer does not fuse into a row norm, a gated activation or
// a matvec epilogue -- a bias add, a scalar Mul, a lone activation.
//
// Semantics follow the reference CPU provider: BinaryOp (src/Sharplight.Cpu/BinaryOp.cs:8-350) with
// numpy-style broadcasting by aligned strides (Align, :37-58: a dim of extent 1, or one the operand lacks,
// gets stride 0), and ScalarMath.Unary (src/Sharplight.Cpu/ScalarMath.cs:100-641) in the forms its vector
// loops compute (fused multiply-adds where they fuse, Gelu's rational erf, GeluTanh through exp).
// Arithmetic in f32; inputs and outputs f32, f16 or bf16.
//
// Layout: the host merges adjacent dims along which every operand stays linear (BinaryOp.Run's trailing
// merge, :84-99, applied to every dim) and drops extent-1 dims, leaving "rows" of L contiguous output
// elements under at most 7 outer dims. When L is a multiple of 8 and the output is 16-byte aligned, each
// wave takes a 512-element span of one row: its row offsets are wave-uniform (scalar registers, divided out
// in 32 bits while the indices fit), each lane one 8-element vector; both operands' loads are issued before
// either is used. Per operand the inner access is a 16-byte vector load (contiguous and aligned), one
// value per wave (broadcast along the row: a bias per row, a scalar), or 8 element loads (strided or
// unaligned). Lanes past the row's end redo its last vector and store the bytes its owner stores. Anything
// else runs a one-thread-per-element kernel over the full index.
#include "act.hpp"
#include "common.hpp"
#include "ew_ops.hpp"

#include <math.h>
#include <stdlib.h>

namespace slhip {

constexpr int kEwMaxDims = 8;

struct EwArgs {
    const void* a;
    const void* b;  // null for a one-operand op
    void* y;
    int op;
    float p0, p1;          // unary parameters (Scale: scale, bias; Clip: min, max; alpha/gamma)
    int nd;                // outer dims (the row index decomposes over them)
    int64_t dims[kEwMaxDims];
    int64_t sa[kEwMaxDims], sb[kEwMaxDims], sy[kEwMaxDims];  // outer strides, elements
    int64_t L;             // row length (innermost dim)
    int64_t sa_in, sb_in;  // innermost strides of a and b (0: broadcast along the row)
    int mode_a, mode_b;    // 0: 16-byte vectors, 1: one value per row, 2: element loads
    int64_t rows;          // product of the outer dims
    int64_t spans;         // 512-element spans per row (one per wave)
    int idx32;             // rows * spans < 2^32: the row index decomposes in 32-bit arithmetic
};

// ---- kernels ----------------------------------------------------------------------------------------

// Eight values of an operand at row offset `off`, columns c .. c + 7, in two steps: fetch8 issues the loads
// (a 16-byte vector, one value per row, or eight element loads), unpack8 turns them into f32. A kernel
// fetches both operands before it unpacks either, so that their loads are in flight together (a load whose
// result is used inside the mode branch makes the compiler wait for it before the next operand's loads).
template <int DT> struct Fetch8 {
    uint4 r[Vec<DT>::N == 4 ? 2 : 1];
    float v[8];
};

template <int DT>
__device__ __forceinline__ void fetch8(const void* base, int64_t off, int mode, int64_t s_in, int64_t c, Fetch8<DT>& f)
{
    using V = Vec<DT>;
    if (mode == 0) {
        const char* p = static_cast<const char*>(base) + (off + c) * V::BYTES;
        f.r[0] = load_nt(p);
        if constexpr (V::N == 4) f.r[1] = load_nt(p + 16);
    } else if (mode == 1) {
        f.v[0] = V::load1(base, off);
    } else {
#pragma unroll
        for (int e = 0; e < 8; e++) f.v[e] = V::load1(base, off + (c + e) * s_in);
    }
}

template <int DT>
__device__ __forceinline__ void unpack8(int mode, const Fetch8<DT>& f, float* v)
{
    using V = Vec<DT>;
    if (mode == 0) {
        V::unpack(f.r[0], v);
        if constexpr (V::N == 4) V::unpack(f.r[1], v + 4);
    } else if (mode == 1) {
#pragma unroll
        for (int e = 0; e < 8; e++) v[e] = f.v[0];
    } else {
#pragma unroll
        for (int e = 0; e < 8; e++) v[e] = f.v[e];
    }
}

template <int DA, int DB, int DO, bool BIN>
__global__ __launch_bounds__(256) void ew_vec(EwArgs a)
{
    const int64_t w = static_cast<int64_t>(blockIdx.x) * 4 + wave_id();
    if (w >= a.rows * a.spans) return;  // wave-uniform: whole waves past the end
    int64_t span, ao = 0, bo = 0, yo = 0;
    if (a.idx32) {  // wave-uniform row offsets; 32-bit divisions while the indices fit
        uint32_t r = static_cast<uint32_t>(w) / static_cast<uint32_t>(a.spans);
        span = static_cast<uint32_t>(w) - r * static_cast<uint32_t>(a.spans);
        for (int k = a.nd - 1; k >= 0; k--) {
            const uint32_t d = static_cast<uint32_t>(a.dims[k]);
            const uint32_t q = r / d;
            const int64_t ix = r - q * d;
            r = q;
            ao += ix * a.sa[k];
            bo += ix * a.sb[k];
            yo += ix * a.sy[k];
        }
    } else {
        int64_t r = w / a.spans;
        span = w - r * a.spans;
        for (int k = a.nd - 1; k >= 0; k--) {
            const int64_t q = r / a.dims[k];
            const int64_t ix = r - q * a.dims[k];
            r = q;
            ao += ix * a.sa[k];
            bo += ix * a.sb[k];
            yo += ix * a.sy[k];
        }
    }
    int64_t c = span * 512 + (threadIdx.x & 63) * 8;
    c = c < a.L - 8 ? c : a.L - 8;
    float x[8], o[8];
    Fetch8<DA> fa;
    Fetch8<DB> fb;
    fetch8<DA>(a.a, ao, a.mode_a, a.sa_in, c, fa);
    if constexpr (BIN) fetch8<DB>(a.b, bo, a.mode_b, a.sb_in, c, fb);
    unpack8<DA>(a.mode_a, fa, x);
    if constexpr (BIN) {
        float z[8];
        unpack8<DB>(a.mode_b, fb, z);
        switch (a.op) {  // the common ops get a loop of their own; the rest one switch per element
        case SLHIP_BIN_ADD:
#pragma unroll
            for (int e = 0; e < 8; e++) o[e] = x[e] + z[e];
            break;
        case SLHIP_BIN_MUL:
#pragma unroll
            for (int e = 0; e < 8; e++) o[e] = x[e] * z[e];
            break;
        case SLHIP_BIN_SUB:
#pragma unroll
            for (int e = 0; e < 8; e++) o[e] = x[e] - z[e];
            break;
        default:
#pragma unroll
            for (int e = 0; e < 8; e++) o[e] = binary_op(a.op, x[e], z[e], a.p0 != 0.0f);
        }
    } else {
        switch (a.op) {
        case SLHIP_UN_SILU:
#pragma unroll
            for (int e = 0; e < 8; e++) o[e] = unary_op(SLHIP_UN_SILU, x[e], 0.f, 0.f);
            break;
        case SLHIP_UN_SCALE:
#pragma unroll
            for (int e = 0; e < 8; e++) o[e] = fmaf(x[e], a.p0, a.p1);
            break;
        default:
#pragma unroll
            for (int e = 0; e < 8; e++) o[e] = unary_op(a.op, x[e], a.p0, a.p1);
        }
    }
    store_packed<DO, 8>(static_cast<char*>(a.y) + (yo + c) * Vec<DO>::BYTES, o);
}

// Any shape, stride and alignment: one thread per output element, the full index decomposed per element.
template <int DA, int DB, int DO, bool BIN>
__global__ __launch_bounds__(256) void ew_scalar(EwArgs a)
{
    const int64_t total = a.rows * a.L;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < total;
         i += static_cast<int64_t>(gridDim.x) * 256) {
        int64_t r = i / a.L;
        const int64_t c = i - r * a.L;
        int64_t ao = c * a.sa_in, bo = c * a.sb_in, yo = c;
        for (int k = a.nd - 1; k >= 0; k--) {
            const int64_t q = r / a.dims[k];
            const int64_t ix = r - q * a.dims[k];
            r = q;
            ao += ix * a.sa[k];
            bo += ix * a.sb[k];
            yo += ix * a.sy[k];
        }
        const float x = Vec<DA>::load1(a.a, ao);
        float o;
        if constexpr (BIN)
            o = binary_op(a.op, x, Vec<DB>::load1(a.b, bo), a.p0 != 0.0f);
        else
            o = unary_op(a.op, x, a.p0, a.p1);
        Vec<DO>::store1(a.y, yo, o);
    }
}

// ---- host -------------------------------------------------------------------------------------------

struct Shape {
    int n = 0;
    int64_t d[kEwMaxDims + 1];
    int64_t s[3][kEwMaxDims + 1];  // a, b, y
};

// Drops extent-1 dims and merges dim k into k+1 wherever every operand is linear across the pair.
static Shape canonical(const int64_t* dims, const int64_t* const* strides, int rank, int nops)
{
    Shape in;
    for (int k = 0; k < rank; k++) {
        if (dims[k] == 1) continue;
        in.d[in.n] = dims[k];
        for (int o = 0; o < nops; o++) in.s[o][in.n] = strides[o][k];
        in.n++;
    }
    Shape out;
    for (int k = 0; k < in.n; k++) {
        if (out.n > 0) {
            bool linear = true;
            for (int o = 0; o < nops; o++) linear &= out.s[o][out.n - 1] == in.s[o][k] * in.d[k];
            if (linear) {
                out.d[out.n - 1] *= in.d[k];
                for (int o = 0; o < nops; o++) out.s[o][out.n - 1] = in.s[o][k];
                continue;
            }
        }
        out.d[out.n] = in.d[k];
        for (int o = 0; o < nops; o++) out.s[o][out.n] = in.s[o][k];
        out.n++;
    }
    if (out.n == 0) {  // a single element
        out.d[0] = 1;
        for (int o = 0; o < nops; o++) out.s[o][0] = 1;
        out.n = 1;
    }
    return out;
}

template <int DA, int DB, int DO, bool BIN>
static int launch(EwArgs& a, bool vec, hipStream_t st)
{
    if (vec) {
        const int64_t waves = a.rows * a.spans;
        const int64_t blocks = (waves + 3) / 4;
        if (blocks > 0x7FFFFFFF) return fail(SLHIP_ERR_UNSUPPORTED, "elementwise: tensor too large");
        // (SLHIP_EW_INDEX64=1 takes the 64-bit form at any size, so that tests reach it)
        static const bool force64 = [] {
            const char* e = getenv("SLHIP_EW_INDEX64");
            return e && *e == '1';
        }();
        a.idx32 = waves <= 0xFFFFFFFFll && !force64 ? 1 : 0;
        ew_vec<DA, DB, DO, BIN><<<dim3(static_cast<unsigned>(blocks)), 256, 0, st>>>(a);
        return check_launch("ew_vec");
    }
    const int64_t total = a.rows * a.L;
    int64_t blocks = (total + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    ew_scalar<DA, DB, DO, BIN><<<dim3(static_cast<unsigned>(blocks)), 256, 0, st>>>(a);
    return check_launch("ew_scalar");
}

template <int DA, int DB, bool BIN>
static int by_out(EwArgs& a, int dout, bool vec, hipStream_t st)
{
    switch (dout) {
    case SLHIP_F32: return launch<DA, DB, SLHIP_F32, BIN>(a, vec, st);
    case SLHIP_F16: return launch<DA, DB, SLHIP_F16, BIN>(a, vec, st);
    case SLHIP_BF16: return launch<DA, DB, SLHIP_BF16, BIN>(a, vec, st);
    default: return fail(SLHIP_ERR_UNSUPPORTED, "elementwise: output dtype %d", dout);
    }
}

// Operand access mode along the row and the vector-path conditions on it.
static int operand_mode(const void* p, int64_t s_in, const int64_t* outer, int nd)
{
    if (s_in == 0) return 1;
    if (s_in != 1 || !aligned16(p)) return 2;
    for (int k = 0; k < nd; k++)
        if (outer[k] % 8 != 0) return 2;
    return 0;
}

static int run(int op, bool bin, int da, int db, int dout, const void* a, const int64_t* a_strides, const void* b,
               const int64_t* b_strides, void* y, const int64_t* y_strides, const int64_t* dims, int rank, float p0,
               float p1, hipStream_t st)
{
    if (rank < 0 || rank > kEwMaxDims) return fail(SLHIP_ERR_INVALID, "elementwise: rank %d outside 0..%d", rank, kEwMaxDims);
    if (rank > 0 && !dims) return fail(SLHIP_ERR_INVALID, "elementwise: dims are required");
    int64_t total = 1;
    for (int k = 0; k < rank; k++) {
        if (dims[k] < 0) return fail(SLHIP_ERR_INVALID, "elementwise: negative extent");
        total *= dims[k];
    }
    if (total == 0) return SLHIP_OK;
    if (!a || !y || (bin && !b)) return fail(SLHIP_ERR_INVALID, "elementwise: null tensor");
    for (int dt : {da, db, dout})
        if (dt != SLHIP_F32 && dt != SLHIP_F16 && dt != SLHIP_BF16)
            return fail(SLHIP_ERR_UNSUPPORTED, "elementwise: dtype %d", dt);
    if (bin && db != da && db != SLHIP_F32)
        return fail(SLHIP_ERR_UNSUPPORTED, "elementwise: b must have a's dtype or f32");

    // dense row-major strides for any operand given without strides
    int64_t dense[kEwMaxDims];
    int64_t acc = 1;
    for (int k = rank - 1; k >= 0; k--) {
        dense[k] = acc;
        acc *= dims[k];
    }
    const int64_t* ps[3] = {a_strides ? a_strides : dense, bin ? (b_strides ? b_strides : dense) : dense,
                            y_strides ? y_strides : dense};
    for (int k = 0; k < rank; k++)
        if (ps[2][k] < 0 || ps[0][k] < 0 || ps[1][k] < 0) return fail(SLHIP_ERR_INVALID, "elementwise: negative stride");
    const int64_t* order[3] = {ps[0], ps[1], ps[2]};
    Shape s = canonical(dims, order, rank, 3);

    EwArgs e{};
    e.a = a;
    e.b = bin ? b : nullptr;
    e.y = y;
    e.op = op;
    e.p0 = p0;
    e.p1 = p1;
    e.nd = s.n - 1;
    for (int k = 0; k < e.nd; k++) {
        e.dims[k] = s.d[k];
        e.sa[k] = s.s[0][k];
        e.sb[k] = s.s[1][k];
        e.sy[k] = s.s[2][k];
    }
    e.L = s.d[s.n - 1];
    e.sa_in = s.s[0][s.n - 1];
    e.sb_in = s.s[1][s.n - 1];
    const int64_t sy_in = s.s[2][s.n - 1];
    e.rows = total / e.L;
    e.spans = (e.L + 511) / 512;

    bool vec = e.L % 8 == 0 && sy_in == 1 && aligned16(y);
    for (int k = 0; k < e.nd; k++) vec &= e.sy[k] % 8 == 0;
    e.mode_a = operand_mode(a, e.sa_in, e.sa, e.nd);
    e.mode_b = bin ? operand_mode(b, e.sb_in, e.sb, e.nd) : 1;
    if (!vec) {
        if (sy_in != 1) {  // the scalar kernel writes y at yo = c + sum(ix * sy): make the inner stride explicit
            // fold the inner dim into the outer list so the kernel's column index is always stride 1 in y
            if (e.nd + 1 > kEwMaxDims) return fail(SLHIP_ERR_UNSUPPORTED, "elementwise: rank too high");
            e.dims[e.nd] = e.L;
            e.sa[e.nd] = e.sa_in;
            e.sb[e.nd] = e.sb_in;
            e.sy[e.nd] = sy_in;
            e.nd++;
            e.L = 1;
            e.sa_in = e.sb_in = 0;
            e.rows = total;
        }
    }

    if (!bin) db = da;
    if (da == SLHIP_F32) return bin ? by_out<SLHIP_F32, SLHIP_F32, true>(e, dout, vec, st) : by_out<SLHIP_F32, SLHIP_F32, false>(e, dout, vec, st);
    if (da == SLHIP_BF16) {
        if (!bin) return by_out<SLHIP_BF16, SLHIP_BF16, false>(e, dout, vec, st);
        return db == SLHIP_BF16 ? by_out<SLHIP_BF16, SLHIP_BF16, true>(e, dout, vec, st) : by_out<SLHIP_BF16, SLHIP_F32, true>(e, dout, vec, st);
    }
    if (!bin) return by_out<SLHIP_F16, SLHIP_F16, false>(e, dout, vec, st);
    return db == SLHIP_F16 ? by_out<SLHIP_F16, SLHIP_F16, true>(e, dout, vec, st) : by_out<SLHIP_F16, SLHIP_F32, true>(e, dout, vec, st);
}

}  // namespace slhip

using namespace slhip;

extern "C" SLHIP_API int slhip_binary(int op, int dtype_a, int dtype_b, int dtype_out, const void* a,
                                      const int64_t* a_strides, const void* b, const int64_t* b_strides, void* y,
                                      const int64_t* dims, int rank, slhip_stream stream)
{
    if (op < SLHIP_BIN_ADD || op > SLHIP_BIN_FMOD) return fail(SLHIP_ERR_INVALID, "binary: bad op %d", op);
    // BinaryOp.Apply's special exponents apply when b's stride along y's innermost dim is 0 (Align gives a
    // dim of extent 1 stride 0; a rank-0 output has no dims at all).
    const bool pow_special = rank == 0 || (dims && dims[rank - 1] == 1) || (b_strides && b_strides[rank - 1] == 0);
    return run(op, true, dtype_a, dtype_b, dtype_out, a, a_strides, b, b_strides, y, nullptr, dims, rank,
               pow_special ? 1.f : 0.f, 0.f, to_stream(stream));
}

extern "C" SLHIP_API int slhip_unary(int op, int dtype_in, int dtype_out, const void* x, void* y, int64_t rows,
                                     int64_t cols, int64_t x_stride, int64_t y_stride, float p0, float p1,
                                     slhip_stream stream)
{
    if (op < SLHIP_UN_NEG || op > SLHIP_UN_IS_INF) return fail(SLHIP_ERR_INVALID, "unary: bad op %d", op);
    if (rows < 0 || cols < 0) return fail(SLHIP_ERR_INVALID, "unary: negative shape");
    if (rows > 1 && (x_stride < cols || y_stride < cols)) return fail(SLHIP_ERR_INVALID, "unary: a row stride is smaller than cols");
    const int64_t dims[2] = {rows, cols};
    const int64_t xs[2] = {x_stride, 1}, ys[2] = {y_stride, 1};
    return run(op, false, dtype_in, dtype_in, dtype_out, x, xs, nullptr, nullptr, y, ys, dims, 2, p0, p1,
               to_stream(stream));
}
