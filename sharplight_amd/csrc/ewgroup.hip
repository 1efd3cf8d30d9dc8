// Fused elementwise groups: a chain of elementwise nodes of one output shape evaluated per element in one
// launch, optionally with the row norm before it (a norm whose output only the group reads) or after it (a
// norm of one of the group's values) -- the reference lowerer's fused elementwise unit and its NormHead /
// NormTail folds (src/Sharplight.Shaders/Lowering/GraphLowerer.Fusion.cs:88-285; the generated kernels of
// ElementwiseCodegen.cs and RowNormKernelSource.cs:75-106).
//
// The group arrives as a small program (slhip_ew_program): inputs are loaded into registers 0 .. n_inputs-1,
// then each op writes its destination register; each op is the f32 arithmetic of the standalone op (ew_ops.hpp), its
// result rounded to the node's output type when that is not f32 -- so the group computes bit for bit what the
// nodes compute one launch at a time. Only the registers some reader outside the group needs are stored.
//
// Flat form (no norm): a wave takes 256 consecutive elements of one row, four per lane; every input is
// fetched before any op runs. The op codes are wave-uniform, so the interpreter's dispatch runs on the scalar
// unit while the vector unit does the arithmetic on four values per lane.
// Row form (a norm head or tail): a wave per row, two passes over it in 256-element steps: pass 1 sums the
// squares of the norm's operand (the head's input, or the tail's register after running the group, whose
// outputs it stores); pass 2 runs the group with the normalized head (and stores its outputs), or runs it
// again to normalize the tail register into y. The row's second read hits the cache.
#include "common.hpp"
#include "ew_ops.hpp"

#include <stdlib.h>
#include <string.h>

namespace slhip {

constexpr int kEwgRegs = SLHIP_EW_MAX_REGS;

struct EwgArgs {
    slhip_ew_program p;
    int64_t rows, cols;
    int pow_special[SLHIP_EW_MAX_OPS];  // Pow with a per-row or scalar exponent: the reference's special forms
};

typedef float f4v __attribute__((ext_vector_type(4)));

// The register file: sixteen named four-value registers read and written through switches on the (wave-
// uniform) index, which keeps them in VGPRs -- an array indexed at run time would live in scratch memory.
struct Regs {
    f4v r0, r1, r2, r3, r4, r5, r6, r7, r8, r9, r10, r11, r12, r13, r14, r15;
#define SLHIP_EWG_CASES(X) X(0) X(1) X(2) X(3) X(4) X(5) X(6) X(7) X(8) X(9) X(10) X(11) X(12) X(13) X(14) X(15)
    __device__ __forceinline__ f4v get(int i) const
    {
        switch (i) {
#define SLHIP_EWG_GET(k) case k: return r##k;
            SLHIP_EWG_CASES(SLHIP_EWG_GET)
#undef SLHIP_EWG_GET
        default: return r0;
        }
    }
    __device__ __forceinline__ void set(int i, f4v v)
    {
        switch (i) {
#define SLHIP_EWG_SET(k) case k: r##k = v; break;
            SLHIP_EWG_CASES(SLHIP_EWG_SET)
#undef SLHIP_EWG_SET
        default: break;
        }
    }
#undef SLHIP_EWG_CASES
};
static_assert(kEwgRegs == 16, "the register file has sixteen registers");

// Four values of input i at row r, columns c .. c + 3 (c + 3 < cols, or the clamped last vector).
__device__ __forceinline__ f4v fetch4(const slhip_ew_input& in, int64_t r, int64_t c, int64_t cols)
{
    f4v v;
    int64_t off;
    switch (in.mode) {
    case SLHIP_EWI_ROW: off = c; break;
    case SLHIP_EWI_COL: off = r; break;
    case SLHIP_EWI_SCALAR: off = 0; break;
    default: off = r * cols + c; break;
    }
    if (in.mode == SLHIP_EWI_COL || in.mode == SLHIP_EWI_SCALAR) {
        float x;
        if (in.dtype == SLHIP_F32) x = static_cast<const float*>(in.data)[off];
        else if (in.dtype == SLHIP_BF16) x = __uint_as_float(static_cast<uint32_t>(static_cast<const uint16_t*>(in.data)[off]) << 16);
        else x = static_cast<float>(static_cast<const _Float16*>(in.data)[off]);
        v[0] = v[1] = v[2] = v[3] = x;
        return v;
    }
    if (in.dtype == SLHIP_F32) {
        const float4 f = *reinterpret_cast<const float4*>(static_cast<const float*>(in.data) + off);
        v[0] = f.x; v[1] = f.y; v[2] = f.z; v[3] = f.w;
    } else {
        const uint2 b = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(in.data) + off);
        if (in.dtype == SLHIP_BF16) {
            v[0] = bf16_lo(b.x); v[1] = bf16_hi(b.x); v[2] = bf16_lo(b.y); v[3] = bf16_hi(b.y);
        } else {
            v[0] = f16_lo(b.x); v[1] = f16_hi(b.x); v[2] = f16_lo(b.y); v[3] = f16_hi(b.y);
        }
    }
    return v;
}

__device__ __forceinline__ void store4(void* p, int dt, int64_t off, f4v v)
{
    if (dt == SLHIP_F32) {
        *reinterpret_cast<float4*>(static_cast<float*>(p) + off) = make_float4(v[0], v[1], v[2], v[3]);
    } else if (dt == SLHIP_BF16) {
        *reinterpret_cast<uint2*>(static_cast<uint16_t*>(p) + off) =
            make_uint2(f32_to_bf16_bits(v[0]) | (f32_to_bf16_bits(v[1]) << 16), f32_to_bf16_bits(v[2]) | (f32_to_bf16_bits(v[3]) << 16));
    } else {
        *reinterpret_cast<uint2*>(static_cast<uint16_t*>(p) + off) = make_uint2(pack_f16x2(v[0], v[1]), pack_f16x2(v[2], v[3]));
    }
}

// A value rounded to a node's output type (the unfused graph stores it in that type).
__device__ __forceinline__ float round_to(int dt, float v)
{
    if (dt == SLHIP_BF16) return __uint_as_float(f32_to_bf16_bits(v) << 16);
    if (dt == SLHIP_F16) return static_cast<float>(static_cast<_Float16>(v));
    return v;
}

// The ops of the program on the registers.
__device__ __forceinline__ void run_ops(const EwgArgs& a, Regs& R)
{
    for (int k = 0; k < a.p.n_ops; k++) {  // uniform
        const slhip_ew_op& o = a.p.ops[k];
        const f4v x = R.get(o.a);
        f4v r;
        if (o.kind == SLHIP_EWK_BINARY) {
            const f4v y = R.get(o.b);
            const bool ps = a.pow_special[k] != 0;
#pragma unroll
            for (int e = 0; e < 4; e++) r[e] = binary_op(o.op, x[e], y[e], ps);
        } else {
#pragma unroll
            for (int e = 0; e < 4; e++) r[e] = unary_op(o.op, x[e], o.p0, o.p1);
        }
        if (o.round != SLHIP_F32) {
#pragma unroll
            for (int e = 0; e < 4; e++) r[e] = round_to(o.round, r[e]);
        }
        R.set(o.dst, r);
    }
}

__device__ __forceinline__ void fetch_inputs(const EwgArgs& a, int64_t r, int64_t c, Regs& R)
{
    for (int i = 0; i < a.p.n_inputs; i++) R.set(i, fetch4(a.p.inputs[i], r, c, a.cols));
}

__device__ __forceinline__ void store_outputs(const EwgArgs& a, int64_t r, int64_t c, const Regs& R)
{
    for (int j = 0; j < a.p.n_outputs; j++) {
        const slhip_ew_output& o = a.p.outputs[j];
        store4(o.data, o.dtype, r * a.cols + c, R.get(o.reg));
    }
}

// Flat form: wave w of the grid takes row w / spans, elements 256 (w % spans) + 4 lane .. + 3.
__global__ __launch_bounds__(256) void ewg_flat(EwgArgs a, int64_t spans)
{
    const int64_t w = static_cast<int64_t>(blockIdx.x) * 4 + wave_id();
    if (w >= a.rows * spans) return;
    const int64_t r = w / spans;
    int64_t c = (w - r * spans) * 256 + 4 * (threadIdx.x & 63);
    c = c < a.cols ? c : a.cols - 4;  // lanes past the row's end redo its last vector
    Regs R{};
    fetch_inputs(a, r, c, R);
    run_ops(a, R);
    store_outputs(a, r, c, R);
}

// Row form: one wave per row (see the file comment).
__global__ __launch_bounds__(256) void ewg_row(EwgArgs a)
{
    const int64_t r = static_cast<int64_t>(blockIdx.x) * 4 + wave_id();
    if (r >= a.rows) return;
    const int lane = threadIdx.x & 63;
    const bool head = a.p.head.kind != 0;
    const slhip_ew_norm& nm = head ? a.p.head : a.p.tail;
    Regs R{};
    // pass 1: the sum of squares of the norm's operand (tail: after the group, whose outputs are stored now)
    float q = 0.0f;
    for (int64_t c0 = 0; c0 < a.cols; c0 += 256) {
        int64_t c = c0 + 4 * lane;
        const bool own = c < a.cols;
        c = own ? c : a.cols - 4;
        fetch_inputs(a, r, c, R);
        if (!head) {
            run_ops(a, R);
            store_outputs(a, r, c, R);
        }
        const f4v v = R.get(nm.reg);
        const float s = fmaf(v[0], v[0], v[1] * v[1]) + fmaf(v[2], v[2], v[3] * v[3]);
        q += own ? s : 0.0f;
    }
    q = wave_sum(q);
    // RowOp (src/Sharplight.Cpu/RowOp.cs:63-84): scale = 1 / sqrt(sum / n + eps), L2Norm 1 / sqrt(sum + eps)
    const float scale = nm.kind == SLHIP_EWN_L2 ? 1.0f / sqrtf(q + nm.eps) : 1.0f / sqrtf(q / static_cast<float>(a.cols) + nm.eps);
    // pass 2
    for (int64_t c0 = 0; c0 < a.cols; c0 += 256) {
        int64_t c = c0 + 4 * lane;
        c = c < a.cols ? c : a.cols - 4;
        fetch_inputs(a, r, c, R);
        float wv[4] = {1.0f, 1.0f, 1.0f, 1.0f};
        if (nm.w) {
            const float4 t = *reinterpret_cast<const float4*>(nm.w + c);
            wv[0] = t.x; wv[1] = t.y; wv[2] = t.z; wv[3] = t.w;
        }
        if (head) {
            f4v h = R.get(nm.reg);
#pragma unroll
            for (int e = 0; e < 4; e++) h[e] = round_to(nm.dtype_y, (h[e] * scale) * wv[e]);
            R.set(nm.reg, h);
            run_ops(a, R);
            store_outputs(a, r, c, R);
        } else {
            run_ops(a, R);
            const f4v t = R.get(nm.reg);
            f4v y;
#pragma unroll
            for (int e = 0; e < 4; e++) y[e] = (t[e] * scale) * wv[e];
            store4(nm.y, nm.dtype_y, r * a.cols + c, y);
        }
    }
}

static int check_program(const slhip_ew_program* p, int64_t rows, int64_t cols)
{
    if (!p) return fail(SLHIP_ERR_INVALID, "ew_program: null program");
    if (rows < 0 || cols < 0) return fail(SLHIP_ERR_INVALID, "ew_program: negative shape");
    if (p->n_inputs < 1 || p->n_inputs > SLHIP_EW_MAX_INPUTS || p->n_ops < 0 || p->n_ops > SLHIP_EW_MAX_OPS ||
        p->n_outputs < 0 || p->n_outputs > SLHIP_EW_MAX_OUTPUTS)
        return fail(SLHIP_ERR_INVALID, "ew_program: %d inputs (1..%d), %d ops (0..%d), %d outputs (0..%d)", p->n_inputs,
                    SLHIP_EW_MAX_INPUTS, p->n_ops, SLHIP_EW_MAX_OPS, p->n_outputs, SLHIP_EW_MAX_OUTPUTS);
    const int nreg = SLHIP_EW_MAX_REGS;
    auto dt_ok = [](int d) { return d == SLHIP_F32 || d == SLHIP_BF16 || d == SLHIP_F16; };
    for (int i = 0; i < p->n_inputs; i++) {
        const slhip_ew_input& in = p->inputs[i];
        if (!in.data || !dt_ok(in.dtype) || in.mode < SLHIP_EWI_FULL || in.mode > SLHIP_EWI_SCALAR)
            return fail(SLHIP_ERR_INVALID, "ew_program: input %d is incomplete", i);
        if (in.mode == SLHIP_EWI_FULL || in.mode == SLHIP_EWI_ROW) {
            const uintptr_t al = in.dtype == SLHIP_F32 ? 16 : 8;
            if (reinterpret_cast<uintptr_t>(in.data) % al != 0)
                return fail(SLHIP_ERR_UNSUPPORTED, "ew_program: input %d is not %d-byte aligned", i, static_cast<int>(al));
        }
    }
    for (int k = 0; k < p->n_ops; k++) {
        const slhip_ew_op& o = p->ops[k];
        if (o.kind != SLHIP_EWK_BINARY && o.kind != SLHIP_EWK_UNARY) return fail(SLHIP_ERR_INVALID, "ew_program: op %d kind", k);
        if (o.a < 0 || o.a >= nreg || (o.kind == SLHIP_EWK_BINARY && (o.b < 0 || o.b >= nreg)) || o.dst < 0 || o.dst >= nreg)
            return fail(SLHIP_ERR_INVALID, "ew_program: op %d register out of range", k);
        if (o.kind == SLHIP_EWK_BINARY ? (o.op < SLHIP_BIN_ADD || o.op > SLHIP_BIN_FMOD)
                                       : (o.op < 0 || o.op > SLHIP_UN_IS_INF))
            return fail(SLHIP_ERR_INVALID, "ew_program: op %d code %d", k, o.op);
        if (!dt_ok(o.round)) return fail(SLHIP_ERR_INVALID, "ew_program: op %d rounding type", k);
    }
    for (int j = 0; j < p->n_outputs; j++) {
        const slhip_ew_output& o = p->outputs[j];
        if (!o.data || !dt_ok(o.dtype) || o.reg < 0 || o.reg >= nreg)
            return fail(SLHIP_ERR_INVALID, "ew_program: output %d is incomplete", j);
        if (reinterpret_cast<uintptr_t>(o.data) % (o.dtype == SLHIP_F32 ? 16 : 8) != 0)
            return fail(SLHIP_ERR_UNSUPPORTED, "ew_program: output %d is misaligned", j);
    }
    if (p->head.kind && p->tail.kind) return fail(SLHIP_ERR_INVALID, "ew_program: a norm head or a norm tail, not both");
    const slhip_ew_norm& nm = p->head.kind ? p->head : p->tail;
    if (nm.kind) {
        if (nm.kind != SLHIP_EWN_RMS && nm.kind != SLHIP_EWN_L2) return fail(SLHIP_ERR_INVALID, "ew_program: norm kind");
        if (p->head.kind && (nm.reg < 0 || nm.reg >= p->n_inputs || p->inputs[nm.reg].mode != SLHIP_EWI_FULL))
            return fail(SLHIP_ERR_INVALID, "ew_program: the norm head normalizes a full-shape input register");
        if (p->tail.kind && (nm.reg < 0 || nm.reg >= nreg || !nm.y || !dt_ok(nm.dtype_y)))
            return fail(SLHIP_ERR_INVALID, "ew_program: the norm tail is incomplete");
        if (p->head.kind && !dt_ok(nm.dtype_y)) return fail(SLHIP_ERR_INVALID, "ew_program: the norm head's type");
        if (nm.w && reinterpret_cast<uintptr_t>(nm.w) % 16 != 0) return fail(SLHIP_ERR_UNSUPPORTED, "ew_program: norm weight misaligned");
        if (p->tail.kind && reinterpret_cast<uintptr_t>(nm.y) % (nm.dtype_y == SLHIP_F32 ? 16 : 8) != 0)
            return fail(SLHIP_ERR_UNSUPPORTED, "ew_program: norm output misaligned");
    } else if (p->n_outputs == 0) {
        return fail(SLHIP_ERR_INVALID, "ew_program: nothing to store");
    }
    if (cols % 4 != 0) return fail(SLHIP_ERR_UNSUPPORTED, "ew_program: rows of %lld values (a multiple of 4 is required)",
                                   static_cast<long long>(cols));
    return SLHIP_OK;
}

}  // namespace slhip

using namespace slhip;

extern "C" SLHIP_API int slhip_ew_program_run(const slhip_ew_program* prog, int64_t rows, int64_t cols, slhip_stream stream)
{
    const int st = check_program(prog, rows, cols);
    if (st != SLHIP_OK) return st;
    if (rows == 0 || cols == 0) return SLHIP_OK;
    EwgArgs a{};
    a.p = *prog;
    a.rows = rows;
    a.cols = cols;
    for (int k = 0; k < prog->n_ops; k++) {
        const slhip_ew_op& o = prog->ops[k];
        // the reference's special Pow forms apply when the exponent is one value along the row (BinaryOp.Apply)
        a.pow_special[k] = o.kind == SLHIP_EWK_BINARY && o.op == SLHIP_BIN_POW && o.b < prog->n_inputs &&
                           (prog->inputs[o.b].mode == SLHIP_EWI_COL || prog->inputs[o.b].mode == SLHIP_EWI_SCALAR);
    }
    hipStream_t s = to_stream(stream);
    if (prog->head.kind || prog->tail.kind) {
        if (rows > 0x7FFFFFFFLL * 4) return fail(SLHIP_ERR_UNSUPPORTED, "ew_program: too many rows");
        ewg_row<<<dim3(static_cast<unsigned>((rows + 3) / 4)), 256, 0, s>>>(a);
        return check_launch("ewg_row");
    }
    const int64_t spans = (cols + 255) / 256;
    const int64_t blocks = (rows * spans + 3) / 4;
    if (blocks > 0x7FFFFFFF) return fail(SLHIP_ERR_UNSUPPORTED, "ew_program: grid too large");
    ewg_flat<<<dim3(static_cast<unsigned>(blocks)), 256, 0, s>>>(a, spans);
    return check_launch("ewg_flat");
}
