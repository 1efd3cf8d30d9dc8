// Gated activations out = act(gate) * up (SwiGLU, GeGLU with tanh-GELU, GELU-erf gating).
//
// Semantics: the reference computes Mul(act(gate), up) as two f32 ops on the CPU
// (src/Sharplight.Cpu/ScalarMath.cs:552-641, BinaryOp.cs:8-103) and as one generated elementwise
// kernel on the GPU (fused[Silu,Mul], src/Sharplight.Shaders/Lowering/GraphLowerer.Fusion.cs:89-142).
// The activation forms are the CPU provider's vector forms:
//   SILU:      g / (1 + exp(-g))
//   GELU_TANH: g / (1 + exp(-u)),  u = (2*0.7978845608) * fma(0.044715*g, g*g, g)
//   GELU_ERF:  0.5*g*(1 + erf(g*0.70710678)), erf as below
// SILU and GELU_TANH run in f32 with the hardware exp2 / reciprocal (v_exp_f32, v_rcp_f32: ~1 ulp),
// which keeps the kernel on the HBM roofline (a bf16 SwiGLU moves 6 bytes per element, leaving ~20 VALU
// slots per element at 8 TB/s).
//
// Layout: pure streaming. Each lane owns U consecutive 16-byte vectors of the output per iteration; a
// block of 256 lanes covers 256*U vectors; the grid strides over the flattened tensor (contiguous rows)
// or over (row, vector) pairs (strided rows, e.g. gate/up halves of one merged projection).
#include "act.hpp"
#include "common.hpp"

#include <stdlib.h>

namespace slhip {

struct GatedArgs {
    const void* g;
    const void* u;
    void* o;
    int64_t rows;
    int64_t vpr;  // 16-byte input vectors per row
    int64_t gs, us, os;  // row strides in elements
    int64_t total;  // rows * vpr
};

template <int ACT, int DTI, int DTO, int U, bool CONTIG>
__global__ __launch_bounds__(256) void gated_vec(GatedArgs a)
{
    using VI = Vec<DTI>;
    constexpr int E = VI::N;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * 256 * U;
    for (int64_t base = (static_cast<int64_t>(blockIdx.x) * 256) * U + threadIdx.x; base < a.total; base += stride) {
        uint4 gr[U], ur[U];
        int64_t gi[U], ui[U], oi[U];
        bool ok[U];
#pragma unroll
        for (int k = 0; k < U; k++) {
            int64_t v = base + k * 256;
            ok[k] = v < a.total;
            if (CONTIG) {
                gi[k] = ui[k] = oi[k] = v * E;
            } else {
                int64_t r = v / a.vpr, c = (v - r * a.vpr) * E;
                gi[k] = r * a.gs + c;
                ui[k] = r * a.us + c;
                oi[k] = r * a.os + c;
            }
            if (ok[k]) {
                gr[k] = load_nt(static_cast<const char*>(a.g) + gi[k] * VI::BYTES);
                ur[k] = load_nt(static_cast<const char*>(a.u) + ui[k] * VI::BYTES);
            }
        }
#pragma unroll
        for (int k = 0; k < U; k++) {
            if (!ok[k]) continue;
            float gf[E], uf[E], of[E];
            VI::unpack(gr[k], gf);
            VI::unpack(ur[k], uf);
#pragma unroll
            for (int e = 0; e < E; e++) of[e] = activate<ACT>(gf[e]) * uf[e];
            store_packed<DTO, E>(static_cast<char*>(a.o) + oi[k] * Vec<DTO>::BYTES, of);
        }
    }
}

template <int ACT, int DTI, int DTO>
__global__ __launch_bounds__(256) void gated_scalar(const void* g, const void* u, void* o, int64_t rows, int64_t cols,
                                                    int64_t gs, int64_t us, int64_t os)
{
    const int64_t total = rows * cols;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < total;
         i += static_cast<int64_t>(gridDim.x) * 256) {
        int64_t r = i / cols, c = i - r * cols;
        float gv = Vec<DTI>::load1(g, r * gs + c);
        float uv = Vec<DTI>::load1(u, r * us + c);
        Vec<DTO>::store1(o, r * os + c, activate<ACT>(gv) * uv);
    }
}

static int env_int(const char* name, int dflt)
{
    const char* s = getenv(name);
    return s && *s ? atoi(s) : dflt;
}

static int device_cus()
{
    static int cus = 0;
    if (!cus) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
            cus = 256;
    }
    return cus;
}

template <int ACT, int DTI, int DTO>
static int dispatch(const void* g, const void* u, void* o, int64_t rows, int64_t cols, int64_t gs, int64_t us,
                    int64_t os, hipStream_t st)
{
    constexpr int E = Vec<DTI>::N;
    constexpr int OA = E * Vec<DTO>::BYTES < 16 ? E * Vec<DTO>::BYTES : 16;
    bool vec_ok = cols % E == 0 && aligned16(g) && aligned16(u) && gs % E == 0 && us % E == 0 &&
                  reinterpret_cast<uintptr_t>(o) % OA == 0 && (os * Vec<DTO>::BYTES) % OA == 0;
    if (vec_ok) {
        GatedArgs a{g, u, o, rows, cols / E, gs, us, os, rows * (cols / E)};
        const bool contig = gs == cols && us == cols && os == cols;
        // A flat grid: every wave streams one span and exits (measured on MI355X: ~8% more bandwidth than
        // a grid-stride loop over a resident grid). The loop remains for grids beyond 2^31 blocks.
        const int u = env_int("SLHIP_GATED_U", 1) == 2 ? 2 : 1;  // 1: one 16-byte vector per lane (fastest)
        const int64_t blocks_needed = (a.total + 256 * u - 1) / (256 * u);
        const unsigned grid = static_cast<unsigned>(blocks_needed < 0x7FFFFFFF ? blocks_needed : 0x7FFFFFFF);
        if (u == 1) {
            if (contig) gated_vec<ACT, DTI, DTO, 1, true><<<grid, 256, 0, st>>>(a);
            else gated_vec<ACT, DTI, DTO, 1, false><<<grid, 256, 0, st>>>(a);
        } else {
            if (contig) gated_vec<ACT, DTI, DTO, 2, true><<<grid, 256, 0, st>>>(a);
            else gated_vec<ACT, DTI, DTO, 2, false><<<grid, 256, 0, st>>>(a);
        }
        return check_launch("gated_vec");
    }
    int64_t total = rows * cols;
    int64_t blocks = (total + 255) / 256;
    int64_t cap = static_cast<int64_t>(device_cus()) * 8;
    gated_scalar<ACT, DTI, DTO><<<static_cast<unsigned>(blocks < cap ? blocks : cap), 256, 0, st>>>(g, u, o, rows, cols,
                                                                                                  gs, us, os);
    return check_launch("gated_scalar");
}

template <int ACT>
static int by_dtype(int di, int dout, const void* g, const void* u, void* o, int64_t rows, int64_t cols, int64_t gs,
                    int64_t us, int64_t os, hipStream_t st)
{
    if (di == SLHIP_BF16 && dout == SLHIP_BF16) return dispatch<ACT, SLHIP_BF16, SLHIP_BF16>(g, u, o, rows, cols, gs, us, os, st);
    if (di == SLHIP_F32 && dout == SLHIP_F32) return dispatch<ACT, SLHIP_F32, SLHIP_F32>(g, u, o, rows, cols, gs, us, os, st);
    if (di == SLHIP_BF16 && dout == SLHIP_F32) return dispatch<ACT, SLHIP_BF16, SLHIP_F32>(g, u, o, rows, cols, gs, us, os, st);
    if (di == SLHIP_F32 && dout == SLHIP_BF16) return dispatch<ACT, SLHIP_F32, SLHIP_BF16>(g, u, o, rows, cols, gs, us, os, st);
    return fail(SLHIP_ERR_UNSUPPORTED, "gated_act: dtype pair (%d -> %d) not supported", di, dout);
}

}  // namespace slhip

using namespace slhip;

extern "C" SLHIP_API int slhip_gated_act(int act, int dtype_in, int dtype_out, const void* gate, const void* up,
                                         void* out, int64_t rows, int64_t cols, int64_t gate_stride, int64_t up_stride,
                                         int64_t out_stride, slhip_stream stream)
{
    if (rows < 0 || cols < 0) return fail(SLHIP_ERR_INVALID, "gated_act: negative shape");
    if (rows == 0 || cols == 0) return SLHIP_OK;
    if (!gate || !up || !out) return fail(SLHIP_ERR_INVALID, "gated_act: null tensor");
    if (rows > 1 && (gate_stride < cols || up_stride < cols || out_stride < cols))
        return fail(SLHIP_ERR_INVALID, "gated_act: a row stride is smaller than cols");
    if (rows == 1) gate_stride = up_stride = out_stride = cols;
    hipStream_t st = to_stream(stream);
    switch (act) {
    case SLHIP_ACT_SILU: return by_dtype<SLHIP_ACT_SILU>(dtype_in, dtype_out, gate, up, out, rows, cols, gate_stride, up_stride, out_stride, st);
    case SLHIP_ACT_GELU_TANH: return by_dtype<SLHIP_ACT_GELU_TANH>(dtype_in, dtype_out, gate, up, out, rows, cols, gate_stride, up_stride, out_stride, st);
    case SLHIP_ACT_GELU_ERF: return by_dtype<SLHIP_ACT_GELU_ERF>(dtype_in, dtype_out, gate, up, out, rows, cols, gate_stride, up_stride, out_stride, st);
    default: return fail(SLHIP_ERR_INVALID, "gated_act: bad activation %d", act);
    }
}
