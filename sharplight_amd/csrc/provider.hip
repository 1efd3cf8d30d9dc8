// The Sharplight.Hip execution provider's host side: a compiled graph segment over the fused-layer-op
// kernels, mirroring the reference's provider contracts (src/Sharplight.Core/Runtime/IExecutionProvider.cs,
// IComputeDevice.cs, ICompiledSegment.cs) for the ops on this path.
//
//   IExecutionProvider.CheckAvailability  -> slhip_provider_check
//   IComputeDevice.Supports(Node)         -> slhip_node_supports / SegmentCompiler::supports
//   IComputeDevice.Compile(segment, opts) -> slhip_segment_compile (opts.MaxTokens bounds the symbol T)
//   ICompiledSegment.SetInput / Execute / GetOutput / ResetState / DeviceMemoryBytes
//                                         -> slhip_segment_set_input / _execute / _get_output / ...
//
// Compile lowers the segment's nodes into fused units with the fusion rules of the reference's shared
// lowerer (src/Sharplight.Shaders/Lowering/GraphLowerer.Fusion.cs):
//   * Add followed by RmsNorm / L2Norm of its result (rank-1 f32 weight or none) -> one residual row-norm
//     launch that also writes the sum when anything else reads it (FoldNormTails, :215-238);
//   * Silu / GeluTanh / Gelu whose only consumer is a Mul -> one gated-activation launch (the fused
//     elementwise unit, :89-142; IMlpActivation.ActivateGated, Architectures/IMlpActivation.cs:12);
//   * RmsNorm with an f32 [D] weight whose only consumer is a Rope -> computed inside the rope launch
//     (AbsorbIntoConsumers, :618-630); Rope launches that share positions and settings (q and k of a
//     layer) are merged into one launch of up to four tensors;
//   * a Rope whose only consumer is a CacheWrite -> the rope stores into the cache rows (:633-648);
//   * a Cast to f16 of a row norm's f32 output -> the f16 copy written by the norm launch, which then skips
//     the f32 rows when nothing else reads them (GraphLowerer.HalfCopies.cs:106-151);
//   * two MatMuls sharing x whose products feed act(gate) * up -> one dual matvec launch with the gating
//     epilogue (FoldDualMatMuls, :286-353);
//   * RmsNorm, L2Norm, LayerNorm, Rope, Gather, Cast, CacheWrite and MatMul (decode matvec) on their own;
//   * every other elementwise node -- the binary ops with numpy broadcasting (a bias add, a scalar Mul),
//     the one-operand ops, Scale and Clip -- as one standalone elementwise launch (the CPU provider's
//     BinaryOp / UnaryOp, src/Sharplight.Cpu/CpuCompiledSegment.LowerElementwise.cs:8-72).
//
// The graph reaches the C ABI as a small line-based text form (one value, node, input, weight or output
// per line; see slhip_segment_compile in include/sharplight_hip.h); the managed provider writes it from a
// GraphSegment.
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <cmath>
#include <tuple>
#include <map>
#include <memory>
#include <set>
#include <sstream>
#include <stdexcept>
#include <string>
#include <vector>

#include "common.hpp"

namespace slhip {
namespace {

// ---- errors: the reference's exception types, as statuses --------------------------------------------

struct Error : std::runtime_error {
    int status;
    Error(int s, const std::string& m) : std::runtime_error(m), status(s) {}
};
[[noreturn]] void invalid(const std::string& m) { throw Error(SLHIP_ERR_INVALID, m); }       // ArgumentException
[[noreturn]] void unsupported(const std::string& m) { throw Error(SLHIP_ERR_UNSUPPORTED, m); }  // NotSupportedException
void check(int st)
{
    if (st != SLHIP_OK) throw Error(st, slhip_last_error());
}

// ---- graph ---------------------------------------------------------------------------------------------

enum class DType { F32, F16, BF16, I32, Q8_0, Q4_0, Q4_1, Q5_0, Q5_1, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, IQ4_NL, IQ4_XS, TQ1_0, TQ2_0, MXFP4, NVFP4,
                   IQ2_XXS, IQ2_XS, IQ2_S, IQ3_XXS, IQ3_S, IQ1_S, IQ1_M, Q1_0, Q2_0, Q2_0_G128, TERN1_G128, NVFP4_GS, Q4Z_G32, Q4Z_G128, Q8Z_G32, Q8Z_G128, NF4_B64, FP4_B64, Q8A_G32, Q2S_G128, F8E4M3, F8E5M2, F8E4M3_B32, F8E4M3_B128, TRELLIS_V4K8_G128, TRELLIS_V4K6_G128, TRELLIS_V4K7_G128, TRELLIS_V2K5_G128, TRELLIS_V2K6_G128, TRELLIS_V2K7_G128 };

struct TypeInfo {
    const char* name;
    DType t;
    int block;      // values per block
    int block_bytes;
};
const TypeInfo kTypes[] = {
    {"f32", DType::F32, 1, 4},     {"f16", DType::F16, 1, 2},     {"bf16", DType::BF16, 1, 2},
    {"i32", DType::I32, 1, 4},     {"q8_0", DType::Q8_0, 32, 34}, {"q4_0", DType::Q4_0, 32, 18},
    {"q4_1", DType::Q4_1, 32, 20}, {"q5_0", DType::Q5_0, 32, 22}, {"q5_1", DType::Q5_1, 32, 24},
    {"q2_k", DType::Q2_K, 256, 84}, {"q3_k", DType::Q3_K, 256, 110}, {"q4_k", DType::Q4_K, 256, 144},
    {"q5_k", DType::Q5_K, 256, 176}, {"q6_k", DType::Q6_K, 256, 210}, {"iq4_nl", DType::IQ4_NL, 32, 18},
    {"iq4_xs", DType::IQ4_XS, 256, 136}, {"tq1_0", DType::TQ1_0, 256, 54}, {"tq2_0", DType::TQ2_0, 256, 66},
    {"mxfp4", DType::MXFP4, 32, 17}, {"nvfp4", DType::NVFP4, 64, 36}, {"iq2_xxs", DType::IQ2_XXS, 256, 66},
    {"iq2_xs", DType::IQ2_XS, 256, 74}, {"iq2_s", DType::IQ2_S, 256, 82}, {"iq3_xxs", DType::IQ3_XXS, 256, 98},
    {"iq3_s", DType::IQ3_S, 256, 110}, {"iq1_s", DType::IQ1_S, 256, 50}, {"iq1_m", DType::IQ1_M, 256, 56},
    // the reference's own formats (src/Sharplight.Core/Tensors/DataType.cs:154-244)
    {"q1_0", DType::Q1_0, 128, 18},
    {"q2_0", DType::Q2_0, 64, 18},
    {"q2_0_g128", DType::Q2_0_G128, 128, 34},
    {"tern1_g128", DType::TERN1_G128, 128, 28},
    {"nvfp4_gs", DType::NVFP4_GS, 64, 40},
    {"q4z_g32", DType::Q4Z_G32, 32, 20},
    {"q4z_g128", DType::Q4Z_G128, 128, 68},
    {"q8z_g32", DType::Q8Z_G32, 32, 36},
    {"q8z_g128", DType::Q8Z_G128, 128, 132},
    {"nf4_b64", DType::NF4_B64, 64, 36},
    {"fp4_b64", DType::FP4_B64, 64, 36},
    {"q8a_g32", DType::Q8A_G32, 32, 36},
    {"q2s_g128", DType::Q2S_G128, 128, 36},
    {"f8e4m3", DType::F8E4M3, 1, 1},
    {"f8e5m2", DType::F8E5M2, 1, 1},
    {"f8e4m3_b32", DType::F8E4M3_B32, 32, 36},
    {"f8e4m3_b128", DType::F8E4M3_B128, 128, 132},
    {"trellis_v4k8_g128", DType::TRELLIS_V4K8_G128, 128, 34},
    {"trellis_v4k6_g128", DType::TRELLIS_V4K6_G128, 128, 26},
    {"trellis_v4k7_g128", DType::TRELLIS_V4K7_G128, 128, 30},
    {"trellis_v2k5_g128", DType::TRELLIS_V2K5_G128, 128, 42},
    {"trellis_v2k6_g128", DType::TRELLIS_V2K6_G128, 128, 50},
    {"trellis_v2k7_g128", DType::TRELLIS_V2K7_G128, 128, 58},
};

const TypeInfo& type_info(DType t)
{
    for (const auto& ti : kTypes)
        if (ti.t == t) return ti;
    invalid("unknown type");
}

bool is_activation(DType t) { return t == DType::F32 || t == DType::F16 || t == DType::BF16; }

int act_code(DType t)
{
    switch (t) {
    case DType::F32: return SLHIP_F32;
    case DType::F16: return SLHIP_F16;
    case DType::BF16: return SLHIP_BF16;
    default: invalid("not an activation type");
    }
}

int format_code(DType t)
{
    switch (t) {
    case DType::F32: return SLHIP_FMT_F32;
    case DType::F16: return SLHIP_FMT_F16;
    case DType::BF16: return SLHIP_FMT_BF16;
    case DType::Q8_0: return SLHIP_FMT_Q8_0;
    case DType::Q4_0: return SLHIP_FMT_Q4_0;
    case DType::Q4_1: return SLHIP_FMT_Q4_1;
    case DType::Q5_0: return SLHIP_FMT_Q5_0;
    case DType::Q5_1: return SLHIP_FMT_Q5_1;
    case DType::Q2_K: return SLHIP_FMT_Q2_K;
    case DType::Q3_K: return SLHIP_FMT_Q3_K;
    case DType::Q4_K: return SLHIP_FMT_Q4_K;
    case DType::Q5_K: return SLHIP_FMT_Q5_K;
    case DType::Q6_K: return SLHIP_FMT_Q6_K;
    case DType::IQ4_NL: return SLHIP_FMT_IQ4_NL;
    case DType::IQ4_XS: return SLHIP_FMT_IQ4_XS;
    case DType::TQ1_0: return SLHIP_FMT_TQ1_0;
    case DType::TQ2_0: return SLHIP_FMT_TQ2_0;
    case DType::MXFP4: return SLHIP_FMT_MXFP4;
    case DType::NVFP4: return SLHIP_FMT_NVFP4;
    case DType::IQ2_XXS: return SLHIP_FMT_IQ2_XXS;
    case DType::IQ2_XS: return SLHIP_FMT_IQ2_XS;
    case DType::IQ2_S: return SLHIP_FMT_IQ2_S;
    case DType::IQ3_XXS: return SLHIP_FMT_IQ3_XXS;
    case DType::IQ3_S: return SLHIP_FMT_IQ3_S;
    case DType::IQ1_S: return SLHIP_FMT_IQ1_S;
    case DType::IQ1_M: return SLHIP_FMT_IQ1_M;
    case DType::Q1_0: return SLHIP_FMT_Q1_0;
    case DType::Q2_0: return SLHIP_FMT_Q2_0;
    case DType::Q2_0_G128: return SLHIP_FMT_Q2_0_G128;
    case DType::TERN1_G128: return SLHIP_FMT_TERN1_G128;
    case DType::NVFP4_GS: return SLHIP_FMT_NVFP4_GS;
    case DType::Q4Z_G32: return SLHIP_FMT_Q4Z_G32;
    case DType::Q4Z_G128: return SLHIP_FMT_Q4Z_G128;
    case DType::Q8Z_G32: return SLHIP_FMT_Q8Z_G32;
    case DType::Q8Z_G128: return SLHIP_FMT_Q8Z_G128;
    case DType::NF4_B64: return SLHIP_FMT_NF4_B64;
    case DType::FP4_B64: return SLHIP_FMT_FP4_B64;
    case DType::Q8A_G32: return SLHIP_FMT_Q8A_G32;
    case DType::Q2S_G128: return SLHIP_FMT_Q2S_G128;
    case DType::F8E4M3: return SLHIP_FMT_F8E4M3;
    case DType::F8E5M2: return SLHIP_FMT_F8E5M2;
    case DType::F8E4M3_B32: return SLHIP_FMT_F8E4M3_B32;
    case DType::F8E4M3_B128: return SLHIP_FMT_F8E4M3_B128;
    case DType::TRELLIS_V4K8_G128: return SLHIP_FMT_TRELLIS_V4K8_G128;
    case DType::TRELLIS_V4K6_G128: return SLHIP_FMT_TRELLIS_V4K6_G128;
    case DType::TRELLIS_V4K7_G128: return SLHIP_FMT_TRELLIS_V4K7_G128;
    case DType::TRELLIS_V2K5_G128: return SLHIP_FMT_TRELLIS_V2K5_G128;
    case DType::TRELLIS_V2K6_G128: return SLHIP_FMT_TRELLIS_V2K6_G128;
    case DType::TRELLIS_V2K7_G128: return SLHIP_FMT_TRELLIS_V2K7_G128;
    default: unsupported("gather table type");
    }
}

constexpr int64_t kSymT = -1;  // the symbolic token dimension T

struct Value {
    int id = -1;
    DType type = DType::F32;
    std::vector<int64_t> dims;  // dims[k] == kSymT: the token count of the run
    bool input = false, weight = false, output = false, state = false;

    int64_t elems(int64_t T) const
    {
        int64_t n = 1;
        for (int64_t d : dims) n *= d == kSymT ? T : d;
        return n;
    }
    int64_t bytes(int64_t T) const
    {
        const TypeInfo& ti = type_info(type);
        return elems(T) / ti.block * ti.block_bytes;
    }
    int64_t last() const { return dims.empty() ? 1 : dims.back(); }
    // elements per entry of the first dimension (T counted as 1 past it)
    int64_t inner() const
    {
        int64_t n = 1;
        for (size_t k = 1; k < dims.size(); k++) n *= dims[k] == kSymT ? 1 : dims[k];
        return n;
    }
    int64_t rows(int64_t T) const { return last() == 0 ? 0 : elems(T) / last(); }
    bool symbolic() const
    {
        for (int64_t d : dims)
            if (d == kSymT) return true;
        return false;
    }
};

struct Node {
    std::string op;
    std::vector<int> in, out;
    std::map<std::string, std::string> attr;

    float f(const char* k, float d) const
    {
        auto it = attr.find(k);
        return it == attr.end() ? d : strtof(it->second.c_str(), nullptr);
    }
    long long i(const char* k, long long d) const
    {
        auto it = attr.find(k);
        return it == attr.end() ? d : strtoll(it->second.c_str(), nullptr, 10);
    }
    std::string s(const char* k, const std::string& d) const
    {
        auto it = attr.find(k);
        return it == attr.end() ? d : it->second;
    }
};

struct Graph {
    std::map<int, Value> values;
    std::vector<Node> nodes;
    // Compile options (`option key=value` lines): reduced_precision (CompileOptions.AllowReducedPrecision,
    // src/Sharplight.Core/Runtime/CompileOptions.cs:23) and int_dot, the rule that picks the integer-dot matvec
    // (see IntDotPolicy).
    std::map<std::string, std::string> options;

    Value& value(int id)
    {
        auto it = values.find(id);
        if (it == values.end()) invalid("unknown value " + std::to_string(id));
        return it->second;
    }
    const Value& value(int id) const { return const_cast<Graph*>(this)->value(id); }
};

std::vector<int> parse_ids(const std::string& s)
{
    std::vector<int> ids;
    if (s == "-") return ids;
    std::stringstream ss(s);
    std::string tok;
    while (std::getline(ss, tok, ',')) {
        if (tok.empty() || tok.find_first_not_of("0123456789") != std::string::npos)
            invalid("bad value id list '" + s + "' (ids, or '-' for none)");
        ids.push_back(atoi(tok.c_str()));
    }
    return ids;
}

DType parse_type(const std::string& s)
{
    for (const auto& ti : kTypes)
        if (s == ti.name) return ti.t;
    invalid("unknown type '" + s + "'");
}

Node parse_node(std::istringstream& ls)
{
    Node n;
    std::string ins, arrow, outs;
    if (!(ls >> n.op >> ins >> arrow >> outs) || arrow != "->") invalid("node: expected '<op> <ins> -> <outs> [k=v...]'");
    n.in = parse_ids(ins);
    n.out = parse_ids(outs);
    std::string kv;
    while (ls >> kv) {
        const size_t eq = kv.find('=');
        if (eq == std::string::npos) invalid("node attribute '" + kv + "' is not key=value");
        n.attr[kv.substr(0, eq)] = kv.substr(eq + 1);
    }
    return n;
}

Graph parse(const char* text)
{
    Graph g;
    std::istringstream in(text ? text : "");
    std::string line;
    int ln = 0;
    while (std::getline(in, line)) {
        ln++;
        std::istringstream ls(line);
        std::string kw;
        if (!(ls >> kw) || kw[0] == '#') continue;
        try {
            if (kw == "value") {
                Value v;
                std::string t, d;
                if (!(ls >> v.id >> t)) invalid("value: expected '<id> <type> <dims...>'");
                v.type = parse_type(t);
                while (ls >> d) {
                    if (d == "T") {
                        v.dims.push_back(kSymT);
                        continue;
                    }
                    if (d.find_first_not_of("0123456789") != std::string::npos)
                        invalid("dimension '" + d + "' is neither a size nor the token count T (other symbols and "
                                "symbolic expressions are not supported)");
                    // sizes up to 2^40 each and 2^46 elements without T: the byte counts of every launch stay
                    // far inside int64 for any token count the segment accepts
                    if (d.size() > 13 || strtoll(d.c_str(), nullptr, 10) > (int64_t{1} << 40))
                        invalid("dimension " + d + " is above 2^40");
                    v.dims.push_back(strtoll(d.c_str(), nullptr, 10));
                }
                int64_t fixed = 1;
                for (int64_t dd : v.dims)
                    if (dd != kSymT && (__builtin_mul_overflow(fixed, dd, &fixed) || fixed > (int64_t{1} << 46)))
                        invalid("value " + std::to_string(v.id) + " has more than 2^46 elements");
                if (g.values.count(v.id)) invalid("value " + std::to_string(v.id) + " declared twice");
                g.values[v.id] = v;
            } else if (kw == "input" || kw == "weight" || kw == "output" || kw == "state") {
                int id;
                if (!(ls >> id)) invalid(kw + ": expected a value id");
                Value& v = g.value(id);
                (kw == "input" ? v.input : kw == "weight" ? v.weight : kw == "output" ? v.output : v.state) = true;
                if (v.state && v.symbolic()) invalid("state " + std::to_string(id) + " must have fixed dims");
            } else if (kw == "option") {
                std::string kv;
                while (ls >> kv) {
                    const size_t eq = kv.find('=');
                    if (eq == std::string::npos) invalid("option '" + kv + "' is not key=value");
                    const std::string k = kv.substr(0, eq), v = kv.substr(eq + 1);
                    if (k == "reduced_precision") {
                        if (v != "0" && v != "1" && v != "true" && v != "false") invalid("reduced_precision is 0 or 1");
                    } else if (k == "int_dot") {
                        if (v != "lowerer" && v != "cpu" && v != "off") invalid("int_dot is lowerer, cpu or off");
                    } else {
                        invalid("unknown option '" + k + "'");
                    }
                    g.options[k] = v;
                }
            } else if (kw == "node") {
                Node n = parse_node(ls);
                for (int id : n.in) g.value(id);
                for (int id : n.out) g.value(id);
                g.nodes.push_back(n);
            } else {
                invalid("unknown keyword '" + kw + "'");
            }
        } catch (const Error& e) {
            throw Error(e.status, "line " + std::to_string(ln) + ": " + e.what());
        }
    }
    return g;
}

// ---- op support (IComputeDevice.Supports) ----------------------------------------------------------

struct Support {
    bool ok;
    std::string reason;
};

const std::set<std::string> kActs = {"Silu", "GeluTanh", "Gelu"};

// StandardOps.BinaryNames (src/Sharplight.Core/Graph/StandardOps.cs:39-45) -> slhip_binary_op.
const std::map<std::string, int> kBinaryOps = {
    {"Add", SLHIP_BIN_ADD}, {"Sub", SLHIP_BIN_SUB}, {"Mul", SLHIP_BIN_MUL}, {"Div", SLHIP_BIN_DIV},
    {"Max", SLHIP_BIN_MAX}, {"Min", SLHIP_BIN_MIN}, {"Pow", SLHIP_BIN_POW}, {"Mod", SLHIP_BIN_MOD},
    {"PRelu", SLHIP_BIN_PRELU}, {"Equal", SLHIP_BIN_EQUAL}, {"NotEqual", SLHIP_BIN_NOT_EQUAL},
    {"Less", SLHIP_BIN_LESS}, {"LessEqual", SLHIP_BIN_LESS_EQUAL}, {"Greater", SLHIP_BIN_GREATER},
    {"GreaterEqual", SLHIP_BIN_GREATER_EQUAL}, {"And", SLHIP_BIN_AND}, {"Or", SLHIP_BIN_OR}, {"Xor", SLHIP_BIN_XOR},
    {"Atan2", SLHIP_BIN_ATAN2}};
// Commutative ops: an f32 a with a bf16/f16 b runs as op(b, a) (slhip_binary takes b as a's type or f32).
const std::set<int> kCommutative = {SLHIP_BIN_ADD, SLHIP_BIN_MUL, SLHIP_BIN_MAX, SLHIP_BIN_MIN, SLHIP_BIN_EQUAL,
                                    SLHIP_BIN_NOT_EQUAL, SLHIP_BIN_AND, SLHIP_BIN_OR, SLHIP_BIN_XOR};

// StandardOps.UnaryNames (StandardOps.cs:25-33), Scale (:48) and Clip (StandardOps.Spatial.cs:12) ->
// slhip_unary_op (the reference's UnaryKind order).
const std::map<std::string, int> kUnaryOps = {
    {"Neg", SLHIP_UN_NEG}, {"Exp", SLHIP_UN_EXP}, {"Log", SLHIP_UN_LOG}, {"Sqrt", SLHIP_UN_SQRT},
    {"Rsqrt", SLHIP_UN_RSQRT}, {"Sigmoid", SLHIP_UN_SIGMOID}, {"Silu", SLHIP_UN_SILU}, {"Gelu", SLHIP_UN_GELU},
    {"GeluTanh", SLHIP_UN_GELU_TANH}, {"Tanh", SLHIP_UN_TANH}, {"Softplus", SLHIP_UN_SOFTPLUS},
    {"Relu", SLHIP_UN_RELU}, {"Abs", SLHIP_UN_ABS}, {"Square", SLHIP_UN_SQUARE}, {"Recip", SLHIP_UN_RECIP},
    {"Scale", SLHIP_UN_SCALE}, {"Erf", SLHIP_UN_ERF}, {"HardSwish", SLHIP_UN_HARD_SWISH},
    {"HardSigmoid", SLHIP_UN_HARD_SIGMOID}, {"Clip", SLHIP_UN_CLIP}, {"Sin", SLHIP_UN_SIN}, {"Cos", SLHIP_UN_COS},
    {"Tan", SLHIP_UN_TAN}, {"Asin", SLHIP_UN_ASIN}, {"Acos", SLHIP_UN_ACOS}, {"Atan", SLHIP_UN_ATAN},
    {"Sinh", SLHIP_UN_SINH}, {"Cosh", SLHIP_UN_COSH}, {"Asinh", SLHIP_UN_ASINH}, {"Acosh", SLHIP_UN_ACOSH},
    {"Atanh", SLHIP_UN_ATANH}, {"Floor", SLHIP_UN_FLOOR}, {"Ceil", SLHIP_UN_CEIL}, {"Round", SLHIP_UN_ROUND},
    {"Sign", SLHIP_UN_SIGN}, {"Softsign", SLHIP_UN_SOFTSIGN}, {"Mish", SLHIP_UN_MISH}, {"Elu", SLHIP_UN_ELU},
    {"Celu", SLHIP_UN_CELU}, {"Selu", SLHIP_UN_SELU}, {"LeakyRelu", SLHIP_UN_LEAKY_RELU},
    {"ThresholdedRelu", SLHIP_UN_THRESHOLDED_RELU}, {"Not", SLHIP_UN_NOT}, {"IsNaN", SLHIP_UN_IS_NAN},
    {"IsInf", SLHIP_UN_IS_INF}};

// numpy broadcasting of two dim lists (the symbolic T broadcasts against T or 1 only); false if they clash.
bool broadcast_dims(const std::vector<int64_t>& a, const std::vector<int64_t>& b, std::vector<int64_t>& out)
{
    const size_t r = std::max(a.size(), b.size());
    out.assign(r, 1);
    for (size_t k = 0; k < r; k++) {
        const int64_t da = k < r - a.size() ? 1 : a[k - (r - a.size())];
        const int64_t db = k < r - b.size() ? 1 : b[k - (r - b.size())];
        if (da == db) out[k] = da;
        else if (da == 1) out[k] = db;
        else if (db == 1) out[k] = da;
        else return false;
    }
    return true;
}

// The two UnaryOp parameters of a node (CpuCompiledSegment.LowerElementwise.cs:31-50).
std::pair<float, float> unary_params(int code, const Node& n)
{
    const float inf = INFINITY;
    switch (code) {
    case SLHIP_UN_SCALE: return {n.f("scale", 1.f), n.f("bias", 0.f)};
    case SLHIP_UN_HARD_SIGMOID: return {n.f("alpha", 0.2f), n.f("beta", 0.5f)};
    case SLHIP_UN_ELU:
    case SLHIP_UN_CELU:
    case SLHIP_UN_THRESHOLDED_RELU: return {n.f("alpha", 1.f), 0.f};
    case SLHIP_UN_SELU: return {n.f("alpha", 1.67326319217681884765625f), n.f("gamma", 1.05070102214813232421875f)};
    case SLHIP_UN_LEAKY_RELU: return {n.f("alpha", 0.01f), 0.f};
    case SLHIP_UN_CLIP: return {n.f("min", -inf), n.f("max", inf)};
    default: return {1.f, 0.f};
    }
}

// Rope's `sections` attribute: empty, or four comma-separated non-negative integers.
bool parse_sections(const std::string& text, std::vector<int>& sec)
{
    sec.assign(4, 0);
    if (text.empty()) return true;
    std::stringstream ss(text);
    std::string tok;
    int k = 0;
    while (std::getline(ss, tok, ',')) {
        if (k == 4 || tok.empty() || tok.find_first_not_of("0123456789") != std::string::npos) return false;
        sec[k++] = atoi(tok.c_str());
    }
    return k == 4;
}

bool flag(const Node& n, const char* key)
{
    const std::string v = n.s(key, "false");
    return v == "true" || v == "True" || v == "1";
}

}  // namespace
int ew_program_prepare(const slhip_ew_program* prog, int64_t cols);  // ewgroup.hip
bool matvec_q8_fits(int fmt, int64_t K, bool dual);  // matvec_i8.hip
namespace {

// When a MatMul quantizes its activations to q8 and takes the integer-dot matvec, and for which activation
// row counts. The node may not when it carries f32_activations, unless the compile allows reduced precision
// (QuantizedActivationsAllowed, src/Sharplight.Shaders/Lowering/GraphLowerer.IntDot.cs:61-62;
// CpuCompiledSegment.LowerLinear.cs:39). Rules (option int_dot):
//   lowerer (default) -- the Vulkan lowerer's UseIntDotMatvec (GraphLowerer.IntDot.cs:52-55,68-75; IntDotMaxRows
//     :18-19; IntDotFirstRow, GraphLowerer.RowInvariance.cs:21-25): Q8_0 from 2 to 16 rows, Q4_K/Q5_K/Q6_K (K a
//     multiple of 256) and the 32-value block formats Q4_0/Q5_0/IQ4_NL/MXFP4 (SHARPLIGHT_MMVQ_BLOCK, on by
//     default) from 1 to 8 rows;
//   cpu -- the CPU provider's MatMulOp (MatMulOp.cs:104,138-147): every IntDot.Supports format (IntDot.cs:36-38)
//     below IntDotGemmMinRows (32) rows;
//   off -- never (a device without DeviceFeatures.IntDot).
struct IntDotRange {
    int64_t lo = 0, hi = -1;  // rows lo..hi take the integer-dot matvec; empty when hi < lo
    bool any() const { return hi >= lo; }
    bool covers(int64_t r) const { return r >= lo && r <= hi; }
};

IntDotRange int_dot_range(const Graph& g, const Node& mm, DType w, int64_t K)
{
    IntDotRange r;
    auto opt = [&](const char* k, const char* d) {
        auto it = g.options.find(k);
        return it == g.options.end() ? std::string(d) : it->second;
    };
    const std::string policy = opt("int_dot", "lowerer");
    const std::string rp = opt("reduced_precision", "0");
    const bool reduced = rp == "1" || rp == "true";
    if (policy == "off" || (!reduced && flag(mm, "f32_activations"))) return r;
    const bool candidate = w == DType::Q8_0 || w == DType::Q4_0 || w == DType::Q4_1 || w == DType::Q5_0 ||
                           w == DType::Q5_1 || w == DType::Q4_K || w == DType::Q5_K || w == DType::Q6_K ||
                           w == DType::IQ4_NL || w == DType::IQ4_XS || w == DType::MXFP4;
    if (!candidate) return r;
    const int fmt = format_code(w);
    if (!matvec_q8_fits(fmt, K, false)) return r;
    const bool kq = w == DType::Q4_K || w == DType::Q5_K || w == DType::Q6_K;
    if (policy == "cpu") {
        r.lo = 1;
        r.hi = 31;
        return r;
    }
    if (w == DType::Q8_0) {
        r.lo = 2;
        r.hi = 16;
    } else if ((kq && K % 256 == 0) || w == DType::Q4_0 || w == DType::Q5_0 || w == DType::IQ4_NL || w == DType::MXFP4) {
        r.lo = 1;
        r.hi = 8;
    }
    return r;
}

// Weight formats the f32-activation matvec reads (slhip_matvec); the others run on the integer-dot path only.
bool float_matvec_format(DType t)
{
    return t == DType::F32 || t == DType::F16 || t == DType::BF16 || t == DType::Q8_0 || t == DType::Q4_0 ||
           t == DType::Q4_1 || t == DType::Q5_0 || t == DType::Q5_1 || t == DType::Q2_K || t == DType::Q3_K ||
           t == DType::Q4_K || t == DType::Q5_K || t == DType::Q6_K;
}

Support supports(const Graph& g, const Node& n)
{
    auto no = [](const std::string& r) { return Support{false, r}; };
    auto act = [&](int id) { return is_activation(g.value(id).type); };
    const std::string& op = n.op;
    if (kBinaryOps.count(op)) {
        if (n.in.size() != 2 || n.out.size() != 1) return no(op + " takes two inputs");
        if (!act(n.in[0]) || !act(n.in[1]) || !act(n.out[0])) return no(op + ": f32, f16 or bf16 operands");
        const DType ta = g.value(n.in[0]).type, tb = g.value(n.in[1]).type;
        const bool swap = ta == DType::F32 && tb != DType::F32 && kCommutative.count(kBinaryOps.at(op));
        if (tb != ta && tb != DType::F32 && !swap) return no(op + ": b must have a's type or be f32");
        std::vector<int64_t> bd;
        if (!broadcast_dims(g.value(n.in[0]).dims, g.value(n.in[1]).dims, bd)) return no(op + ": shapes do not broadcast");
        if (bd != g.value(n.out[0]).dims) return no(op + ": output shape is not the broadcast shape");
        if (bd.size() > 8) return no(op + ": rank above 8");
        return {true, ""};
    }
    if (kUnaryOps.count(op)) {
        if (n.in.size() != 1 || n.out.size() != 1 || !act(n.in[0]) || !act(n.out[0])) return no(op + " takes one activation");
        if (g.value(n.in[0]).dims != g.value(n.out[0]).dims) return no(op + ": output shape differs from the input's");
        return {true, ""};
    }
    if (op == "RmsNorm" || op == "L2Norm" || op == "LayerNorm") {
        const size_t maxin = op == "LayerNorm" ? 3 : op == "RmsNorm" ? 2 : 1;
        if (n.in.empty() || n.in.size() > maxin || n.out.size() != 1) return no(op + ": wrong operand count");
        const Value& x = g.value(n.in[0]);
        if (!act(n.in[0]) || x.type == DType::F16) return no(op + ": f32 or bf16 rows");
        for (size_t k = 1; k < n.in.size(); k++) {
            const Value& w = g.value(n.in[k]);
            if (w.type != DType::F32 || w.dims.size() != 1 || w.dims[0] != x.last())
                return no(op + ": weights must be f32 [D]");  // the reference's fused norms require f32 weights
        }
        return {true, ""};
    }
    if (op == "Rope") {
        if (n.in.size() < 2 || n.in.size() > 3 || n.out.size() != 1) return no("Rope takes x, positions[, freq factors]");
        const Value& x = g.value(n.in[0]);
        const Value& p = g.value(n.in[1]);
        if (x.dims.size() != 3 || !act(n.in[0]) || x.type == DType::F16) return no("Rope: x must be f32/bf16 [T, H, D]");
        if (p.type != DType::I32 || p.dims.empty() || p.dims[0] != x.dims[0]) return no("Rope: positions must be i32 [T]");
        if (p.dims.size() > 2 || (p.dims.size() == 2 && (p.dims[1] < 1 || p.dims[1] > 4)))
            return no("Rope: positions must be i32 [T] or [T, A] with A <= 4 axes");
        std::vector<int> sec;
        if (!parse_sections(n.s("sections", ""), sec)) return no("Rope: sections must be four non-negative integers");
        if (n.in.size() == 3 && g.value(n.in[2]).type != DType::F32) return no("Rope: frequency factors must be f32");
        return {true, ""};
    }
    if (op == "Gather") {
        if (n.in.size() != 2 || n.out.size() != 1) return no("Gather takes table, indices");
        const Value& t = g.value(n.in[0]);
        if (t.type == DType::I32) return no("Gather: integer tables are not supported");
        if (g.value(n.in[1]).type != DType::I32) return no("Gather: indices must be i32");
        const DType o = g.value(n.out[0]).type;
        if (o != DType::F32 && o != DType::BF16) return no("Gather: f32 or bf16 output");
        return {true, ""};
    }
    if (op == "CacheWrite") {
        // StandardOps.CacheWrite (src/Sharplight.Core/Graph/StandardOps.cs:310-319): state, x [, sequence rows
        // [T, 4] (multi-sequence form) [, block table (paged form)]]; no outputs.
        if (n.in.size() < 2 || n.in.size() > 4 || !n.out.empty()) return no("CacheWrite takes state, x[, rows[, pages]]");
        const Value& st = g.value(n.in[0]);
        const Value& x = g.value(n.in[1]);
        if (!st.state) return no("CacheWrite: the first input must be a state");
        if (!is_activation(st.type)) return no("CacheWrite: f32, f16 or bf16 caches (quantized caches are not supported)");
        if (x.type != DType::F32 && x.type != DType::BF16) return no("CacheWrite: f32 or bf16 rows");
        if (n.i("compression", 1) != 1) return no("CacheWrite: compressed caches are not supported");
        if (st.dims.size() < 2 || x.dims.empty() || st.inner() != x.inner())
            return no("CacheWrite: x rows must match the cache rows");
        for (size_t k = 2; k < n.in.size(); k++)
            if (g.value(n.in[k]).type != DType::I32) return no("CacheWrite: sequence rows and block table are i32");
        return {true, ""};
    }
    if (op == "Cast") {
        if (n.in.size() != 1 || n.out.size() != 1 || !act(n.in[0]) || !act(n.out[0])) return no("Cast: activation types");
        return {true, ""};
    }
    if (op == "MatMul") {
        // StandardOps.MatMul (src/Sharplight.Core/Graph/StandardOps.cs:143-162): y = x . W^T, W a weight [N, K];
        // run here as the decode matvec (few activation rows).
        if (n.in.size() != 2 || n.out.size() != 1) return no("MatMul takes x, weight");
        const Value& x = g.value(n.in[0]);
        const Value& w = g.value(n.in[1]);
        const Value& y = g.value(n.out[0]);
        if (x.type != DType::F32 && x.type != DType::BF16) return no("MatMul: f32 or bf16 activations");
        if (y.type != DType::F32 && y.type != DType::BF16) return no("MatMul: f32 or bf16 output");
        if (!w.weight || w.dims.size() != 2) return no("MatMul: the second operand must be a weight [N, K]");
        if (x.dims.empty() || w.dims[1] != x.last()) return no("MatMul: K mismatch");
        if (y.last() != w.dims[0]) return no("MatMul: output must be [.., N]");
        const int64_t K = x.last();
        const bool dense = w.type == DType::F32 || w.type == DType::F16 || w.type == DType::BF16;
        const IntDotRange id = int_dot_range(g, n, w.type, K);
        if (float_matvec_format(w.type)) {
            if (dense && (K % 8 != 0 || K > 16384)) return no("MatMul: K must be a multiple of 8 and at most 16384");
            if (!dense && (K % 256 != 0 || K > 16384)) return no("MatMul: block-format K must be a multiple of 256, at most 16384");
            if (!matvec_fits(format_code(w.type), K, false))
                return no("MatMul: the weight rows do not fit the matvec's staging");
            return {true, ""};
        }
        // no f32 matvec for the format: the integer-dot path must serve every row count from one (compile
        // refuses a token bound whose row count passes the range's end)
        if (id.any() && id.lo == 1) return {true, ""};
        return no("MatMul: f32, f16, bf16, Q8_0/Q4_0/Q4_1/Q5_0/Q5_1 or Q2_K..Q6_K weights (IQ4_NL, IQ4_XS and MXFP4 "
                  "only with quantized activations, the integer-dot matvec) on this provider");
    }
    return no("op " + op + " is not on the fused-layer-op path of the HIP provider");
}

// ---- lowering into fused units -------------------------------------------------------------------------

struct Unit {
    enum Kind { RowNorm, Gated, Rope, Gather, Cast, CacheWrite, Matvec, Binary, Unary, QuantizeQ8, EwGroup } kind;
    std::string label;
    // RowNorm
    int norm = SLHIP_NORM_RMS;
    int x = -1, res = -1, w = -1, b = -1, y = -1, h = -1;
    int y16 = -1;         // f16 copy of y (an absorbed Cast), or -1
    bool skip_y = false;  // y itself is read by nothing else: only the copy is written
    float eps = 0.f;
    // Gated
    int act = SLHIP_ACT_SILU, gate = -1, up = -1;
    // Matvec: x . Wg^T (+ bias), or act(x . Wg^T) * (x . Wu^T) when wu >= 0
    int wg = -1, wu = -1;
    int mm_node = -1;   // the (gate) MatMul node
    int bias = -1;      // an absorbed Add of a constant f32 row vector [N] (FoldMatMulBiases)
    IntDotRange q8;     // Matvec / QuantizeQ8: the activation rows that take the integer-dot path
    int q8buf = -1;     // the quantized copy of x (scratch buffer index) the integer-dot path reads
    // Rope: up to 4 tensors sharing positions and settings
    struct RopeTensor {
        int x, y, w;
        int cache_node = -1;  // the CacheWrite this tensor's rows go through (y is its state)
    };
    std::vector<RopeTensor> rt;
    int pos = -1, ff = -1;
    slhip_rope_cfg cfg{};
    // Gather
    int table = -1, ids = -1;
    // CacheWrite (standalone): x into the state y
    int cache_node = -1;
    // Binary: y = op(x, up) with broadcasting; Unary: y = op(x) with parameters p0, p1
    int op = 0;
    float p0 = 0.f, p1 = 0.f;
    // EwGroup: the program of a fused elementwise group (value ids in place of the device pointers), the value
    // whose shape is the group's, and the folded norms (node indices, -1 for none)
    std::vector<int> ew_in, ew_mode;
    std::vector<slhip_ew_op> ew_ops;
    std::vector<std::pair<int, int>> ew_out;  // (value, register)
    int shape_of = -1, head_node = -1, tail_node = -1, norm_reg = -1;
};

class Segment {
public:
    // plan_only: lower the nodes into launches and stop (no stream, no device memory).
    Segment(Graph g, int64_t max_tokens, bool plan_only = false) : g_(std::move(g)), max_t_(max_tokens)
    {
        if (max_t_ < 0) invalid("MaxTokens must not be negative");
        if (max_t_ > (int64_t{1} << 20)) invalid("MaxTokens above 2^20 is not supported");
        for (const Node& n : g_.nodes) {
            Support s = supports(g_, n);
            if (!s.ok) unsupported(s.reason);
        }
        lower();
        assign_q8();
        if (plan_only) return;
        check(slhip_stream_create(&stream_));
        allocate();
        prepare_groups();
        reset_state();
    }

    ~Segment()
    {
        for (auto& kv : mem_) slhip_free(kv.second);
        for (void* p : scratch_) slhip_free(p);
        if (stream_) slhip_stream_destroy(stream_);
    }

    void set_input(int id, const void* data, size_t bytes)
    {
        Value& v = g_.value(id);
        if (!v.input && !v.weight) invalid("value " + std::to_string(id) + " is not an input or weight of the segment");
        const int64_t cap = v.bytes(max_t_);
        if (static_cast<int64_t>(bytes) > cap) invalid("input " + std::to_string(id) + ": " + std::to_string(bytes) +
                                                       " bytes exceed the compiled size " + std::to_string(cap));
        if (bytes && !data) invalid("input data is null");
        check(slhip_memcpy_h2d(mem_.at(id), data, bytes, stream_));
        check(slhip_stream_sync(stream_));
    }

    void execute(int64_t T)
    {
        if (T < 0) invalid("T must not be negative");
        if (T > max_t_)  // CpuCompiledSegment.Execute (src/Sharplight.Cpu/CpuCompiledSegment.cs:115-121)
            throw Error(SLHIP_ERR_INVALID, "Symbol 'T' = " + std::to_string(T) + " exceeds the compiled bound " +
                                               std::to_string(max_t_) + ".");
        t_ = T;
        for (const Unit& u : units_) run(u, T);
    }

    // Runtime scalars (RunParameters.Scalars, src/Sharplight.Core/Runtime/RunParameters.cs:12), e.g. n_past.
    void set_scalar(const std::string& name, int64_t value) { scalars_[name] = value; }

    // ICompiledSegment.ResetState: states (KV caches) back to zero, as CpuCompiledSegment.ResetState clears
    // them (src/Sharplight.Cpu/CpuCompiledSegment.cs:259-265).
    void reset_state()
    {
        for (auto& kv : g_.values)
            if (kv.second.state) check(slhip_memset(mem_.at(kv.first), 0, static_cast<size_t>(kv.second.bytes(0)), stream_));
        check(slhip_stream_sync(stream_));
    }

    void get_output(int id, void* data, size_t bytes)
    {
        const Value& v = g_.value(id);
        if (!v.output && !v.state) invalid("value " + std::to_string(id) + " is neither an output nor a state of the segment");
        const int64_t n = v.bytes(t_);
        if (static_cast<int64_t>(bytes) != n)
            invalid("output " + std::to_string(id) + " holds " + std::to_string(n) + " bytes, destination " + std::to_string(bytes));
        check(slhip_stream_sync(stream_));  // raises a pending gather index error
        if (n) check(slhip_memcpy_d2h(data, mem_.at(id), bytes, stream_));
        check(slhip_stream_sync(stream_));
    }

    int64_t device_bytes() const { return device_bytes_; }

    std::string launches() const
    {
        std::string s;
        for (const Unit& u : units_) s += u.label + "\n";
        return s;
    }

    // The launches a run of T tokens makes: the units whose row-count condition holds, each matvec with the
    // path it takes at that count.
    std::string launches_at(int64_t T) const
    {
        std::string s;
        for (const Unit& u : units_) {
            if (u.kind == Unit::QuantizeQ8 || u.kind == Unit::Matvec) {
                const int64_t rows = g_.value(u.x).rows(T);
                if (rows == 0) continue;
                if (u.kind == Unit::QuantizeQ8) {
                    if (u.q8.covers(rows)) s += "x->q8\n";
                    continue;
                }
                std::string l = u.label.substr(0, u.label.find(" (int-dot"));
                s += l + (u.q8.covers(rows) ? " int-dot\n" : " f32\n");
                continue;
            }
            s += u.label + "\n";
        }
        return s;
    }

private:
    Graph g_;
    int64_t max_t_, t_ = 0;
    std::vector<Unit> units_;
    std::map<int, void*> mem_;
    std::vector<int64_t> scratch_bytes_;  // the quantized activation copies (assign_q8)
    std::vector<void*> scratch_;
    std::map<std::string, int64_t> scalars_;
    int64_t device_bytes_ = 0;
    slhip_stream stream_ = nullptr;

    std::map<int, std::vector<int>> consumers() const
    {
        std::map<int, std::vector<int>> c;
        for (size_t k = 0; k < g_.nodes.size(); k++)
            for (int id : g_.nodes[k].in) c[id].push_back(static_cast<int>(k));
        return c;
    }

    static int norm_kind(const std::string& op)
    {
        return op == "RmsNorm" ? SLHIP_NORM_RMS : op == "L2Norm" ? SLHIP_NORM_L2 : SLHIP_NORM_LAYER;
    }

    Unit rownorm_unit(const Node& n)
    {
        Unit u{Unit::RowNorm};
        u.norm = norm_kind(n.op);
        u.x = n.in[0];
        u.w = n.in.size() > 1 ? n.in[1] : -1;
        u.b = n.in.size() > 2 ? n.in[2] : -1;
        u.y = n.out[0];
        u.eps = n.f("eps", n.op == "LayerNorm" ? 1e-5f : 1e-6f);
        u.label = n.op;
        return u;
    }

    void lower()
    {
        auto cons = consumers();
        const size_t N = g_.nodes.size();
        std::vector<bool> done(N, false);
        auto single_use = [&](int id) { return !g_.value(id).output && cons[id].size() == 1; };
        find_dual_matvecs(cons, single_use);
        form_groups(cons);
        for (size_t k = 0; k < N; k++) {
            if (done[k]) continue;
            const Node& n = g_.nodes[k];
            if (group_of_[k] >= 0) {  // a fused group, emitted at its last node
                done[k] = true;
                const EwGroup& G = groups_[group_of_[k]];
                if (static_cast<int>(k) == G.nodes.back()) emit_group(G, cons, done);
                continue;
            }
            if (folded_norms_.count(static_cast<int>(k))) {
                done[k] = true;
                continue;
            }
            if (n.op == "Add" && k + 1 < N && !done[k + 1] && !folded_norms_.count(static_cast<int>(k) + 1)) {
                const Node& m = g_.nodes[k + 1];
                const auto& od = g_.value(n.out[0]).dims;
                if ((m.op == "RmsNorm" || m.op == "L2Norm") && m.in[0] == n.out[0] && g_.value(n.in[0]).dims == od &&
                    g_.value(n.in[1]).dims == od) {
                    Unit u = rownorm_unit(m);
                    u.x = n.in[0];
                    u.res = n.in[1];
                    // the sum is written only when something besides the norm reads it
                    u.h = single_use(n.out[0]) ? -1 : n.out[0];
                    u.label = std::string("fused[Add]+") + m.op;
                    if (g_.value(n.in[0]).type != g_.value(n.out[0]).type ||
                        g_.value(n.in[1]).type != g_.value(n.out[0]).type)
                        unsupported("Add+" + m.op + ": the residual stream must keep one type");
                    done[k] = done[k + 1] = true;
                    attach_half_copy(u, cons, done);
                    units_.push_back(u);
                    continue;
                }
            }
            auto dual = dual_at_.find(static_cast<int>(k));
            if (dual != dual_at_.end()) {  // the Mul closing act(x Wg^T) * (x Wu^T): one dual matvec launch
                const DualPattern& d = dual->second;
                Unit u{Unit::Matvec};
                u.x = g_.nodes[d.mm_gate].in[0];
                u.wg = g_.nodes[d.mm_gate].in[1];
                u.wu = g_.nodes[d.mm_up].in[1];
                u.act = d.act;
                u.y = n.out[0];
                u.mm_node = d.mm_gate;
                u.label = "matvec2+fused[" + g_.nodes[d.act_node].op + ",Mul]";
                units_.push_back(u);
                done[k] = true;
                continue;
            }
            if (absorbed_.count(static_cast<int>(k))) {  // a MatMul or activation of a dual matvec
                done[k] = true;
                continue;
            }
            if (kActs.count(n.op) && single_use(n.out[0])) {
                const int mk = cons[n.out[0]][0];
                const Node& m = g_.nodes[mk];
                const int up = m.in.size() == 2 ? (m.in[0] == n.out[0] ? m.in[1] : m.in[0]) : -1;
                // The unit is emitted here, at the activation, so `up` must already exist: made by an earlier
                // node (or an input). Same shapes only: a broadcast Mul runs as its own launch.
                const bool ready = up >= 0 && producer_before(up, static_cast<int>(k));
                if (m.op == "Mul" && !done[mk] && ready && g_.value(up).dims == g_.value(n.in[0]).dims &&
                    g_.value(m.out[0]).dims == g_.value(n.in[0]).dims) {
                    Unit u{Unit::Gated};
                    u.act = n.op == "Silu" ? SLHIP_ACT_SILU : n.op == "GeluTanh" ? SLHIP_ACT_GELU_TANH : SLHIP_ACT_GELU_ERF;
                    u.gate = n.in[0];
                    u.up = m.in[0] == n.out[0] ? m.in[1] : m.in[0];
                    u.y = m.out[0];
                    if (g_.value(u.gate).type != g_.value(u.up).type) unsupported("gated activation: gate and up types differ");
                    u.label = "fused[" + n.op + ",Mul]";
                    units_.push_back(u);
                    done[k] = done[mk] = true;
                    continue;
                }
            }
            if (n.op == "RmsNorm" && n.in.size() == 2 && single_use(n.out[0])) {
                const int rk = cons[n.out[0]][0];
                const Node& r = g_.nodes[rk];
                if (r.op == "Rope" && r.in[0] == n.out[0] && !done[rk] && rk > static_cast<int>(k)) {
                    // computed inside the rope launch; marked here, emitted at the rope
                    absorbed_norm_[rk] = static_cast<int>(k);
                    done[k] = true;
                    continue;
                }
            }
            done[k] = true;
            if (n.op == "RmsNorm" || n.op == "L2Norm" || n.op == "LayerNorm") {
                Unit u = rownorm_unit(n);
                attach_half_copy(u, cons, done);
                units_.push_back(u);
            } else if (n.op == "Rope") {
                Unit u = rope_unit(static_cast<int>(k));
                // A rope whose only consumer is a cache write stores into the cache
                // (GraphLowerer.Fusion.cs:633-648; f32/f16/bf16 caches, no compression).
                if (single_use(n.out[0])) {
                    const int mk = cons[n.out[0]][0];
                    const Node& m = g_.nodes[mk];
                    const Value& st = m.op == "CacheWrite" ? g_.value(m.in[0]) : g_.value(n.out[0]);
                    const Value& rv = g_.value(n.out[0]);
                    if (m.op == "CacheWrite" && !done[mk] && m.in[1] == n.out[0] && st.dims.size() == 3 &&
                        rv.dims.size() == 3 && st.dims[1] == rv.dims[1] && st.dims[2] == rv.dims[2]) {
                        u.rt[0].y = m.in[0];
                        u.rt[0].cache_node = mk;
                        u.label += "+cache";
                        done[mk] = true;
                    }
                }
                units_.push_back(u);
            } else if (n.op == "Gather") {
                Unit u{Unit::Gather};
                u.table = n.in[0];
                u.ids = n.in[1];
                u.y = n.out[0];
                const Value& t = g_.value(u.table);
                if (t.dims.size() < 2) invalid("Gather: table must be [V, ...]");
                u.label = "Gather";
                units_.push_back(u);
            } else if (n.op == "Cast") {
                Unit u{Unit::Cast};
                u.x = n.in[0];
                u.y = n.out[0];
                u.label = "Cast";
                units_.push_back(u);
            } else if (n.op == "MatMul") {
                Unit u{Unit::Matvec};
                u.x = n.in[0];
                u.wg = n.in[1];
                u.y = n.out[0];
                u.mm_node = static_cast<int>(k);
                u.label = "matvec";
                fold_bias(u, cons, done, single_use);
                units_.push_back(u);
            } else if (n.op == "CacheWrite") {
                Unit u{Unit::CacheWrite};
                u.x = n.in[1];
                u.y = n.in[0];
                u.cache_node = static_cast<int>(k);
                u.label = "CacheWrite";
                units_.push_back(u);
            } else if (kBinaryOps.count(n.op) || kUnaryOps.count(n.op)) {
                units_.push_back(elementwise_unit(static_cast<int>(k)));
            } else {
                unsupported("op " + n.op + " has no lowering on the HIP provider");
            }
        }
        merge_ropes();
    }

    std::map<int, int> absorbed_norm_;  // rope node -> RmsNorm node computed inside it

    // Whether value `id` is a segment input/weight/state or is produced by a node before node k.
    bool producer_before(int id, int k) const
    {
        for (int j = 0; j < static_cast<int>(g_.nodes.size()); j++)
            for (int o : g_.nodes[j].out)
                if (o == id) return j < k;
        return true;
    }

    std::vector<int64_t> dims_at(int id, int64_t T) const
    {
        std::vector<int64_t> d = g_.value(id).dims;
        for (auto& x : d)
            if (x == kSymT) x = T;
        return d;
    }

    // BinaryOp.Align (src/Sharplight.Cpu/BinaryOp.cs:37-58) for a dense operand: its strides against y's rank,
    // 0 along a dim it lacks or holds once.
    static std::vector<int64_t> align(const std::vector<int64_t>& d, size_t rank)
    {
        std::vector<int64_t> s(rank, 0);
        int64_t acc = 1;
        for (size_t i = d.size(); i-- > 0;) {
            const size_t k = i + (rank - d.size());
            s[k] = d[i] == 1 ? 0 : acc;
            acc *= d[i];
        }
        return s;
    }

    // ---- fused elementwise groups (GraphLowerer.Fusion.cs:88-285) -------------------------------------------

    struct EwGroup {
        std::vector<int> nodes;
        int head = -1, tail = -1;  // folded row norms
        bool dead = false;
    };
    std::vector<EwGroup> groups_;
    std::vector<int> group_of_;    // node -> its group, or -1
    std::set<int> folded_norms_;   // norm nodes folded into a group

    // How an input of dims `in` feeds an output of dims `out` in a group program, or -1 when no mode fits.
    static int input_mode(const std::vector<int64_t>& in, const std::vector<int64_t>& out)
    {
        const size_t r = out.size();
        if (in.size() > r) return -1;
        std::vector<int64_t> a(r - in.size(), 1);
        a.insert(a.end(), in.begin(), in.end());
        if (a == out) return SLHIP_EWI_FULL;
        bool lead_one = true, lead_same = true;
        for (size_t k = 0; k + 1 < r; k++) {
            lead_one = lead_one && a[k] == 1;
            lead_same = lead_same && a[k] == out[k];
        }
        if (lead_one && a[r - 1] == 1) return SLHIP_EWI_SCALAR;
        if (lead_one && a[r - 1] == out[r - 1]) return SLHIP_EWI_ROW;
        if (lead_same && a[r - 1] == 1) return SLHIP_EWI_COL;
        return -1;
    }

    // IsFusable (GraphLowerer.Fusion.cs:9-11): an elementwise op with an f32 output and activation inputs; here also
    // inputs whose broadcast the group program can express and rows of a multiple of 4 values.
    bool fusable(int k) const
    {
        const Node& n = g_.nodes[k];
        if (absorbed_.count(k) || dual_at_.count(k)) return false;
        if (!kBinaryOps.count(n.op) && !kUnaryOps.count(n.op)) return false;
        if (n.out.size() != 1) return false;
        const Value& y = g_.value(n.out[0]);
        if (y.type != DType::F32 || y.dims.empty() || y.dims.back() == kSymT || y.dims.back() % 4 != 0) return false;
        for (int id : n.in) {
            const Value& v = g_.value(id);
            if (!is_activation(v.type) || input_mode(v.dims, y.dims) < 0) return false;
        }
        return true;
    }

    int ext_inputs(const std::vector<int>& nodes) const
    {
        std::set<int> produced, ext;
        for (int k : nodes) produced.insert(g_.nodes[k].out[0]);
        for (int k : nodes)
            for (int id : g_.nodes[k].in)
                if (!produced.count(id)) ext.insert(id);
        return static_cast<int>(ext.size());
    }

    static bool norm_weight_fusable(const Graph& g, const Node& norm)
    {
        return norm.in.size() <= 1 || (g.value(norm.in[1]).type == DType::F32 && g.value(norm.in[1]).dims.size() == 1);
    }

    // The values of group `G` that the launch stores: read by a node outside the unit, or segment outputs.
    std::vector<int> group_outputs(const EwGroup& G, std::map<int, std::vector<int>>& cons) const
    {
        std::set<int> in(G.nodes.begin(), G.nodes.end());
        std::vector<int> outs;
        for (int k : G.nodes) {
            const int v = g_.nodes[k].out[0];
            bool esc = g_.value(v).output;
            for (int c : cons[v]) esc = esc || (!in.count(c) && c != G.tail);
            if (esc) outs.push_back(v);
        }
        return outs;
    }

    // GroupElementwiseChains, MergeElementwiseGroups, FoldNormTails and FoldNormHeads (GraphLowerer.Fusion.cs:
    // 88-284) over the nodes not taken by a dual matvec.
    void form_groups(std::map<int, std::vector<int>>& cons)
    {
        const int N = static_cast<int>(g_.nodes.size());
        constexpr int kMaxIn = SLHIP_EW_MAX_INPUTS - 1;  // a register kept for a norm head's input
        struct URef {
            int group, node;
        };
        std::vector<URef> us;
        int open = -1;
        std::set<int> open_vals;
        auto dims_of = [&](const EwGroup& G) { return g_.value(g_.nodes[G.nodes[0]].out[0]).dims; };
        for (int k = 0; k < N; k++) {
            if (fusable(k)) {
                const Node& n = g_.nodes[k];
                bool joins = false;
                if (open >= 0) {
                    EwGroup& G = groups_[open];
                    std::vector<int> with = G.nodes;
                    with.push_back(k);
                    bool reads = false;
                    for (int id : n.in) reads = reads || open_vals.count(id);
                    joins = reads && g_.value(n.out[0]).dims == dims_of(G) && ext_inputs(with) <= kMaxIn &&
                            static_cast<int>(with.size()) <= SLHIP_EW_MAX_OPS;
                }
                if (!joins) {
                    groups_.push_back(EwGroup{});
                    open = static_cast<int>(groups_.size()) - 1;
                    open_vals.clear();
                    us.push_back({open, -1});
                }
                groups_[open].nodes.push_back(k);
                open_vals.insert(n.out[0]);
                continue;
            }
            open = -1;
            us.push_back({-1, k});
        }
        // merge along data flow: a group reading an earlier group's output takes its nodes when nothing in
        // between reads those outputs or writes a state
        for (int j = 0; j < static_cast<int>(us.size()); j++) {
            if (us[j].group < 0) continue;
            for (int i = j - 1; i >= std::max(0, j - 16); i--) {
                if (us[i].group < 0) continue;
                EwGroup& E = groups_[us[i].group];
                EwGroup& L = groups_[us[j].group];
                if (dims_of(E) != dims_of(L)) continue;
                std::set<int> outs;
                for (int k : E.nodes) outs.insert(g_.nodes[k].out[0]);
                bool reads = false;
                for (int k : L.nodes)
                    for (int id : g_.nodes[k].in) reads = reads || outs.count(id);
                std::vector<int> both = E.nodes;
                both.insert(both.end(), L.nodes.begin(), L.nodes.end());
                if (!reads || ext_inputs(both) > kMaxIn || static_cast<int>(both.size()) > SLHIP_EW_MAX_OPS) continue;
                bool blocked = false;
                for (int u = i + 1; u < j && !blocked; u++) {
                    std::vector<int> un = us[u].group >= 0 ? groups_[us[u].group].nodes : std::vector<int>{us[u].node};
                    for (int k : un) {
                        const Node& n = g_.nodes[k];
                        if (n.op == "CacheWrite") blocked = true;
                        for (int id : n.in) blocked = blocked || outs.count(id);
                    }
                }
                if (blocked) continue;
                L.nodes = both;
                E.dead = true;
                us.erase(us.begin() + i);
                j--;
            }
        }
        // a row norm right after a group, of one of its values (FoldNormTails, :211-238)
        for (int i = 0; i + 1 < static_cast<int>(us.size()); i++) {
            if (us[i].group < 0 || us[i + 1].node < 0) continue;
            const Node& nm = g_.nodes[us[i + 1].node];
            if (nm.op != "RmsNorm" && nm.op != "L2Norm") continue;
            EwGroup& G = groups_[us[i].group];
            bool made = false;
            for (int k : G.nodes) made = made || g_.nodes[k].out[0] == nm.in[0];
            if (!made || g_.value(nm.in[0]).dims != dims_of(G) || !norm_weight_fusable(g_, nm)) continue;
            G.tail = us[i + 1].node;
            us.erase(us.begin() + i + 1);
        }
        // a row norm whose output only the next group reads (FoldNormHeads, :240-284)
        for (int i = 0; i + 1 < static_cast<int>(us.size()); i++) {
            if (us[i].node < 0 || us[i + 1].group < 0) continue;
            const Node& nm = g_.nodes[us[i].node];
            if (nm.op != "RmsNorm" && nm.op != "L2Norm") continue;
            EwGroup& G = groups_[us[i + 1].group];
            const int y = nm.out[0];
            if (G.tail >= 0 || G.head >= 0 || g_.value(y).output || g_.value(y).dims != dims_of(G) ||
                !norm_weight_fusable(g_, nm) || !is_activation(g_.value(y).type))
                continue;
            bool only = !cons[y].empty();
            for (int c : cons[y]) only = only && std::find(G.nodes.begin(), G.nodes.end(), c) != G.nodes.end();
            if (!only) continue;
            G.head = us[i].node;
            us.erase(us.begin() + i);
            i--;
        }
        group_of_.assign(N, -1);
        for (size_t gi = 0; gi < groups_.size(); gi++) {
            EwGroup& G = groups_[gi];
            if (G.dead) continue;
            if (group_outputs(G, cons).size() > SLHIP_EW_MAX_OUTPUTS) {  // too many stores: unfused
                G.dead = true;
                continue;
            }
            for (int k : G.nodes) group_of_[k] = static_cast<int>(gi);
            if (G.head >= 0) folded_norms_.insert(G.head);
            if (G.tail >= 0) folded_norms_.insert(G.tail);
        }
    }

    Unit elementwise_unit(int k)
    {
        const Node& n = g_.nodes[k];
        if (kBinaryOps.count(n.op)) {
            Unit u{Unit::Binary};
            u.op = kBinaryOps.at(n.op);
            if (u.op == SLHIP_BIN_MOD && flag(n, "fmod")) u.op = SLHIP_BIN_FMOD;
            u.x = n.in[0];
            u.up = n.in[1];
            if (g_.value(u.x).type == DType::F32 && g_.value(u.up).type != DType::F32) std::swap(u.x, u.up);  // commutative
            u.y = n.out[0];
            u.label = n.op;
            return u;
        }
        Unit u{Unit::Unary};
        u.op = kUnaryOps.at(n.op);
        std::tie(u.p0, u.p1) = unary_params(u.op, n);
        u.x = n.in[0];
        u.y = n.out[0];
        u.label = n.op;
        return u;
    }

    // A group whose program does not fit: its head norm, its nodes and its tail norm as their own launches.
    void emit_unfused(const EwGroup& G, std::map<int, std::vector<int>>& cons, std::vector<bool>& done)
    {
        if (G.head >= 0) units_.push_back(rownorm_unit(g_.nodes[G.head]));
        for (int k : G.nodes) units_.push_back(elementwise_unit(k));
        if (G.tail >= 0) {
            Unit u = rownorm_unit(g_.nodes[G.tail]);
            attach_half_copy(u, cons, done);
            units_.push_back(u);
        }
    }

    // The launch of a group: the row-norm kernel for [Add] + norm of two same-shape operands, the gated kernel
    // for [act, Mul], a standalone launch for a lone node, else the group program.
    void emit_group(const EwGroup& G, std::map<int, std::vector<int>>& cons, std::vector<bool>& done)
    {
        const Node& n0 = g_.nodes[G.nodes[0]];
        const std::vector<int> outs = group_outputs(G, cons);
        if (G.nodes.size() == 1 && G.head < 0 && G.tail < 0) {
            units_.push_back(elementwise_unit(G.nodes[0]));
            return;
        }
        if (G.nodes.size() == 1 && G.tail >= 0 && G.head < 0 && n0.op == "Add") {
            const auto& od = g_.value(n0.out[0]).dims;
            if (g_.value(n0.in[0]).dims == od && g_.value(n0.in[1]).dims == od &&
                g_.value(n0.in[0]).type == DType::F32 && g_.value(n0.in[1]).type == DType::F32) {
                const Node& m = g_.nodes[G.tail];
                Unit u = rownorm_unit(m);
                u.x = n0.in[0];
                u.res = n0.in[1];
                u.h = outs.empty() ? -1 : n0.out[0];
                u.label = std::string("fused[Add]+") + m.op;
                attach_half_copy(u, cons, done);
                units_.push_back(u);
                return;
            }
        }
        if (G.nodes.size() == 2 && G.head < 0 && G.tail < 0 && kActs.count(n0.op) && g_.nodes[G.nodes[1]].op == "Mul") {
            const Node& m = g_.nodes[G.nodes[1]];
            const int a = n0.out[0];
            const int up = m.in[0] == a ? m.in[1] : m.in[0];
            if ((m.in[0] == a) != (m.in[1] == a) && outs.size() == 1 && outs[0] == m.out[0] &&
                g_.value(up).dims == g_.value(n0.in[0]).dims && g_.value(m.out[0]).dims == g_.value(n0.in[0]).dims &&
                g_.value(up).type == g_.value(n0.in[0]).type) {
                Unit u{Unit::Gated};
                u.act = n0.op == "Silu" ? SLHIP_ACT_SILU : n0.op == "GeluTanh" ? SLHIP_ACT_GELU_TANH : SLHIP_ACT_GELU_ERF;
                u.gate = n0.in[0];
                u.up = up;
                u.y = m.out[0];
                u.label = "fused[" + n0.op + ",Mul]";
                units_.push_back(u);
                return;
            }
        }
        Unit u{Unit::EwGroup};
        u.shape_of = n0.out[0];
        u.head_node = G.head;
        u.tail_node = G.tail;
        std::map<int, int> reg;
        auto input = [&](int id) {
            auto it = reg.find(id);
            if (it != reg.end()) return it->second;
            const int r = static_cast<int>(u.ew_in.size());
            u.ew_in.push_back(id);
            u.ew_mode.push_back(input_mode(g_.value(id).dims, g_.value(u.shape_of).dims));
            reg[id] = r;
            return r;
        };
        if (G.head >= 0) {  // the head's input takes register 0; the norm's output is that register once normed
            const Node& h = g_.nodes[G.head];
            u.ew_in.push_back(h.in[0]);
            u.ew_mode.push_back(SLHIP_EWI_FULL);
            reg[h.out[0]] = 0;
            u.norm_reg = 0;
        }
        for (int k : G.nodes)  // every external input first: registers 0 .. n_inputs-1
            for (int id : g_.nodes[k].in) {
                bool produced = false;
                for (int j : G.nodes) produced = produced || g_.nodes[j].out[0] == id;
                if (!produced) input(id);
            }
        // registers: the inputs 0 .. n-1, then each op's result in a register whose value is dead (linear scan;
        // the stored values and the tail's operand live to the end)
        const int nin = static_cast<int>(u.ew_in.size());
        std::map<int, int> last;  // value -> index of the last op reading it (a large index: live to the end)
        constexpr int kEnd = 1 << 20;
        for (size_t i = 0; i < G.nodes.size(); i++)
            for (int id : g_.nodes[G.nodes[i]].in) last[id] = static_cast<int>(i);
        for (int v : outs) last[v] = kEnd;
        if (G.tail >= 0) last[g_.nodes[G.tail].in[0]] = kEnd;
        std::vector<bool> busy(SLHIP_EW_MAX_REGS, false);
        for (int r = 0; r < nin; r++) busy[r] = true;
        std::string label;
        for (size_t i = 0; i < G.nodes.size(); i++) {
            const Node& n = g_.nodes[G.nodes[i]];
            slhip_ew_op o{};
            o.round = SLHIP_F32;
            if (kBinaryOps.count(n.op)) {
                o.kind = SLHIP_EWK_BINARY;
                o.op = kBinaryOps.at(n.op);
                if (o.op == SLHIP_BIN_MOD && flag(n, "fmod")) o.op = SLHIP_BIN_FMOD;
                o.a = reg.at(n.in[0]);
                o.b = reg.at(n.in[1]);
            } else {
                o.kind = SLHIP_EWK_UNARY;
                o.op = kUnaryOps.at(n.op);
                std::tie(o.p0, o.p1) = unary_params(o.op, n);
                o.a = reg.at(n.in[0]);
            }
            for (int id : n.in)  // operands read for the last time free their registers (read before the write)
                if (last.at(id) == static_cast<int>(i)) busy[reg.at(id)] = false;
            int dst = -1;
            for (int r = 0; r < SLHIP_EW_MAX_REGS && dst < 0; r++)
                if (!busy[r]) dst = r;
            if (dst < 0) {  // more live values than registers: the nodes run one by one
                emit_unfused(G, cons, done);
                return;
            }
            busy[dst] = true;
            o.dst = dst;
            u.ew_ops.push_back(o);
            reg[n.out[0]] = dst;
            label += (i ? "," : "") + n.op;
        }
        for (int v : outs) u.ew_out.push_back({v, reg.at(v)});
        if (G.tail >= 0) u.norm_reg = reg.at(g_.nodes[G.tail].in[0]);
        u.label = (G.head >= 0 ? g_.nodes[G.head].op + "+" : std::string()) + "fused[" + label + "]" +
                  (G.tail >= 0 ? "+" + g_.nodes[G.tail].op : std::string());
        units_.push_back(u);
    }

    // Gate/up matmul pairs sharing x that feed act(gate) * up (FoldDualMatMuls,
    // src/Sharplight.Shaders/Lowering/GraphLowerer.Fusion.cs:286-353): both products read only by the
    // pattern, weights of one type and shape, the activation's output read only by the Mul.
    struct DualPattern {
        int mm_gate, mm_up, act_node, act;
    };
    std::map<int, DualPattern> dual_at_;  // Mul node -> its pattern
    std::set<int> absorbed_;              // MatMul and activation nodes inside a pattern

    template <class F>
    void find_dual_matvecs(std::map<int, std::vector<int>>& cons, F single_use)
    {
        std::map<int, int> producer;
        for (size_t k = 0; k < g_.nodes.size(); k++)
            for (int o : g_.nodes[k].out) producer[o] = static_cast<int>(k);
        auto prod = [&](int id) { auto it = producer.find(id); return it == producer.end() ? -1 : it->second; };
        for (size_t k = 0; k < g_.nodes.size(); k++) {
            const Node& m = g_.nodes[k];
            if (m.op != "Mul" || m.in.size() != 2) continue;
            for (int side = 0; side < 2; side++) {
                const int a = prod(m.in[side]), b = prod(m.in[1 - side]);
                if (a < 0 || b < 0 || !kActs.count(g_.nodes[a].op)) continue;
                const int ga = prod(g_.nodes[a].in[0]);
                if (ga < 0 || g_.nodes[ga].op != "MatMul" || g_.nodes[b].op != "MatMul") continue;
                const Node& mg = g_.nodes[ga];
                const Node& mu = g_.nodes[b];
                const Value& wg = g_.value(mg.in[1]);
                const Value& wu = g_.value(mu.in[1]);
                if (mg.in[0] != mu.in[0] || wg.type != wu.type || wg.dims != wu.dims) continue;
                if (!single_use(mg.out[0]) || !single_use(mu.out[0]) || !single_use(g_.nodes[a].out[0])) continue;
                // two matvecs + the gated unit when neither path fits the pair
                const bool fits_f32 = float_matvec_format(wg.type) && matvec_fits(format_code(wg.type), wg.dims[1], true);
                if (!fits_f32 && !(int_dot_range(g_, mg, wg.type, wg.dims[1]).any() &&
                                   matvec_q8_fits(format_code(wg.type), wg.dims[1], true)))
                    continue;
                if (g_.value(mg.out[0]).type != DType::F32 || g_.value(mu.out[0]).type != DType::F32 ||
                    g_.value(g_.nodes[a].out[0]).type != DType::F32)
                    continue;  // the unfused graph rounds nothing between the products and the Mul
                const std::string& an = g_.nodes[a].op;
                dual_at_[static_cast<int>(k)] = {ga, b, a, an == "Silu" ? SLHIP_ACT_SILU : an == "GeluTanh" ? SLHIP_ACT_GELU_TANH : SLHIP_ACT_GELU_ERF};
                absorbed_.insert(ga);
                absorbed_.insert(b);
                absorbed_.insert(a);
                break;
            }
        }
        (void)cons;
    }

    // A MatMul whose product is read only by an Add of a constant f32 row vector [N] (a weight) with an f32
    // result of the product's shape: the Add joins the matvec launch (FoldMatMulBiases,
    // src/Sharplight.Shaders/Lowering/GraphLowerer.Fusion.cs:355-408; LowerMatMulBias, GraphLowerer.MatMul.cs:205-245).
    template <class F>
    void fold_bias(Unit& u, std::map<int, std::vector<int>>& cons, std::vector<bool>& done, F single_use)
    {
        const int prod = u.y;
        if (!single_use(prod) || g_.value(prod).type != DType::F32) return;
        const int c = cons[prod][0];
        const Node& a = g_.nodes[c];
        if (a.op != "Add" || a.in.size() != 2 || done[c] || a.in[0] == a.in[1]) return;
        if (group_of_[c] >= 0) {  // a single-node Add group only (FoldMatMulBiases)
            const EwGroup& G = groups_[group_of_[c]];
            if (G.nodes.size() != 1 || G.head >= 0 || G.tail >= 0) return;
        }
        const int b = a.in[0] == prod ? a.in[1] : a.in[0];
        const Value& bv = g_.value(b);
        const Value& wv = g_.value(u.wg);
        const Value& ov = g_.value(a.out[0]);
        if (!bv.weight || bv.type != DType::F32 || bv.dims.size() != 1 || bv.dims[0] != wv.dims[0] ||
            ov.type != DType::F32 || ov.dims != g_.value(prod).dims)
            return;
        u.bias = b;
        u.y = a.out[0];
        u.label += "+bias";
        done[c] = true;
        if (group_of_[c] >= 0) {
            groups_[group_of_[c]].dead = true;
            group_of_[c] = -1;
        }
    }

    // The integer-dot range of every matvec unit, and the quantized copies of x they read: one per (x, row
    // range), made by a quantization launch placed before the first matvec that reads it and run for the row
    // counts of that range -- the lowerer's shared q8 copies (QuantizedActivations, GraphLowerer.IntDot.cs:119-220).
    void assign_q8()
    {
        std::map<std::tuple<int, int64_t, int64_t>, int> bufs;
        std::vector<Unit> out;
        for (Unit& u : units_) {
            if (u.kind == Unit::Matvec) {
                const Value& wv = g_.value(u.wg);
                u.q8 = int_dot_range(g_, g_.nodes[u.mm_node], wv.type, wv.dims[1]);
                const int64_t max_rows = g_.value(u.x).rows(max_t_);
                if (!float_matvec_format(wv.type) && max_rows > u.q8.hi)
                    unsupported(std::string("MatMul of ") + type_info(wv.type).name + " weights runs on the integer-dot "
                                "matvec only, up to " + std::to_string(u.q8.hi) + " activation rows; the segment may "
                                "run " + std::to_string(max_rows));
                if (u.q8.any()) {
                    const auto key = std::make_tuple(u.x, u.q8.lo, u.q8.hi);
                    auto it = bufs.find(key);
                    if (it == bufs.end()) {
                        Unit q{Unit::QuantizeQ8};
                        q.x = u.x;
                        q.q8 = u.q8;
                        q.q8buf = static_cast<int>(scratch_bytes_.size());
                        const Value& xv = g_.value(u.x);
                        scratch_bytes_.push_back(xv.rows(max_t_) * slhip_q8_row_bytes(xv.last()));
                        q.label = "x->q8 rows " + std::to_string(q.q8.lo) + ".." + std::to_string(q.q8.hi);
                        it = bufs.emplace(key, q.q8buf).first;
                        out.push_back(q);
                    }
                    u.q8buf = it->second;
                    u.label += " (int-dot rows " + std::to_string(u.q8.lo) + ".." + std::to_string(u.q8.hi) + ")";
                }
            }
            out.push_back(u);
        }
        units_.swap(out);
    }

    // A Cast of an f32 norm output to f16 is the f16 copy the norm writes beside its rows: the norm's f32
    // values rounded once, as the reference's row norm writes the half copy its GEMM readers take
    // (GraphLowerer.HalfCopies.cs:106-151, RowNormKernelSource.cs:45-49). The f32 rows are then written only
    // when something else reads them (GraphLowerer.Elementwise.cs:184-200).
    void attach_half_copy(Unit& u, std::map<int, std::vector<int>>& cons, std::vector<bool>& done)
    {
        const Value& yv = g_.value(u.y);
        if (yv.type != DType::F32) return;  // a bf16 y rounded again to f16 would differ from the copy
        for (int c : cons[u.y]) {
            const Node& m = g_.nodes[c];
            if (m.op != "Cast" || done[c] || g_.value(m.out[0]).type != DType::F16) continue;
            u.y16 = m.out[0];
            done[c] = true;
            u.skip_y = !yv.output && cons[u.y].size() == 1;
            u.label += u.skip_y ? "+f16copy(no f32 rows)" : "+f16copy";
            return;
        }
    }

    Unit rope_unit(int k)
    {
        const Node& r = g_.nodes[k];
        Unit u{Unit::Rope};
        int x = r.in[0], w = -1;
        float eps = 0.f;
        auto it = absorbed_norm_.find(k);
        if (it != absorbed_norm_.end()) {
            const Node& nn = g_.nodes[it->second];
            x = nn.in[0];
            w = nn.in[1];
            eps = nn.f("eps", 1e-6f);
        }
        const Value& xv = g_.value(x);
        u.rt.push_back({x, r.out[0], w});
        u.pos = r.in[1];
        u.ff = r.in.size() > 2 ? r.in[2] : -1;
        const std::string style = r.s("style", "neox");
        u.cfg.dims = static_cast<int32_t>(r.i("dims", 0));
        u.cfg.neox = !(style == "gptj" || style == "normal");  // RopeOp.cs:43
        u.cfg.base = r.f("base", 10000.f);
        u.cfg.freq_scale = r.f("freq_scale", 1.f);
        u.cfg.attn_factor = r.f("attn_factor", 1.f);
        u.cfg.norm = w >= 0 ? 1 : 0;
        u.cfg.eps = eps;
        // multi-axis positions [T, A] and the M-RoPE sections (StandardOps.cs:182-192)
        const Value& pv = g_.value(r.in[1]);
        u.cfg.pos_axes = pv.dims.size() == 2 ? static_cast<int32_t>(pv.dims[1]) : 1;
        std::vector<int> sec;
        parse_sections(r.s("sections", ""), sec);
        for (int q = 0; q < 4; q++) u.cfg.sections[q] = sec[q];
        u.cfg.interleaved = flag(r, "interleaved") ? 1 : 0;
        u.cfg.per_element = flag(r, "sections_per_element") ? 1 : 0;
        u.label = w >= 0 ? "rope+norm" : "rope";
        if (xv.type != g_.value(r.out[0]).type && !(is_activation(g_.value(r.out[0]).type)))
            unsupported("Rope output type");
        return u;
    }

    // Consecutive rope units with the same positions, frequency factors, settings and types become one launch.
    void merge_ropes()
    {
        std::vector<Unit> out;
        for (Unit& u : units_) {
            if (u.kind == Unit::Rope && !out.empty()) {
                Unit& p = out.back();
                const Value& a = g_.value(p.rt[0].x);
                const Value& b = g_.value(u.rt[0].x);
                int pc = -1;  // the cache rows already in the launch, if any
                for (const auto& t : p.rt)
                    if (t.cache_node >= 0) pc = t.cache_node;
                const int uc = u.rt[0].cache_node;
                const bool same = p.kind == Unit::Rope && p.pos == u.pos && p.ff == u.ff && p.rt.size() < 4 &&
                                  memcmp(&p.cfg, &u.cfg, sizeof p.cfg) == 0 && a.type == b.type &&
                                  g_.value(p.rt[0].y).type == g_.value(u.rt[0].y).type && a.dims[2] == b.dims[2] &&
                                  a.dims[0] == b.dims[0] && (pc < 0 || uc < 0 || same_rows(pc, uc));
                if (same) {
                    p.rt.push_back(u.rt[0]);
                    p.label += "|" + u.label;
                    continue;
                }
            }
            out.push_back(u);
        }
        units_ = out;
    }

    void allocate()
    {
        for (auto& kv : g_.values) {
            const int64_t n = kv.second.bytes(max_t_);
            void* p = nullptr;
            check(slhip_malloc(&p, static_cast<size_t>(n > 0 ? n : 0)));
            mem_[kv.first] = p;
            device_bytes_ += n;
        }
        for (int64_t n : scratch_bytes_) {
            void* p = nullptr;
            check(slhip_malloc(&p, static_cast<size_t>(n > 0 ? n : 0)));
            scratch_.push_back(p);
            device_bytes_ += n;
        }
    }

    // The fused group's program (slhip_ew_program) on the segment's buffers.
    slhip_ew_program ew_program_of(const Unit& u) const
    {
        slhip_ew_program p{};
        p.n_inputs = static_cast<int>(u.ew_in.size());
        p.n_ops = static_cast<int>(u.ew_ops.size());
        p.n_outputs = static_cast<int>(u.ew_out.size());
        for (int i = 0; i < p.n_inputs; i++)
            p.inputs[i] = slhip_ew_input{ptr(u.ew_in[i]), act_code(g_.value(u.ew_in[i]).type), u.ew_mode[i]};
        for (int k = 0; k < p.n_ops; k++) p.ops[k] = u.ew_ops[k];
        for (int j = 0; j < p.n_outputs; j++)
            p.outputs[j] = slhip_ew_output{ptr(u.ew_out[j].first), act_code(g_.value(u.ew_out[j].first).type), u.ew_out[j].second};
        auto norm_of = [&](int node, bool tail) {
            const Node& nm = g_.nodes[node];
            slhip_ew_norm r{};
            r.kind = nm.op == "L2Norm" ? SLHIP_EWN_L2 : SLHIP_EWN_RMS;
            r.reg = u.norm_reg;
            r.w = nm.in.size() > 1 ? static_cast<const float*>(ptr(nm.in[1])) : nullptr;
            r.eps = nm.f("eps", 1e-6f);
            r.y = tail ? ptr(nm.out[0]) : nullptr;
            r.dtype_y = act_code(g_.value(nm.out[0]).type);
            return r;
        };
        if (u.head_node >= 0) p.head = norm_of(u.head_node, false);
        if (u.tail_node >= 0) p.tail = norm_of(u.tail_node, true);
        return p;
    }

    // The fused groups' generated kernels are made at compile time, so that the first Execute (or a graph
    // recorded from it) launches them rather than the interpreter.
    void prepare_groups()
    {
        for (const Unit& u : units_) {
            if (u.kind != Unit::EwGroup) continue;
            const slhip_ew_program p = ew_program_of(u);
            check(ew_program_prepare(&p, g_.value(u.shape_of).last()));
        }
    }

    void* ptr(int id) const { return id < 0 ? nullptr : mem_.at(id); }

    // Two cache writes that map tokens to the same rows (one launch may carry one row map).
    bool same_rows(int a, int b) const
    {
        const Node& x = g_.nodes[a];
        const Node& y = g_.nodes[b];
        return x.in.size() == y.in.size() && std::equal(x.in.begin() + 2, x.in.end(), y.in.begin() + 2) &&
               x.s("offset", "n_past") == y.s("offset", "n_past") && x.i("slots", 1) == y.i("slots", 1) &&
               x.i("block_size", 16) == y.i("block_size", 16) && g_.value(x.in[0]).dims[0] == g_.value(y.in[0]).dims[0];
    }

    // The rows of cache write `node` for a run of T tokens: n_past + t from the offset scalar, or the
    // multi-sequence rows [T, 4] (3rd input, attribute slots), or those through the block table (4th input,
    // attribute block_size) -- the inputs the reference's MultiSequence rewrite appends
    // (src/Sharplight.Core/Graph/MultiSequence.cs:201-233).
    slhip_cache_rows rows_of(int node, int64_t T) const
    {
        const Node& n = g_.nodes[node];
        const Value& st = g_.value(n.in[0]);
        slhip_cache_rows r{};
        r.ctx = st.dims[0];
        if (n.in.size() == 2) {
            const std::string name = n.s("offset", "n_past");
            auto it = scalars_.find(name);
            if (it == scalars_.end())  // CacheWriteOp.Run (src/Sharplight.Cpu/CacheWriteOp.cs:114-117)
                throw Error(SLHIP_ERR_INVALID, "Runtime scalar '" + name + "' was not provided.");
            r.mode = SLHIP_ROWS_PAST;
            r.n_past = it->second;
            return r;
        }
        r.seq = static_cast<const int32_t*>(ptr(n.in[2]));
        if (n.in.size() == 3) {
            r.mode = SLHIP_ROWS_SEQ;
            r.slots = n.i("slots", 1);
            return r;
        }
        const Value& pg = g_.value(n.in[3]);
        r.mode = SLHIP_ROWS_PAGED;
        r.pages = static_cast<const int32_t*>(ptr(n.in[3]));
        r.page_slots = pg.dims.size() == 2 ? pg.dims[0] : 1;
        r.blocks_per_slot = pg.dims.back();
        r.block_size = n.i("block_size", 16);
        (void)T;
        return r;
    }

    void run(const Unit& u, int64_t T)
    {
        switch (u.kind) {
        case Unit::RowNorm: {
            const Value& x = g_.value(u.x);
            const Value& y = g_.value(u.y);
            const int64_t D = x.last(), rows = x.rows(T);
            const slhip_norm_copies copies{ptr(u.y16), D, nullptr, 0};
            check(slhip_rownorm_copies(u.norm, act_code(x.type), act_code(y.type), ptr(u.x), ptr(u.res),
                                       static_cast<const float*>(ptr(u.w)), static_cast<const float*>(ptr(u.b)),
                                       u.skip_y ? nullptr : ptr(u.y), ptr(u.h), rows, D, D, D, D, D, u.eps,
                                       u.y16 >= 0 ? &copies : nullptr, stream_));
            break;
        }
        case Unit::QuantizeQ8: {
            const Value& xv = g_.value(u.x);
            const int64_t K = xv.last(), rows = xv.rows(T);
            if (u.q8.covers(rows))
                check(slhip_quantize_q8(act_code(xv.type), ptr(u.x), K, rows, K, scratch_.at(u.q8buf), stream_));
            break;
        }
        case Unit::Matvec: {
            const Value& xv = g_.value(u.x);
            const Value& wv = g_.value(u.wg);
            const int64_t K = xv.last(), rows = xv.rows(T), Nw = wv.dims[0];
            const int fmt = format_code(wv.type);
            const int dy = act_code(g_.value(u.y).type);
            const float* bias = static_cast<const float*>(ptr(u.bias));
            if (rows == 0) break;
            if (u.q8.covers(rows)) {
                void* xq = scratch_.at(u.q8buf);
                if (u.wu >= 0)
                    check(slhip_dual_matvec_q8(u.act, fmt, dy, xq, rows, K, ptr(u.wg), ptr(u.wu), Nw, ptr(u.y), Nw, stream_));
                else
                    check(slhip_matvec_q8(fmt, dy, xq, rows, K, ptr(u.wg), Nw, ptr(u.y), Nw, bias, stream_));
                break;
            }
            if (!float_matvec_format(wv.type))  // refused at compile; kept as a guard
                unsupported(std::string("MatMul of ") + type_info(wv.type).name + " weights [" + std::to_string(Nw) +
                            ", " + std::to_string(K) + "] runs on the integer-dot matvec only, for " +
                            std::to_string(u.q8.lo) + ".." + std::to_string(u.q8.hi) + " activation rows; this run has " +
                            std::to_string(rows));
            if (u.wu >= 0)
                check(slhip_dual_matvec(u.act, fmt, act_code(xv.type), dy, ptr(u.x), K, rows, K, ptr(u.wg), ptr(u.wu), Nw,
                                        ptr(u.y), Nw, stream_));
            else
                check(slhip_matvec_bias(fmt, act_code(xv.type), dy, ptr(u.x), K, rows, K, ptr(u.wg), Nw, bias, ptr(u.y), Nw,
                                        stream_));
            break;
        }
        case Unit::Gated: {
            const Value& gv = g_.value(u.gate);
            const int64_t cols = gv.last(), rows = gv.rows(T);
            check(slhip_gated_act(u.act, act_code(gv.type), act_code(g_.value(u.y).type), ptr(u.gate), ptr(u.up), ptr(u.y),
                                  rows, cols, cols, cols, cols, stream_));
            break;
        }
        case Unit::Rope: {
            std::vector<slhip_rope_tensor> ts;
            std::vector<slhip_cache_rows> rows;
            rows.reserve(u.rt.size());  // the tensors point into it
            const Value& x0 = g_.value(u.rt[0].x);
            const int64_t Tt = x0.dims[0] == kSymT ? T : x0.dims[0];
            const int64_t D = x0.dims[2];
            for (const auto& r : u.rt) {
                const Value& xv = g_.value(r.x);
                const int64_t H = xv.dims[1];
                slhip_rope_tensor t{ptr(r.x), ptr(r.y), static_cast<const float*>(ptr(r.w)), H, H * D, D, H * D, D, nullptr};
                if (r.cache_node >= 0) {
                    const Value& st = g_.value(r.y);
                    rows.push_back(rows_of(r.cache_node, Tt));
                    t.y_stride_t = st.dims[1] * st.dims[2];
                    t.rows = &rows.back();
                }
                ts.push_back(t);
            }
            check(slhip_rope(act_code(x0.type), act_code(g_.value(u.rt[0].y).type), ts.data(), static_cast<int>(ts.size()),
                             static_cast<const int32_t*>(ptr(u.pos)), static_cast<const float*>(ptr(u.ff)), Tt, D, &u.cfg,
                             stream_));
            break;
        }
        case Unit::Gather: {
            const Value& t = g_.value(u.table);
            const Value& ids = g_.value(u.ids);
            int64_t D = 1;
            for (size_t k = 1; k < t.dims.size(); k++) D *= t.dims[k];
            const int64_t N = ids.elems(T);
            check(slhip_gather(format_code(t.type), ptr(u.table), t.dims[0], D, static_cast<const int32_t*>(ptr(u.ids)), N,
                               act_code(g_.value(u.y).type), ptr(u.y), D, stream_));
            break;
        }
        case Unit::Cast: {
            const Value& x = g_.value(u.x);
            check(slhip_convert(act_code(x.type), act_code(g_.value(u.y).type), ptr(u.x), ptr(u.y), x.elems(T), stream_));
            break;
        }
        case Unit::Binary: {
            const std::vector<int64_t> yd = dims_at(u.y, T);
            const std::vector<int64_t> sa = align(dims_at(u.x, T), yd.size()), sb = align(dims_at(u.up, T), yd.size());
            check(slhip_binary(u.op, act_code(g_.value(u.x).type), act_code(g_.value(u.up).type), act_code(g_.value(u.y).type),
                               ptr(u.x), sa.data(), ptr(u.up), sb.data(), ptr(u.y), yd.data(), static_cast<int>(yd.size()),
                               stream_));
            break;
        }
        case Unit::EwGroup: {
            const slhip_ew_program p = ew_program_of(u);
            const Value& sv = g_.value(u.shape_of);
            check(slhip_ew_program_run(&p, sv.rows(T), sv.last(), stream_));
            break;
        }
        case Unit::Unary: {
            const Value& x = g_.value(u.x);
            const int64_t cols = x.last(), rows = x.rows(T);
            check(slhip_unary(u.op, act_code(x.type), act_code(g_.value(u.y).type), ptr(u.x), ptr(u.y), rows, cols, cols, cols,
                              u.p0, u.p1, stream_));
            break;
        }
        case Unit::CacheWrite: {
            const Value& x = g_.value(u.x);
            const Value& st = g_.value(u.y);
            const int64_t Tt = x.dims[0] == kSymT ? T : x.dims[0];
            const int64_t inner = st.inner();
            const slhip_cache_rows r = rows_of(u.cache_node, Tt);
            check(slhip_cache_write(act_code(x.type), act_code(st.type), ptr(u.x), inner, Tt, inner, ptr(u.y), &r, stream_));
            break;
        }
        }
    }
};

template <typename F>
int guarded(F&& f)
{
    try {
        f();
        return SLHIP_OK;
    } catch (const Error& e) {
        return fail(e.status, "%s", e.what());
    } catch (const std::exception& e) {
        return fail(SLHIP_ERR_INVALID, "%s", e.what());
    }
}

}  // namespace
}  // namespace slhip

using namespace slhip;

extern "C" {

SLHIP_API int slhip_provider_check(char* reason, size_t reason_size)
{
    // The library carries gfx950 code objects only: a device of another architecture cannot run them.
    int n = 0;
    int st = slhip_device_count(&n);
    char why[256] = "";
    if (st) {
        snprintf(why, sizeof why, "%s", slhip_last_error());
    } else if (n == 0) {
        snprintf(why, sizeof why, "no HIP device is visible");
    } else {
        int usable = 0;
        char seen[64] = "unknown";
        for (int i = 0; i < n; ++i) {
            slhip_device_props p;
            if (slhip_device_props_get(i, &p) != SLHIP_OK) continue;
            if (strncmp(p.arch, "gfx950", 6) == 0) ++usable;
            else snprintf(seen, sizeof seen, "%s", p.arch);
        }
        if (!usable) snprintf(why, sizeof why, "no gfx950 device among %d visible (found %s)", n, seen);
    }
    if (reason && reason_size) snprintf(reason, reason_size, "%s", why);
    if (st) return st;
    return why[0] ? fail(SLHIP_ERR_NO_DEVICE, "%s", why) : SLHIP_OK;
}

SLHIP_API int slhip_node_supports(const char* segment_ir, int node_index, int* supported, char* reason,
                                  size_t reason_size)
{
    return guarded([&] {
        if (!supported) invalid("supported is null");
        Graph g = parse(segment_ir);
        if (node_index < 0 || node_index >= static_cast<int>(g.nodes.size())) invalid("node index out of range");
        Support s = supports(g, g.nodes[node_index]);
        *supported = s.ok ? 1 : 0;
        if (reason && reason_size) snprintf(reason, reason_size, "%s", s.reason.c_str());
    });
}

SLHIP_API int slhip_segment_compile(const char* segment_ir, int64_t max_tokens, slhip_segment* segment)
{
    return guarded([&] {
        if (!segment) invalid("segment is null");
        *segment = nullptr;
        auto s = std::make_unique<Segment>(parse(segment_ir), max_tokens);
        *segment = s.release();
    });
}

// Copies text into a caller's buffer, failing (not truncating) when it does not fit.
static void put_text(const std::string& text, char* buf, size_t size)
{
    if (!buf || !size) invalid("null argument");
    if (text.size() + 1 > size) invalid("buffer of " + std::to_string(size) + " bytes too small for " +
                                        std::to_string(text.size() + 1));
    memcpy(buf, text.c_str(), text.size() + 1);
}

SLHIP_API int slhip_segment_plan(const char* segment_ir, char* buf, size_t size)
{
    return guarded([&] {
        Segment s(parse(segment_ir), 0, true);
        put_text(s.launches(), buf, size);
    });
}

SLHIP_API int slhip_segment_describe(const char* segment_ir, char* buf, size_t size)
{
    return guarded([&] {
        const Graph g = parse(segment_ir);
        std::string out;
        for (const auto& [k, v] : g.options) out += "option " + k + "=" + v + "\n";
        for (const auto& [id, v] : g.values) {
            out += "value " + std::to_string(id) + " " + type_info(v.type).name;
            for (int64_t d : v.dims) out += " " + (d == kSymT ? std::string("T") : std::to_string(d));
            out += "\n";
        }
        const char* roles[4] = {"input", "weight", "output", "state"};
        for (int r = 0; r < 4; r++)
            for (const auto& [id, v] : g.values)
                if ((r == 0 && v.input) || (r == 1 && v.weight) || (r == 2 && v.output) || (r == 3 && v.state))
                    out += std::string(roles[r]) + " " + std::to_string(id) + "\n";
        auto ids = [](const std::vector<int>& l) {
            if (l.empty()) return std::string("-");
            std::string t;
            for (size_t k = 0; k < l.size(); k++) t += (k ? "," : "") + std::to_string(l[k]);
            return t;
        };
        for (const Node& n : g.nodes) {
            out += "node " + n.op + " " + ids(n.in) + " -> " + ids(n.out);
            for (const auto& [k, v] : n.attr) out += " " + k + "=" + v;  // std::map: sorted by key
            out += "\n";
        }
        put_text(out, buf, size);
    });
}

SLHIP_API int slhip_segment_set_input(slhip_segment segment, int value, const void* data, size_t bytes)
{
    return guarded([&] {
        if (!segment) invalid("segment is null");
        static_cast<Segment*>(segment)->set_input(value, data, bytes);
    });
}

SLHIP_API int slhip_segment_execute(slhip_segment segment, int64_t tokens)
{
    return guarded([&] {
        if (!segment) invalid("segment is null");
        static_cast<Segment*>(segment)->execute(tokens);
    });
}

SLHIP_API int slhip_segment_get_output(slhip_segment segment, int value, void* data, size_t bytes)
{
    return guarded([&] {
        if (!segment) invalid("segment is null");
        static_cast<Segment*>(segment)->get_output(value, data, bytes);
    });
}

SLHIP_API int slhip_segment_device_bytes(slhip_segment segment, int64_t* bytes)
{
    return guarded([&] {
        if (!segment || !bytes) invalid("null argument");
        *bytes = static_cast<Segment*>(segment)->device_bytes();
    });
}

SLHIP_API int slhip_segment_launches(slhip_segment segment, char* buf, size_t size)
{
    return guarded([&] {
        if (!segment || !buf || !size) invalid("null argument");
        snprintf(buf, size, "%s", static_cast<Segment*>(segment)->launches().c_str());
    });
}

SLHIP_API int slhip_segment_launches_at(slhip_segment segment, int64_t tokens, char* buf, size_t size)
{
    return guarded([&] {
        if (!segment || !buf || !size) invalid("null argument");
        if (tokens < 0) invalid("T must not be negative");
        put_text(static_cast<Segment*>(segment)->launches_at(tokens), buf, size);
    });
}

SLHIP_API int slhip_segment_reset_state(slhip_segment segment)
{
    return guarded([&] {
        if (!segment) invalid("segment is null");
        static_cast<Segment*>(segment)->reset_state();
    });
}

SLHIP_API int slhip_segment_set_scalar(slhip_segment segment, const char* name, int64_t value)
{
    return guarded([&] {
        if (!segment || !name) invalid("segment and name are required");
        static_cast<Segment*>(segment)->set_scalar(name, value);
    });
}

SLHIP_API int slhip_segment_destroy(slhip_segment segment)
{
    return guarded([&] { delete static_cast<Segment*>(segment); });
}

}  // extern "C"
