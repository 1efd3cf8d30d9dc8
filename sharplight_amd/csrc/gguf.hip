// GGUF files and the staged weight upload: the on-disk -> device path of the weights and tables the
// kernels of this library read.
//
// Reader: src/Sharplight.Import.Gguf/GgufFile.cs:72-245 (open, header, metadata, tensor table, sizes and
// bounds), GgufReader.cs:1-175 (bounds-checked cursor, value types, array guards), GgmlTypes.cs:52-119
// (type ids), GgufHeaderProbe.cs:17-135 (header prefixes), GgufInterleavedQ4_0Source.cs:43-79 and
// GgufI2sSource.cs:39-64, GgufNarrowIq1Source.cs and GgmlNarrowIq1.cs:55-86 (types read in another layout
// than stored).
// Uploader: src/Sharplight.Vulkan/WeightUploader.cs:6-140 (two staging buffers, one filled by the host
// while the other is copied).
//
// Everything here is host code. The file is mapped read-only once; metadata values are nodes of a tree
// whose numeric arrays and strings point into the mapping (a prefix is copied first, so they point into
// the copy).
#include "common.hpp"
#include "narrow_iq1_grids.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cmath>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <thread>
#include <unordered_map>
#include <vector>

namespace {

using slhip::fail;

constexpr uint32_t kMagic = 0x46554747;  // "GGUF" little-endian
constexpr uint32_t kDefaultAlignment = 32;
constexpr int64_t kHeaderBytes = 24;
constexpr uint32_t kMaxDims = 8;
constexpr int64_t kMinStringBytes = 8;   // a string's length prefix
constexpr int64_t kMinArrayBytes = 12;   // a nested array's element type and count
constexpr int kMaxArrayDepth = 64;      // nesting limit of arrays of arrays
constexpr int64_t kIntMax = 2147483647;

// A malformed file (SLHIP_ERR_FORMAT) or a valid file this library does not read (SLHIP_ERR_UNSUPPORTED).
struct GgufError {
    int status;
    std::string message;
};
[[noreturn]] void format_error(std::string m) { throw GgufError{SLHIP_ERR_FORMAT, std::move(m)}; }
[[noreturn]] void unsupported(std::string m) { throw GgufError{SLHIP_ERR_UNSUPPORTED, std::move(m)}; }

// ---- ggml types ---------------------------------------------------------------------------------

enum class Layout { Plain, InterleavedQ4_0, NarrowIq1, I2S };

struct TypeDesc {
    const char* name = nullptr;  // nullptr: unknown id
    int block_size = 0;
    int block_bytes = 0;
    int format = -1;             // slhip_format, -1 when no kernel here reads it
    Layout layout = Layout::Plain;
    int rows = 0, chunk = 0;     // interleaved Q4_0: rows per group, nibble bytes kept together
    int stored_block = 0;        // narrow IQ1: stored bytes per 256-value block
};

constexpr int kI2S = 36;
constexpr int kWideIq1Bytes = 50;  // an IQ1_S block
constexpr int kI2sBlock = 36, kI2sCodes = 32;

// GgmlTypes.TryGetDataType (GgmlTypes.cs:94-119) with the block geometry of each DataType
// (src/Sharplight.Core/Tensors/DataType.cs:76-244).
TypeDesc type_desc(int id)
{
    auto t = [](const char* n, int bs, int bb, int fmt = -1) {
        TypeDesc d;
        d.name = n;
        d.block_size = bs;
        d.block_bytes = bb;
        d.format = fmt;
        return d;
    };
    switch (id) {
    case 0: return t("f32", 1, 4, SLHIP_FMT_F32);
    case 1: return t("f16", 1, 2, SLHIP_FMT_F16);
    case 2: return t("q4_0", 32, 18, SLHIP_FMT_Q4_0);
    case 3: return t("q4_1", 32, 20, SLHIP_FMT_Q4_1);
    case 6: return t("q5_0", 32, 22, SLHIP_FMT_Q5_0);
    case 7: return t("q5_1", 32, 24, SLHIP_FMT_Q5_1);
    case 8: return t("q8_0", 32, 34, SLHIP_FMT_Q8_0);
    case 9: return t("q8_1", 32, 36);
    case 10: return t("q2_k", 256, 84, SLHIP_FMT_Q2_K);
    case 11: return t("q3_k", 256, 110, SLHIP_FMT_Q3_K);
    case 12: return t("q4_k", 256, 144, SLHIP_FMT_Q4_K);
    case 13: return t("q5_k", 256, 176, SLHIP_FMT_Q5_K);
    case 14: return t("q6_k", 256, 210, SLHIP_FMT_Q6_K);
    case 15: return t("q8_k", 256, 292);
    case 16: return t("iq2_xxs", 256, 66, SLHIP_FMT_IQ2_XXS);
    case 17: return t("iq2_xs", 256, 74, SLHIP_FMT_IQ2_XS);
    case 18: return t("iq3_xxs", 256, 98, SLHIP_FMT_IQ3_XXS);
    case 19: return t("iq1_s", 256, 50, SLHIP_FMT_IQ1_S);
    case 20: return t("iq4_nl", 32, 18, SLHIP_FMT_IQ4_NL);
    case 21: return t("iq3_s", 256, 110, SLHIP_FMT_IQ3_S);
    case 22: return t("iq2_s", 256, 82, SLHIP_FMT_IQ2_S);
    case 23: return t("iq4_xs", 256, 136, SLHIP_FMT_IQ4_XS);
    case 24: return t("i8", 1, 1);
    case 25: return t("i16", 1, 2);
    case 26: return t("i32", 1, 4);
    case 27: return t("i64", 1, 8);
    case 28: return t("f64", 1, 8);
    case 29: return t("iq1_m", 256, 56, SLHIP_FMT_IQ1_M);
    case 30: return t("bf16", 1, 2, SLHIP_FMT_BF16);
    case 31: case 32: case 33: {  // Q4_0_4_4, Q4_0_4_8, Q4_0_8_8: read as Q4_0 rows
        TypeDesc d = t("q4_0", 32, 18, SLHIP_FMT_Q4_0);
        d.layout = Layout::InterleavedQ4_0;
        d.rows = id == 33 ? 8 : 4;
        d.chunk = id == 31 ? 4 : 8;
        return d;
    }
    case 34: return t("tq1_0", 256, 54, SLHIP_FMT_TQ1_0);
    case 35: return t("tq2_0", 256, 66, SLHIP_FMT_TQ2_0);
    case kI2S: {  // BitNet's I2_S: read as Q2S_G128 blocks (f32 scale + 32 code bytes)
        TypeDesc d = t("q2s_g128", 128, kI2sBlock, SLHIP_FMT_Q2S_G128);
        d.layout = Layout::I2S;
        return d;
    }
    case 39: return t("mxfp4", 32, 17, SLHIP_FMT_MXFP4);
    case 40: return t("nvfp4", 64, 36, SLHIP_FMT_NVFP4);
    case 41: return t("q1_0", 128, 18, SLHIP_FMT_Q1_0);
    case 42: return t("q2_0", 64, 18, SLHIP_FMT_Q2_0);
    case 43: return t("f8_e4m3", 1, 1, SLHIP_FMT_F8E4M3);
    case 64: case 65: case 66: {  // unsloth's narrow IQ1 types: read as IQ1_S blocks
        TypeDesc d = t("iq1_s", 256, kWideIq1Bytes, SLHIP_FMT_IQ1_S);
        d.layout = Layout::NarrowIq1;
        d.stored_block = id == 64 ? 46 : id == 65 ? 42 : 38;
        return d;
    }
    case 142: return t("q2_0_g128", 128, 34, SLHIP_FMT_Q2_0_G128);   // PrismML PQ2_0
    case 143: return t("tern1_g128", 128, 28, SLHIP_FMT_TERN1_G128);  // PrismML PTQ1_0
    case 144: return t("trellis_v4k8_g128", 128, 34, SLHIP_FMT_TRELLIS_V4K8_G128);
    case 145: return t("trellis_v4k6_g128", 128, 26, SLHIP_FMT_TRELLIS_V4K6_G128);
    case 146: return t("trellis_v4k7_g128", 128, 30, SLHIP_FMT_TRELLIS_V4K7_G128);
    case 147: return t("trellis_v2k5_g128", 128, 42, SLHIP_FMT_TRELLIS_V2K5_G128);
    case 148: return t("trellis_v2k6_g128", 128, 50, SLHIP_FMT_TRELLIS_V2K6_G128);
    case 149: return t("trellis_v2k7_g128", 128, 58, SLHIP_FMT_TRELLIS_V2K7_G128);
    default: return TypeDesc{};
    }
}

bool mul_overflows(int64_t a, int64_t b, int64_t* r) { return __builtin_mul_overflow(a, b, r); }

// GgufFile.ComputeByteSize (GgufFile.cs:215-230).
int64_t compute_byte_size(const TypeDesc& d, const std::vector<int64_t>& ne, const std::string& name)
{
    int64_t elements = 1;
    for (int64_t n : ne)
        if (mul_overflows(elements, n, &elements)) format_error("Tensor '" + name + "': element count overflows.");
    const int64_t row = ne.empty() ? 1 : ne[0];
    if (row % d.block_size != 0)
        format_error("Tensor '" + name + "': row length " + std::to_string(row) + " is not a multiple of " + d.name +
                     " block size " + std::to_string(d.block_size) + ".");
    int64_t size;
    if (mul_overflows(elements / d.block_size, static_cast<int64_t>(d.block_bytes), &size))
        format_error("Tensor '" + name + "': byte size overflows.");
    return size;
}

// GgufFile.StoredByteSize (GgufFile.cs:207-213).
int64_t stored_byte_size(const TypeDesc& d, int64_t size)
{
    if (d.layout == Layout::NarrowIq1) return size / kWideIq1Bytes * d.stored_block;
    if (d.layout == Layout::I2S) return size / kI2sBlock * kI2sCodes + 32;
    return size;
}

// ---- the parsed file ----------------------------------------------------------------------------

struct Node {
    uint32_t type = 0, elem = 0;
    int64_t count = 0;
    uint64_t u = 0;
    int64_t i = 0;
    double f = 0.0;
    const uint8_t* data = nullptr;
    int64_t first_child = -1;
};

struct Tensor {
    std::string name;
    int ggml = 0;
    TypeDesc desc;
    std::vector<int64_t> ne;
    int64_t rel = 0, abs = 0, size = 0, stored = 0;
};

// The bounds-checked little-endian cursor (GgufReader.cs:34-57).
struct Cursor {
    const uint8_t* base;
    int64_t length;
    int64_t pos = 0;
    const uint8_t* take(int64_t n)
    {
        if (n < 0 || n > length - pos) format_error("Unexpected end of GGUF file.");
        const uint8_t* p = base + pos;
        pos += n;
        return p;
    }
    template <typename T> T read()
    {
        T v;
        std::memcpy(&v, take(sizeof(T)), sizeof(T));
        return v;
    }
    int64_t read_len()  // checked((long)ReadU64())
    {
        const uint64_t v = read<uint64_t>();
        if (v > static_cast<uint64_t>(INT64_MAX)) format_error("Arithmetic operation resulted in an overflow.");
        return static_cast<int64_t>(v);
    }
    int64_t remaining() const { return length - pos; }
};

}  // namespace

struct slhip_gguf {
    // the bytes: a mapping of the file, or an owned copy of a prefix
    int fd = -1;
    const uint8_t* base = nullptr;
    int64_t length = 0;
    std::vector<uint8_t> copy;
    bool has_data = false;
    uint32_t version = 0, alignment = kDefaultAlignment;
    int64_t data_offset = -1;
    bool table_complete = false;
    std::vector<std::pair<std::string, int64_t>> kv;  // key, node
    std::unordered_map<std::string, int64_t> kv_index;
    std::vector<Node> nodes;
    std::vector<Tensor> tensors;
    std::unordered_map<std::string, int64_t> by_name;

    ~slhip_gguf()
    {
        if (base && fd >= 0) munmap(const_cast<uint8_t*>(base), static_cast<size_t>(length));
        if (fd >= 0) close(fd);
    }

    // GgufReader.ReadString: the node keeps a pointer to the bytes.
    void read_string(Cursor& c, Node& n)
    {
        const int64_t len = c.read_len();
        if (len > kIntMax) format_error("String too long.");
        n.type = SLHIP_GGUF_STRING;
        n.count = len;
        n.data = len ? c.take(len) : c.base + c.pos;
    }
    std::string read_key(Cursor& c)
    {
        Node n;
        read_string(c, n);
        return std::string(reinterpret_cast<const char*>(n.data), static_cast<size_t>(n.count));
    }

    // GgufReader.ReadValue / ReadArray (GgufReader.cs:72-144). Fills nodes[id]; children are appended.
    void read_value(Cursor& c, uint32_t type, int64_t id, int depth = 0)
    {
        Node n;
        n.type = type;
        switch (type) {
        case SLHIP_GGUF_UINT8: n.u = c.read<uint8_t>(); break;
        case SLHIP_GGUF_INT8: n.i = c.read<int8_t>(); break;
        case SLHIP_GGUF_UINT16: n.u = c.read<uint16_t>(); break;
        case SLHIP_GGUF_INT16: n.i = c.read<int16_t>(); break;
        case SLHIP_GGUF_UINT32: n.u = c.read<uint32_t>(); break;
        case SLHIP_GGUF_INT32: n.i = c.read<int32_t>(); break;
        case SLHIP_GGUF_FLOAT32: n.f = c.read<float>(); break;
        case SLHIP_GGUF_BOOL: n.u = c.read<uint8_t>() != 0; break;
        case SLHIP_GGUF_STRING: read_string(c, n); break;
        case SLHIP_GGUF_UINT64: n.u = c.read<uint64_t>(); break;
        case SLHIP_GGUF_INT64: n.i = c.read<int64_t>(); break;
        case SLHIP_GGUF_FLOAT64: n.f = c.read<double>(); break;
        case SLHIP_GGUF_ARRAY: {
            const uint32_t elem = c.read<uint32_t>();
            const int64_t count = c.read_len();
            if (count > kIntMax) format_error("Array too large.");
            // arrays of arrays recurse on the native stack: a crafted file of a few MB could nest deep
            // enough to overflow it, so nesting beyond kMaxArrayDepth is a format error
            if (depth >= kMaxArrayDepth) format_error("Arrays nested deeper than " + std::to_string(kMaxArrayDepth) + ".");
            n.elem = elem;
            n.count = count;
            static const int kSize[13] = {1, 1, 2, 2, 4, 4, 4, 1, 0, 0, 8, 8, 8};
            if (elem <= SLHIP_GGUF_FLOAT64 && kSize[elem] > 0) {
                n.data = count ? c.take(count * kSize[elem]) : c.base + c.pos;
            } else if (elem == SLHIP_GGUF_STRING || elem == SLHIP_GGUF_ARRAY) {
                // each element needs at least its length prefix (or type + count): absurd counts fail here,
                // before anything is allocated for them
                if (count * (elem == SLHIP_GGUF_STRING ? kMinStringBytes : kMinArrayBytes) > c.remaining())
                    format_error(elem == SLHIP_GGUF_STRING ? "String array larger than file." : "Array larger than file.");
                const int64_t first = static_cast<int64_t>(nodes.size());
                nodes.resize(nodes.size() + static_cast<size_t>(count));
                for (int64_t k = 0; k < count; k++) {
                    if (elem == SLHIP_GGUF_STRING) {
                        Node s;
                        read_string(c, s);
                        nodes[first + k] = s;
                    } else {
                        read_value(c, SLHIP_GGUF_ARRAY, first + k, depth + 1);
                    }
                }
                n.first_child = first;
            } else {
                format_error("Unknown GGUF array element type " + std::to_string(elem) + ".");
            }
            break;
        }
        default: format_error("Unknown GGUF value type " + std::to_string(type) + ".");
        }
        nodes[id] = n;
    }

    void read_pair(Cursor& c)
    {
        std::string key = read_key(c);
        const uint32_t type = c.read<uint32_t>();
        const int64_t id = static_cast<int64_t>(nodes.size());
        nodes.emplace_back();
        read_value(c, type, id);
        kv_index[key] = static_cast<int64_t>(kv.size());
        kv.emplace_back(std::move(key), id);
    }

    // GgufFile.ReadTensorHeaders (GgufFile.cs:150-177): name, dims, type, offset.
    void read_tensor_entry(Cursor& c, Tensor& t)
    {
        t.name = read_key(c);
        const uint32_t dims = c.read<uint32_t>();
        if (dims > kMaxDims) format_error("Tensor '" + t.name + "' has " + std::to_string(dims) + " dimensions.");
        t.ne.resize(dims);
        for (uint32_t d = 0; d < dims; d++) t.ne[d] = c.read_len();
        t.ggml = static_cast<int>(c.read<uint32_t>());
        t.rel = c.read_len();
    }

    // general.alignment when present and positive (GgufFile.cs:135-148)
    void read_alignment()
    {
        auto it = kv_index.find("general.alignment");
        if (it == kv_index.end()) return;
        const Node& n = nodes[kv[it->second].second];
        int64_t v;
        switch (n.type) {
        case SLHIP_GGUF_UINT8: case SLHIP_GGUF_UINT16: case SLHIP_GGUF_UINT32: case SLHIP_GGUF_UINT64: case SLHIP_GGUF_BOOL:
            if (n.u > static_cast<uint64_t>(kIntMax)) format_error("Value was either too large or too small for an Int32.");
            v = static_cast<int64_t>(n.u);
            break;
        case SLHIP_GGUF_INT8: case SLHIP_GGUF_INT16: case SLHIP_GGUF_INT32: case SLHIP_GGUF_INT64:
            if (n.i > kIntMax || n.i < -kIntMax - 1) format_error("Value was either too large or too small for an Int32.");
            v = n.i;
            break;
        case SLHIP_GGUF_FLOAT32: case SLHIP_GGUF_FLOAT64:  // Convert.ToInt32 rounds half to even
            if (!(n.f < 2147483647.5 && n.f >= -2147483648.5)) format_error("Value was either too large or too small for an Int32.");
            v = static_cast<int64_t>(std::nearbyint(n.f));
            break;
        default: return;
        }
        if (v > 0) alignment = static_cast<uint32_t>(v);
    }

    void parse_file()
    {
        Cursor c{base, length};
        if (c.read<uint32_t>() != kMagic) format_error("Not a GGUF file (bad magic).");
        version = c.read<uint32_t>();
        if (version != 2 && version != 3) unsupported("Unsupported GGUF version " + std::to_string(version) + ".");
        const int64_t n_tensors = c.read_len(), n_kv = c.read_len();
        if (n_tensors > length || n_kv > length) format_error("Implausible tensor/KV count.");
        for (int64_t k = 0; k < n_kv; k++) read_pair(c);
        read_alignment();
        tensors.resize(static_cast<size_t>(n_tensors));
        for (auto& t : tensors) read_tensor_entry(c, t);
        data_offset = (c.pos + alignment - 1) / alignment * alignment;
        table_complete = true;
        // GgufFile.BuildTensorTable (GgufFile.cs:179-205)
        for (size_t k = 0; k < tensors.size(); k++) {
            Tensor& t = tensors[k];
            t.desc = type_desc(t.ggml);
            if (!t.desc.name) unsupported("Unsupported ggml tensor type id " + std::to_string(t.ggml) + ".");
            t.size = compute_byte_size(t.desc, t.ne, t.name);
            if (t.desc.layout == Layout::InterleavedQ4_0) {
                const int64_t rows = t.size / t.desc.block_bytes * t.desc.block_size / std::max<int64_t>(1, t.ne.empty() ? 1 : t.ne[0]);
                if (rows % t.desc.rows != 0)
                    format_error("Tensor '" + t.name + "': " + std::to_string(rows) + " rows are not a multiple of the " +
                                 std::to_string(t.desc.rows) + " rows its type interleaves.");
            }
            t.stored = stored_byte_size(t.desc, t.size);
            if (__builtin_add_overflow(data_offset, t.rel, &t.abs) || t.abs < 0 || t.stored > length - t.abs)
                format_error("Tensor '" + t.name + "' extends beyond the end of the file (offset " + std::to_string(t.abs) +
                             ", size " + std::to_string(t.stored) + ", file " + std::to_string(length) + ").");
            by_name[t.name] = static_cast<int64_t>(k);
        }
    }

    // GgufHeaderProbe.ReadMetadata + ReadTensorTable: keep what the prefix holds whole.
    void parse_prefix()
    {
        if (length < kHeaderBytes) return;
        Cursor c{base, length};
        if (c.read<uint32_t>() != kMagic) return;
        const uint32_t v = c.read<uint32_t>();
        if (v != 2 && v != 3) return;
        version = v;
        const uint64_t n_tensors = c.read<uint64_t>(), n_kv_raw = c.read<uint64_t>();
        const int64_t n_kv = static_cast<int64_t>(std::min<uint64_t>(n_kv_raw, kIntMax));
        bool kv_whole = true;
        for (int64_t k = 0; k < n_kv; k++) {
            const size_t nodes_before = nodes.size(), kv_before = kv.size();
            try {
                read_pair(c);
            } catch (const GgufError&) {  // the prefix ends inside this pair: keep what was read
                nodes.resize(nodes_before);
                if (kv.size() > kv_before) kv.resize(kv_before);
                kv_whole = false;
                break;
            }
        }
        for (size_t k = 0; k < kv.size(); k++) kv_index[kv[k].first] = static_cast<int64_t>(k);
        try {
            read_alignment();
        } catch (const GgufError&) {
        }
        // the table needs every pair first; it is kept only when read to its end
        if (!kv_whole || n_kv_raw > static_cast<uint64_t>(length) || n_tensors > static_cast<uint64_t>(length)) return;
        std::vector<Tensor> table(static_cast<size_t>(n_tensors));
        try {
            for (auto& t : table) read_tensor_entry(c, t);
        } catch (const GgufError&) {
            return;
        }
        data_offset = (c.pos + alignment - 1) / alignment * alignment;
        for (size_t k = 0; k < table.size(); k++) {
            Tensor& t = table[k];
            t.desc = type_desc(t.ggml);
            if (t.desc.name) {
                try {
                    t.size = compute_byte_size(t.desc, t.ne, t.name);
                    t.stored = stored_byte_size(t.desc, t.size);
                } catch (const GgufError&) {
                    t.size = t.stored = 0;
                }
            }
            by_name[t.name] = static_cast<int64_t>(k);
        }
        tensors = std::move(table);
        table_complete = true;
    }
};

namespace {

template <typename F> int guarded(F&& f)
{
    try {
        return f();
    } catch (const GgufError& e) {
        return fail(e.status, "%s", e.message.c_str());
    } catch (const std::bad_alloc&) {
        return fail(SLHIP_ERR_INVALID, "out of host memory while reading the GGUF file");
    }
}

void fill_tensor(const Tensor& t, slhip_gguf_tensor* o)
{
    std::memset(o, 0, sizeof(*o));
    o->name = t.name.c_str();
    o->type_name = t.desc.name ? t.desc.name : "";
    o->ggml_type = t.ggml;
    o->format = t.desc.format;
    o->block_size = t.desc.block_size;
    o->block_bytes = t.desc.block_bytes;
    o->n_dims = static_cast<int32_t>(t.ne.size());
    for (size_t d = 0; d < t.ne.size(); d++) o->ne[d] = t.ne[d];
    o->relative_offset = t.rel;
    o->offset = t.abs;
    o->byte_size = t.size;
    o->stored_bytes = t.stored;
}

// One narrow IQ1 block (46, 42 or 38 bytes) as the IQ1_S block (50 bytes) with the same values
// (GgmlNarrowIq1.Widen, GgmlNarrowIq1.cs:55-86): the f16 scale and the 32 low index bytes carry over with
// each group's index replaced by its IQ1_S grid position; per 32 values the u16 qh holds the three high
// position bits of each group, the 3-bit scale (bits 12-14) and the delta sign (bit 15).
//   IQ1_XS  (64): f16 d, qs[32], qh[8] (group l's two high index bits at 2l), sc[4] (a nibble per 32 values)
//   IQ1_XXS (65): f16 d, qs[32], qh[8] (bit l: group l's ninth index bit; bits 4-7: scale and sign)
//   IQ1_XXXS(66): f16 d, qs[32] (whole 8-bit indices), sc[4]
void widen_narrow_iq1(int ggml, const uint8_t* narrow, uint8_t* wide)
{
    const uint16_t* grid = ggml == 64 ? kNarrowIq1Xs : ggml == 65 ? kNarrowIq1Xxs : kNarrowIq1Xxxs;
    wide[0] = narrow[0];
    wide[1] = narrow[1];
    const uint8_t* qs = narrow + 2;
    const uint8_t* tail = narrow + 34;
    for (int ib = 0; ib < 8; ib++) {
        const int ss = ggml == 65 ? tail[ib] >> 4 : (tail[ggml == 64 ? 8 + ib / 2 : ib / 2] >> (4 * (ib & 1))) & 0xF;
        int qh = (ss & 7) << 12 | (ss >> 3) << 15;
        for (int l = 0; l < 4; l++) {
            const int high = ggml == 64 ? (tail[ib] >> (2 * l)) & 3 : ggml == 65 ? (tail[ib] >> l) & 1 : 0;
            const int index = grid[qs[4 * ib + l] | high << 8];
            wide[2 + 4 * ib + l] = static_cast<uint8_t>(index);
            qh |= (index >> 8) << (3 * l);
        }
        wide[34 + 2 * ib] = static_cast<uint8_t>(qh);
        wide[35 + 2 * ib] = static_cast<uint8_t>(qh >> 8);
    }
}

// IWeightSource.Read of [off, off + n) of tensor t into dst. The range was checked by the caller.
void read_range(const slhip_gguf& g, const Tensor& t, int64_t off, uint8_t* dst, int64_t n)
{
    const uint8_t* data = g.base + t.abs;
    if (n <= 0) return;
    switch (t.desc.layout) {
    case Layout::Plain: std::memcpy(dst, data + off, static_cast<size_t>(n)); return;
    case Layout::InterleavedQ4_0: {
        // R rows per group, block column by block column: the R f16 scales, then the R 16-byte nibble arrays
        // cut into `chunk`-byte pieces interleaved row by row, each byte XOR 0x88 (GgufInterleavedQ4_0Source.cs:43-79)
        const int R = t.desc.rows, C = t.desc.chunk;
        const int64_t bpr = t.ne[0] / 32;
        uint8_t block[18];
        const int64_t end = off + n;
        for (int64_t b = off / 18; b * 18 < end; b++) {
            const int64_t row = b / bpr, col = b % bpr;
            const int w = static_cast<int>(row % R);
            const uint8_t* grp = data + ((row / R) * bpr + col) * R * 18;
            block[0] = grp[2 * w];
            block[1] = grp[2 * w + 1];
            const uint8_t* nib = grp + 2 * R;
            for (int piece = 0; piece < 16 / C; piece++) {
                const uint8_t* s = nib + (piece * R + w) * C;
                for (int i = 0; i < C; i++) block[2 + piece * C + i] = s[i] ^ 0x88;
            }
            const int64_t bs = b * 18;
            const int64_t from = std::max<int64_t>(0, off - bs), to = std::min<int64_t>(18, end - bs);
            std::memcpy(dst + (bs + from - off), block + from, static_cast<size_t>(to - from));
        }
        return;
    }
    case Layout::I2S: {
        // n/4 code bytes (32 per 128 values), then one f32 scale for the tensor; each block read here is
        // that scale followed by the group's 32 code bytes (GgufI2sSource.cs:11-64)
        const int64_t blocks = t.size / kI2sBlock;
        uint8_t block[kI2sBlock];
        std::memcpy(block, data + blocks * kI2sCodes, 4);
        const int64_t end = off + n;
        for (int64_t b = off / kI2sBlock; b * kI2sBlock < end; b++) {
            std::memcpy(block + 4, data + b * kI2sCodes, kI2sCodes);
            const int64_t bs = b * kI2sBlock;
            const int64_t from = std::max<int64_t>(0, off - bs), to = std::min<int64_t>(kI2sBlock, end - bs);
            std::memcpy(dst + (bs + from - off), block + from, static_cast<size_t>(to - from));
        }
        return;
    }
    case Layout::NarrowIq1: {  // GgufNarrowIq1Source: each stored block widened to IQ1_S
        const int sb = t.desc.stored_block;
        uint8_t block[kWideIq1Bytes];
        const int64_t end = off + n;
        for (int64_t b = off / kWideIq1Bytes; b * kWideIq1Bytes < end; b++) {
            widen_narrow_iq1(t.ggml, data + b * sb, block);
            const int64_t bs = b * kWideIq1Bytes;
            const int64_t from = std::max<int64_t>(0, off - bs), to = std::min<int64_t>(kWideIq1Bytes, end - bs);
            std::memcpy(dst + (bs + from - off), block + from, static_cast<size_t>(to - from));
        }
        return;
    }
    }
}

int check_tensor(const slhip_gguf* g, int64_t index, const Tensor** t)
{
    if (!g) return fail(SLHIP_ERR_INVALID, "null GGUF handle");
    if (index < 0 || index >= static_cast<int64_t>(g->tensors.size()))
        return fail(SLHIP_ERR_INDEX, "tensor index %lld outside [0, %zu)", static_cast<long long>(index), g->tensors.size());
    *t = &g->tensors[static_cast<size_t>(index)];
    return SLHIP_OK;
}

int check_readable(const slhip_gguf* g, const Tensor& t)
{
    if (!g->has_data) return fail(SLHIP_ERR_INVALID, "tensor '%s': a header prefix holds no tensor data", t.name.c_str());
    return SLHIP_OK;
}

// ---- the uploader -------------------------------------------------------------------------------

int env_int(const char* name, int dflt)
{
    const char* s = getenv(name);
    return s && *s ? atoi(s) : dflt;
}

// Two pinned staging buffers of one device: host threads fill one while the DMA engine drains the other.
struct Uploader {
    std::mutex mu;
    size_t size = 0;
    uint8_t* staging[2] = {nullptr, nullptr};
    hipEvent_t done[2] = {nullptr, nullptr};
    int threads = 8;

    // (Re)sizes the staging buffers to SLHIP_UPLOAD_STAGING_MB, read on every call so that a process can
    // change it between uploads; the old buffers are freed once the copies that read them have finished.
    int configure()
    {
        const size_t want = static_cast<size_t>(std::max(1, std::min(4096, env_int("SLHIP_UPLOAD_STAGING_MB", 64)))) << 20;
        threads = std::max(1, std::min(64, env_int("SLHIP_UPLOAD_THREADS", 8)));
        if (want == size) return SLHIP_OK;
        for (int s = 0; s < 2; s++) {
            if (done[s]) SLHIP_CHECK_HIP(hipEventSynchronize(done[s]));
            if (staging[s]) SLHIP_CHECK_HIP(hipHostFree(staging[s]));
            staging[s] = nullptr;
        }
        size = 0;
        for (int s = 0; s < 2; s++) {
            SLHIP_CHECK_HIP(hipHostMalloc(reinterpret_cast<void**>(&staging[s]), want, hipHostMallocDefault));
            if (!done[s]) SLHIP_CHECK_HIP(hipEventCreateWithFlags(&done[s], hipEventDisableTiming));
        }
        size = want;
        return SLHIP_OK;
    }

    // fill(off, dst, n) writes source bytes [off, off + n) to dst.
    template <typename Fill> int run(uint8_t* dst, int64_t total, Fill&& fill, hipStream_t stream)
    {
        std::lock_guard<std::mutex> lock(mu);
        const int r = configure();
        if (r != SLHIP_OK) return r;
        int slot = 0;
        for (int64_t off = 0; off < total; off += static_cast<int64_t>(size), slot ^= 1) {
            const int64_t n = std::min<int64_t>(static_cast<int64_t>(size), total - off);
            SLHIP_CHECK_HIP(hipEventSynchronize(done[slot]));  // the copy that last read this buffer
            uint8_t* buf = staging[slot];
            const int nt = n >= (4 << 20) ? threads : 1;
            if (nt == 1) {
                fill(off, buf, n);
            } else {
                const int64_t part = ((n + nt - 1) / nt + 4095) / 4096 * 4096;
                std::vector<std::thread> pool;
                for (int k = 0; k < nt; k++) {
                    const int64_t a = k * part, b = std::min<int64_t>(n, a + part);
                    if (a >= b) break;
                    pool.emplace_back([&, a, b] { fill(off + a, buf + a, b - a); });
                }
                for (auto& th : pool) th.join();
            }
            SLHIP_CHECK_HIP(hipMemcpyAsync(dst + off, buf, static_cast<size_t>(n), hipMemcpyHostToDevice, stream));
            SLHIP_CHECK_HIP(hipEventRecord(done[slot], stream));
        }
        return SLHIP_OK;
    }
};

int uploader(Uploader** out)
{
    static std::mutex mu;
    static std::map<int, Uploader*> per_device;  // kept until the process ends
    int dev = 0;
    SLHIP_CHECK_HIP(hipGetDevice(&dev));
    std::lock_guard<std::mutex> lock(mu);
    auto it = per_device.find(dev);
    if (it != per_device.end()) {
        *out = it->second;
        return SLHIP_OK;
    }
    auto* u = new Uploader();  // staging is sized by its first run
    per_device[dev] = u;
    *out = u;
    return SLHIP_OK;
}

}  // namespace

// ---- C ABI ------------------------------------------------------------------------------------------

SLHIP_API int slhip_gguf_open(const char* path, slhip_gguf** file)
{
    if (!path || !file) return fail(SLHIP_ERR_INVALID, "null argument");
    *file = nullptr;
    auto* g = new slhip_gguf();
    const int r = guarded([&]() -> int {
        g->fd = open(path, O_RDONLY | O_CLOEXEC);
        if (g->fd < 0) return fail(SLHIP_ERR_INVALID, "cannot open '%s': %s", path, strerror(errno));
        struct stat st;
        if (fstat(g->fd, &st) != 0) return fail(SLHIP_ERR_INVALID, "cannot stat '%s': %s", path, strerror(errno));
        g->length = static_cast<int64_t>(st.st_size);
        if (g->length < kHeaderBytes) format_error("File too small to be GGUF.");
        void* m = mmap(nullptr, static_cast<size_t>(g->length), PROT_READ, MAP_SHARED, g->fd, 0);
        if (m == MAP_FAILED) return fail(SLHIP_ERR_INVALID, "cannot map '%s': %s", path, strerror(errno));
        g->base = static_cast<const uint8_t*>(m);
        g->has_data = true;
        g->parse_file();
        return SLHIP_OK;
    });
    if (r != SLHIP_OK) {
        delete g;
        return r;
    }
    *file = g;
    return SLHIP_OK;
}

SLHIP_API int slhip_gguf_open_prefix(const void* bytes, size_t length, slhip_gguf** file)
{
    if (!file || (!bytes && length)) return fail(SLHIP_ERR_INVALID, "null argument");
    *file = nullptr;
    auto* g = new slhip_gguf();
    const int r = guarded([&]() -> int {
        g->copy.assign(static_cast<const uint8_t*>(bytes), static_cast<const uint8_t*>(bytes) + length);
        g->base = g->copy.data();
        g->length = static_cast<int64_t>(length);
        g->parse_prefix();
        return SLHIP_OK;
    });
    if (r != SLHIP_OK) {
        delete g;
        return r;
    }
    *file = g;
    return SLHIP_OK;
}

SLHIP_API int slhip_gguf_close(slhip_gguf* file)
{
    delete file;
    return SLHIP_OK;
}

SLHIP_API int slhip_gguf_get_info(const slhip_gguf* g, slhip_gguf_info* info)
{
    if (!g || !info) return fail(SLHIP_ERR_INVALID, "null argument");
    info->version = g->version;
    info->alignment = g->alignment;
    info->n_tensors = static_cast<int64_t>(g->tensors.size());
    info->n_kv = static_cast<int64_t>(g->kv.size());
    info->data_offset = g->data_offset;
    info->file_length = g->length;
    info->has_data = g->has_data;
    info->table_complete = g->table_complete;
    return SLHIP_OK;
}

SLHIP_API int slhip_gguf_kv(const slhip_gguf* g, int64_t index, const char** key, int64_t* node)
{
    if (!g || !key || !node) return fail(SLHIP_ERR_INVALID, "null argument");
    if (index < 0 || index >= static_cast<int64_t>(g->kv.size()))
        return fail(SLHIP_ERR_INDEX, "metadata index %lld outside [0, %zu)", static_cast<long long>(index), g->kv.size());
    *key = g->kv[static_cast<size_t>(index)].first.c_str();
    *node = g->kv[static_cast<size_t>(index)].second;
    return SLHIP_OK;
}

SLHIP_API int slhip_gguf_find_kv(const slhip_gguf* g, const char* key, int64_t* index)
{
    if (!g || !key || !index) return fail(SLHIP_ERR_INVALID, "null argument");
    auto it = g->kv_index.find(key);
    *index = it == g->kv_index.end() ? -1 : it->second;
    return SLHIP_OK;
}

SLHIP_API int slhip_gguf_get_value(const slhip_gguf* g, int64_t node, slhip_gguf_value* v)
{
    if (!g || !v) return fail(SLHIP_ERR_INVALID, "null argument");
    if (node < 0 || node >= static_cast<int64_t>(g->nodes.size()))
        return fail(SLHIP_ERR_INDEX, "value node %lld outside [0, %zu)", static_cast<long long>(node), g->nodes.size());
    const Node& n = g->nodes[static_cast<size_t>(node)];
    v->type = n.type;
    v->elem_type = n.elem;
    v->count = n.count;
    v->u = n.u;
    v->i = n.i;
    v->f = n.f;
    v->data = n.data;
    v->first_child = n.first_child;
    return SLHIP_OK;
}

SLHIP_API int slhip_gguf_tensor_info(const slhip_gguf* g, int64_t index, slhip_gguf_tensor* out)
{
    const Tensor* t;
    const int r = check_tensor(g, index, &t);
    if (r != SLHIP_OK) return r;
    if (!out) return fail(SLHIP_ERR_INVALID, "null argument");
    fill_tensor(*t, out);
    return SLHIP_OK;
}

SLHIP_API int slhip_gguf_find_tensor(const slhip_gguf* g, const char* name, int64_t* index)
{
    if (!g || !name || !index) return fail(SLHIP_ERR_INVALID, "null argument");
    auto it = g->by_name.find(name);
    *index = it == g->by_name.end() ? -1 : it->second;
    return SLHIP_OK;
}

SLHIP_API int slhip_gguf_type(int ggml_type, slhip_gguf_tensor* out)
{
    if (!out) return fail(SLHIP_ERR_INVALID, "null argument");
    Tensor t;
    t.desc = type_desc(ggml_type);
    if (!t.desc.name) return fail(SLHIP_ERR_UNSUPPORTED, "Unsupported ggml tensor type id %d.", ggml_type);
    t.ggml = ggml_type;
    fill_tensor(t, out);
    out->name = "";
    return SLHIP_OK;
}

SLHIP_API int slhip_gguf_read(const slhip_gguf* g, int64_t index, int64_t offset, void* dst, size_t bytes)
{
    const Tensor* t;
    int r = check_tensor(g, index, &t);
    if (r != SLHIP_OK) return r;
    if ((r = check_readable(g, *t)) != SLHIP_OK) return r;
    if (!dst && bytes) return fail(SLHIP_ERR_INVALID, "null destination");
    const int64_t n = static_cast<int64_t>(bytes);
    if (offset < 0 || n < 0 || n > t->size - offset)
        return fail(SLHIP_ERR_INDEX, "range [%lld, +%lld) outside tensor '%s' of %lld bytes", static_cast<long long>(offset),
                    static_cast<long long>(n), t->name.c_str(), static_cast<long long>(t->size));
    read_range(*g, *t, offset, static_cast<uint8_t*>(dst), n);
    return SLHIP_OK;
}

SLHIP_API int slhip_gguf_tensor_pointer(const slhip_gguf* g, int64_t index, const void** ptr)
{
    const Tensor* t;
    const int r = check_tensor(g, index, &t);
    if (r != SLHIP_OK) return r;
    if (!ptr) return fail(SLHIP_ERR_INVALID, "null argument");
    *ptr = g->has_data && t->desc.layout == Layout::Plain ? g->base + t->abs : nullptr;
    return SLHIP_OK;
}

SLHIP_API int slhip_gguf_upload(const slhip_gguf* g, int64_t index, void* dst, size_t dst_bytes, slhip_stream stream)
{
    const Tensor* t;
    int r = check_tensor(g, index, &t);
    if (r != SLHIP_OK) return r;
    if ((r = check_readable(g, *t)) != SLHIP_OK) return r;
    if (!dst && t->size) return fail(SLHIP_ERR_INVALID, "null destination");
    if (static_cast<int64_t>(dst_bytes) < t->size)
        return fail(SLHIP_ERR_INVALID, "tensor '%s' needs %lld bytes, destination holds %zu", t->name.c_str(),
                    static_cast<long long>(t->size), dst_bytes);
    Uploader* u;
    if ((r = uploader(&u)) != SLHIP_OK) return r;
    const slhip_gguf& gg = *g;
    const Tensor& tt = *t;
    return u->run(static_cast<uint8_t*>(dst), t->size,
                  [&gg, &tt](int64_t off, uint8_t* out, int64_t n) { read_range(gg, tt, off, out, n); },
                  static_cast<hipStream_t>(stream));
}

SLHIP_API int slhip_upload(void* dst, const void* src, size_t bytes, slhip_stream stream)
{
    if (!bytes) return SLHIP_OK;
    if (!dst || !src) return fail(SLHIP_ERR_INVALID, "null argument");
    Uploader* u;
    const int r = uploader(&u);
    if (r != SLHIP_OK) return r;
    const uint8_t* s = static_cast<const uint8_t*>(src);
    return u->run(static_cast<uint8_t*>(dst), static_cast<int64_t>(bytes),
                  [s](int64_t off, uint8_t* out, int64_t n) { std::memcpy(out, s + off, static_cast<size_t>(n)); },
                  static_cast<hipStream_t>(stream));
}
