// gguf.cpp -- GGUF v3 reader (the container of adi::GgufFile, src/gguf.cpp)
// and the upload of one layer's packed MoE tensors into device descriptors
// (the tensor mapping of adi::MachModel, src/model.cpp:267-314, 431-533,
// 808-880). Host code; it runs no kernel.
//
// The file is mapped read-only and indexed once: metadata entries and tensor
// infos are kept as views into the mapping, with hash indexes for lookups (a
// checkpoint carries thousands of mach.* tensors). Every read goes through a
// bounds-checked cursor, so a truncated or inconsistent file is rejected at
// open with a message rather than read past its end.
#include "adi_hip_gguf.h"
#include "context.hpp"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cstring>
#include <limits>
#include <stdexcept>
#include <string>
#include <string_view>
#include <unordered_map>

namespace adi_hip {
namespace {

thread_local std::string g_gguf_error;

// GGUF metadata value types (include/adi/gguf.hpp:13-27).
enum ValueType : uint32_t {
    kU8 = 0, kI8 = 1, kU16 = 2, kI16 = 3, kU32 = 4, kI32 = 5, kF32 = 6, kBool = 7,
    kString = 8, kArray = 9, kU64 = 10, kI64 = 11, kF64 = 12,
};

// Malformed files and tensors are argument errors, as the reference's
// std::runtime_error at load time (src/gguf.cpp:29-31, src/model.cpp).
[[noreturn]] void gguf_fail(const std::string &message) {
    fail(ADI_HIP_INVALID_ARGUMENT, "GGUF: " + message);
}

uint64_t scalar_bytes(uint32_t type) {
    switch (type) {
    case kU8: case kI8: case kBool: return 1;
    case kU16: case kI16: return 2;
    case kU32: case kI32: case kF32: return 4;
    case kU64: case kI64: case kF64: return 8;
    default: return 0;
    }
}

uint64_t element_bytes(uint32_t ggml_type) {
    switch (ggml_type) {
    case ADI_HIP_GGML_I8: return 1;
    case ADI_HIP_GGML_F16: case ADI_HIP_GGML_I16: case ADI_HIP_GGML_BF16: return 2;
    case ADI_HIP_GGML_F32: case ADI_HIP_GGML_I32: return 4;
    case ADI_HIP_GGML_I64: case ADI_HIP_GGML_F64: return 8;
    default: return 0;
    }
}

// Little-endian reads bounded by the mapping.
class Reader {
  public:
    Reader(const uint8_t *data, uint64_t size, uint64_t at = 0) : data_(data), size_(size), at_(at) {}

    template <typename T>
    T get() {
        need(sizeof(T));
        T value;
        std::memcpy(&value, data_ + at_, sizeof(T));
        at_ += sizeof(T);
        return value;
    }
    std::string_view text() {
        const uint64_t length = get<uint64_t>();
        need(length);
        std::string_view s(reinterpret_cast<const char *>(data_ + at_), static_cast<size_t>(length));
        at_ += length;
        return s;
    }
    void skip(uint64_t bytes) {
        need(bytes);
        at_ += bytes;
    }
    uint32_t value_type() {
        const uint32_t type = get<uint32_t>();
        if (type > kF64) {
            gguf_fail("unknown metadata value type " + std::to_string(type));
        }
        return type;
    }
    // Skips one value of `type`, arrays element by element.
    void skip_value(uint32_t type, unsigned depth = 0) {
        if (depth > 8) {
            gguf_fail("metadata arrays are nested too deeply");
        }
        if (const uint64_t n = scalar_bytes(type)) {
            skip(n);
        } else if (type == kString) {
            (void)text();
        } else {
            const uint32_t element = value_type();
            const uint64_t count = get<uint64_t>();
            if (const uint64_t n = scalar_bytes(element)) {
                if (count > std::numeric_limits<uint64_t>::max() / n) {
                    gguf_fail("metadata array size overflows");
                }
                skip(count * n);
            } else {
                for (uint64_t i = 0; i < count; ++i) {
                    skip_value(element, depth + 1);
                }
            }
        }
    }
    uint64_t at() const { return at_; }
    uint64_t left() const { return size_ - at_; }

  private:
    void need(uint64_t bytes) const {
        if (bytes > size_ || at_ > size_ - bytes) {
            gguf_fail("truncated file at byte " + std::to_string(at_));
        }
    }
    const uint8_t *data_;
    uint64_t size_;
    uint64_t at_;
};

}  // namespace
}  // namespace adi_hip

using namespace adi_hip;

struct adi_hip_gguf {
    struct Entry {
        uint32_t type;
        uint64_t value_at;  // offset of the value in the file
    };
    int fd = -1;
    const uint8_t *map = nullptr;
    uint64_t size = 0;
    uint32_t version = 0;
    uint64_t alignment = 32;
    uint64_t metadata_count = 0;
    std::unordered_map<std::string_view, Entry> metadata;
    std::unordered_map<std::string_view, adi_hip_gguf_tensor> tensors;

    ~adi_hip_gguf() {
        if (map != nullptr) {
            ::munmap(const_cast<uint8_t *>(map), size);
        }
        if (fd >= 0) {
            ::close(fd);
        }
    }

    const Entry *entry(const char *key) const {
        if (key == nullptr) {
            return nullptr;
        }
        const auto it = metadata.find(std::string_view(key));
        return it == metadata.end() ? nullptr : &it->second;
    }
    Reader reader(uint64_t at) const { return Reader(map, size, at); }

    void open(const char *path) {
        fd = ::open(path, O_RDONLY | O_CLOEXEC);
        if (fd < 0) {
            fail(ADI_HIP_INVALID_ARGUMENT, std::string("cannot open '") + path + "': " + std::strerror(errno));
        }
        struct stat st {};
        if (::fstat(fd, &st) != 0) {
            fail(ADI_HIP_INVALID_ARGUMENT, std::string("cannot stat '") + path + "': " + std::strerror(errno));
        }
        if (st.st_size < 24) {
            gguf_fail("file is too small");
        }
        size = static_cast<uint64_t>(st.st_size);
        void *m = ::mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0);
        if (m == MAP_FAILED) {
            fail(ADI_HIP_INVALID_ARGUMENT, std::string("cannot mmap '") + path + "': " + std::strerror(errno));
        }
        map = static_cast<const uint8_t *>(m);
        parse();
    }

    // The header, the metadata directory and the tensor infos
    // (src/gguf.cpp:270-324).
    void parse() {
        Reader r = reader(0);
        if (r.get<uint32_t>() != 0x46554747u) {
            gguf_fail("bad magic");
        }
        version = r.get<uint32_t>();
        if (version != 3) {
            gguf_fail("only version 3 is supported");
        }
        const uint64_t tensor_count = r.get<uint64_t>();
        metadata_count = r.get<uint64_t>();
        if (tensor_count > r.left() || metadata_count > r.left()) {
            gguf_fail("directory count exceeds file size");
        }
        metadata.reserve(static_cast<size_t>(metadata_count));
        for (uint64_t i = 0; i < metadata_count; ++i) {
            const std::string_view key = r.text();
            const uint32_t type = r.value_type();
            if (!metadata.emplace(key, Entry{type, r.at()}).second) {
                gguf_fail("duplicate metadata key '" + std::string(key) + "'");
            }
            r.skip_value(type);
        }
        uint64_t align = 0;
        if (integer("general.alignment", align)) {
            if (align == 0 || (align & (align - 1)) != 0) {
                gguf_fail("general.alignment must be a non-zero power of two");
            }
            alignment = align;
        }
        tensors.reserve(static_cast<size_t>(tensor_count));
        std::vector<std::string_view> order;
        order.reserve(static_cast<size_t>(tensor_count));
        for (uint64_t i = 0; i < tensor_count; ++i) {
            const std::string_view name = r.text();
            adi_hip_gguf_tensor t{};
            t.dimension_count = r.get<uint32_t>();
            if (t.dimension_count == 0 || t.dimension_count > 4) {
                gguf_fail("tensor has unsupported dimension count");
            }
            t.elements = 1;
            for (uint32_t d = 0; d < t.dimension_count; ++d) {
                const uint64_t extent = r.get<uint64_t>();
                if (extent == 0 || t.elements > std::numeric_limits<uint64_t>::max() / extent) {
                    gguf_fail("invalid tensor dimensions");
                }
                t.dimensions[d] = extent;
                t.elements *= extent;
            }
            t.type = r.get<uint32_t>();
            const uint64_t offset = r.get<uint64_t>();
            const uint64_t per = element_bytes(t.type);
            if (per == 0) {
                gguf_fail("unsupported tensor type " + std::to_string(t.type));
            }
            if (t.elements > std::numeric_limits<uint64_t>::max() / per) {
                gguf_fail("tensor byte size overflows");
            }
            t.bytes = t.elements * per;
            // offset is relative to the data section until the directory ends
            t.data = reinterpret_cast<const void *>(static_cast<uintptr_t>(offset));
            if (!tensors.emplace(name, t).second) {
                gguf_fail("duplicate tensor name '" + std::string(name) + "'");
            }
        }
        const uint64_t mask = alignment - 1;
        if (r.at() > std::numeric_limits<uint64_t>::max() - mask) {
            gguf_fail("alignment overflows");
        }
        const uint64_t data_start = (r.at() + mask) & ~mask;
        if (data_start > size) {
            gguf_fail("tensor data begins outside file");
        }
        for (auto &kv : tensors) {
            adi_hip_gguf_tensor &t = kv.second;
            const uint64_t offset = static_cast<uint64_t>(reinterpret_cast<uintptr_t>(t.data));
            if (offset > size - data_start || t.bytes > size - data_start - offset) {
                gguf_fail("range points outside file");
            }
            t.data = map + data_start + offset;
        }
    }

    // GgufFile::integer (src/gguf.cpp:427-461).
    bool integer(const char *key, uint64_t &out) const {
        const Entry *e = entry(key);
        if (e == nullptr || scalar_bytes(e->type) == 0) {
            return false;
        }
        Reader r = reader(e->value_at);
        switch (e->type) {
        case kU8: out = r.get<uint8_t>(); return true;
        case kU16: out = r.get<uint16_t>(); return true;
        case kU32: out = r.get<uint32_t>(); return true;
        case kU64: out = r.get<uint64_t>(); return true;
        case kI8: { const int8_t v = r.get<int8_t>(); out = static_cast<uint64_t>(v); return v >= 0; }
        case kI16: { const int16_t v = r.get<int16_t>(); out = static_cast<uint64_t>(v); return v >= 0; }
        case kI32: { const int32_t v = r.get<int32_t>(); out = static_cast<uint64_t>(v); return v >= 0; }
        case kI64: { const int64_t v = r.get<int64_t>(); out = static_cast<uint64_t>(v); return v >= 0; }
        default: return false;
        }
    }
    // GgufFile::number (src/gguf.cpp:463-478).
    bool number(const char *key, double &out) const {
        const Entry *e = entry(key);
        if (e == nullptr) {
            return false;
        }
        if (e->type == kF32) {
            out = reader(e->value_at).get<float>();
            return true;
        }
        if (e->type == kF64) {
            out = reader(e->value_at).get<double>();
            return true;
        }
        uint64_t v = 0;
        if (integer(key, v)) {
            out = static_cast<double>(v);
            return true;
        }
        return false;
    }
    bool boolean(const char *key, bool &out) const {
        const Entry *e = entry(key);
        if (e == nullptr || e->type != kBool) {
            return false;
        }
        out = reader(e->value_at).get<uint8_t>() != 0;
        return true;
    }
    bool string(const char *key, std::string_view &out) const {
        const Entry *e = entry(key);
        if (e == nullptr || e->type != kString) {
            return false;
        }
        Reader r = reader(e->value_at);
        out = r.text();
        return true;
    }
    const adi_hip_gguf_tensor *tensor(const std::string &name) const {
        const auto it = tensors.find(std::string_view(name));
        return it == tensors.end() ? nullptr : &it->second;
    }
};

namespace adi_hip {
namespace {

// Runs a file-level call: exceptions become a status and a message for
// adi_hip_gguf_error().
template <typename F>
int file_call(F &&function) {
    try {
        const int status = function();
        if (status == ADI_HIP_OK) {
            g_gguf_error.clear();
        }
        return status;
    } catch (const Failure &failure) {
        g_gguf_error = failure.message;
        return failure.status;
    } catch (const std::bad_alloc &) {
        g_gguf_error = "host allocation failed";
        return ADI_HIP_OUT_OF_MEMORY;
    } catch (const std::exception &error) {
        g_gguf_error = error.what();
        return ADI_HIP_INVALID_ARGUMENT;
    }
}

int not_found(const std::string &what) {
    g_gguf_error = "GGUF: no " + what;
    return ADI_HIP_NOT_FOUND;
}

// ---- the packed MoE tensors of a checkpoint ---------------------------------

[[noreturn]] void model_fail(const std::string &message) {
    fail(ADI_HIP_INVALID_ARGUMENT, "model: " + message);
}

uint32_t required_u32(const adi_hip_gguf &f, const char *key) {
    uint64_t v = 0;
    if (!f.integer(key, v) || v > 0xFFFFFFFFull) {
        model_fail(std::string("missing or invalid metadata '") + key + "'");
    }
    return static_cast<uint32_t>(v);
}

void require_text(const adi_hip_gguf &f, const char *key, std::string_view expected) {
    std::string_view v;
    if (!f.string(key, v) || v != expected) {
        model_fail(std::string("unsupported metadata '") + key + "'");
    }
}

// required_tensor + the GGUF dims check (src/model.cpp:65-75, 89-104).
const adi_hip_gguf_tensor &required_tensor(const adi_hip_gguf &f, const std::string &name,
                                           uint32_t type,
                                           std::initializer_list<uint64_t> dims) {
    const adi_hip_gguf_tensor *t = f.tensor(name);
    if (t == nullptr || t->type != type) {
        model_fail("missing or invalid tensor '" + name + "'");
    }
    bool same = t->dimension_count == dims.size();
    uint32_t d = 0;
    for (const uint64_t extent : dims) {
        same = same && t->dimensions[d++] == extent;
    }
    if (!same) {
        model_fail("unexpected tensor shape '" + name + "'");
    }
    if (reinterpret_cast<uintptr_t>(t->data) % element_bytes(type) != 0) {
        model_fail("misaligned tensor '" + name + "'");
    }
    return *t;
}

bool finite_f16(uint16_t bits) { return (bits & 0x7C00u) != 0x7C00u; }

// f16 bits to float on the host (finite values: normals and subnormals).
float f16_bits_to_float_host(uint16_t bits) {
    const uint32_t sign = (bits & 0x8000u) << 16;
    const uint32_t exponent = (bits >> 10) & 0x1Fu;
    const uint32_t mantissa = bits & 0x3FFu;
    if (exponent == 0) {
        const float v = std::ldexp(static_cast<float>(mantissa), -24);
        return sign ? -v : v;
    }
    const uint32_t word = sign | ((exponent + 112u) << 23) | (mantissa << 13);
    float v;
    std::memcpy(&v, &word, sizeof(v));
    return v;
}
bool finite_bf16(uint16_t bits) { return (bits & 0x7F80u) != 0x7F80u; }

void require_finite(const adi_hip_gguf_tensor &t, bool (*finite)(uint16_t), const std::string &name) {
    const uint16_t *v = static_cast<const uint16_t *>(t.data);
    for (uint64_t i = 0; i < t.elements; ++i) {
        if (!finite(v[i])) {
            model_fail("nonfinite tensor '" + name + "'");
        }
    }
}

const char *kProjection[3] = {"gate", "up", "down"};

std::string layer_prefix(uint32_t layer) {
    return "model.language_model.layers." + std::to_string(layer) + ".";
}
std::string expert_name(uint32_t layer, uint32_t chunk, int projection, const char *field) {
    return "mach.expert." + std::to_string(layer) + ".e" + std::to_string(chunk) + "." +
           kProjection[projection] + "." + field;
}
std::string shared_name(uint32_t layer, int projection, const char *field) {
    return "mach.ne." + std::to_string(layer) + "." + layer_prefix(layer) + "mlp.shared_expert." +
           kProjection[projection] + "_proj.weight|" + field;
}

bool width_ok(uint32_t n) { return n >= 64 && n <= 8192 && (n & (n - 1)) == 0; }

// Geometry and codec metadata (src/model.cpp:180-224) and the TLUTs
// (src/model.cpp:808-833).
adi_hip_moe_geometry read_geometry(const adi_hip_gguf &f) {
    require_text(f, "general.architecture", "qwen35moe");
    require_text(f, "adi.expert_codec", "trained_susv_wave_gamma_chunked_v1");
    require_text(f, "adi.ne_codec", "canon_rht_bitshift_trellis_intlattice");
    bool additive = false;
    if (!f.boolean("adi.additive", additive) || !additive ||
        required_u32(f, "adi.format_version") != 1 || required_u32(f, "adi.expert.k_num") != 3 ||
        required_u32(f, "adi.expert.k_den") != 2 || required_u32(f, "adi.expert.l") != 16 ||
        required_u32(f, "adi.expert.v") != 8 || required_u32(f, "adi.expert.tlut_bits") != 15 ||
        required_u32(f, "adi.expert.tile_x") != 16 || required_u32(f, "adi.expert.tile_y") != 16) {
        model_fail("unsupported additive format");
    }
    adi_hip_moe_geometry g{};
    g.layers = required_u32(f, "qwen35moe.block_count");
    g.hidden = required_u32(f, "qwen35moe.embedding_length");
    g.experts = required_u32(f, "qwen35moe.expert_count");
    g.active_experts = required_u32(f, "qwen35moe.expert_used_count");
    g.expert_hidden = required_u32(f, "qwen35moe.expert_feed_forward_length");
    g.shared_hidden = required_u32(f, "qwen35moe.expert_shared_feed_forward_length");
    if (g.layers == 0 || g.active_experts != 8 || g.experts < 32 || g.experts % 32 != 0 ||
        g.experts > 1024 || !width_ok(g.hidden) || !width_ok(g.expert_hidden) ||
        g.shared_hidden != g.expert_hidden) {
        model_fail("unsupported MoE geometry");
    }
    const adi_hip_gguf_tensor &et = required_tensor(f, "mach.tlut.expert.tlut", ADI_HIP_GGML_F32, {8, 32768});
    const adi_hip_gguf_tensor &nt = required_tensor(f, "mach.tlut.ne.tlut", ADI_HIP_GGML_F32, {2, 512});
    for (const adi_hip_gguf_tensor *t : {&et, &nt}) {
        const float *v = static_cast<const float *>(t->data);
        for (uint64_t i = 0; i < t->elements; ++i) {
            if (!std::isfinite(v[i])) {
                model_fail("malformed lookup tables");
            }
        }
    }
    return g;
}

// The tensors of one layer's MoE block, checked (src/model.cpp:267-314,
// 431-533, 834-880).
struct LayerTensors {
    const adi_hip_gguf_tensor *router, *gate_row;
    // [projection][chunk] of trellis, su, sv, wave_gamma
    std::vector<const adi_hip_gguf_tensor *> expert[3][4];
    const adi_hip_gguf_tensor *shared[3][3];  // trellis, SU, SV
    float wscale[3];
};

LayerTensors check_layer(const adi_hip_gguf &f, const adi_hip_moe_geometry &g, uint32_t layer) {
    if (layer >= g.layers) {
        model_fail("layer index is out of range");
    }
    LayerTensors L{};
    const std::string p = "hf." + layer_prefix(layer);
    L.router = &required_tensor(f, p + "mlp.gate.weight", ADI_HIP_GGML_BF16, {g.hidden, g.experts});
    L.gate_row = &required_tensor(f, p + "mlp.shared_expert_gate.weight", ADI_HIP_GGML_BF16, {g.hidden, 1});
    require_finite(*L.router, finite_bf16, p + "mlp.gate.weight");
    require_finite(*L.gate_row, finite_bf16, p + "mlp.shared_expert_gate.weight");
    for (int pr = 0; pr < 3; ++pr) {
        const uint64_t rows = pr == 2 ? g.hidden : g.expert_hidden;
        const uint64_t columns = pr == 2 ? g.expert_hidden : g.hidden;
        const uint64_t tiles = (rows / 16) * (columns / 16);
        const uint64_t gammas = rows / 16 + columns / 16;
        for (uint32_t chunk = 0; chunk < g.experts; chunk += 32) {
            const std::string t = expert_name(layer, chunk, pr, "trellis");
            const std::string su = expert_name(layer, chunk, pr, "su");
            const std::string sv = expert_name(layer, chunk, pr, "sv");
            const std::string gm = expert_name(layer, chunk, pr, "wave_gamma");
            L.expert[pr][0].push_back(&required_tensor(f, t, ADI_HIP_GGML_I16, {24, tiles, 32}));
            L.expert[pr][1].push_back(&required_tensor(f, su, ADI_HIP_GGML_F16, {columns, 32}));
            L.expert[pr][2].push_back(&required_tensor(f, sv, ADI_HIP_GGML_F16, {rows, 32}));
            L.expert[pr][3].push_back(&required_tensor(f, gm, ADI_HIP_GGML_F16, {gammas, 32}));
            require_finite(*L.expert[pr][1].back(), finite_f16, su);
            require_finite(*L.expert[pr][2].back(), finite_f16, sv);
            require_finite(*L.expert[pr][3].back(), finite_f16, gm);
        }
        // the shared expert (require_ne_shape, src/model.cpp:149-175)
        const uint64_t srows = pr == 2 ? g.hidden : g.shared_hidden;
        const uint64_t scols = pr == 2 ? g.shared_hidden : g.hidden;
        const std::string st = shared_name(layer, pr, "trellis");
        L.shared[pr][0] = &required_tensor(f, st, ADI_HIP_GGML_I16, {64, (srows / 16) * (scols / 16)});
        L.shared[pr][1] = &required_tensor(f, shared_name(layer, pr, "SU"), ADI_HIP_GGML_I8, {scols});
        L.shared[pr][2] = &required_tensor(f, shared_name(layer, pr, "SV"), ADI_HIP_GGML_I8, {srows});
        const adi_hip_gguf_tensor &ws = required_tensor(f, shared_name(layer, pr, "Wscale"), ADI_HIP_GGML_F32, {1});
        L.wscale[pr] = *static_cast<const float *>(ws.data);
        if (!std::isfinite(L.wscale[pr]) || L.wscale[pr] <= 0.0f) {
            model_fail("unexpected non-expert shape '" + st + "'");
        }
        for (int s = 1; s < 3; ++s) {
            const int8_t *v = static_cast<const int8_t *>(L.shared[pr][s]->data);
            for (uint64_t i = 0; i < L.shared[pr][s]->elements; ++i) {
                if (v[i] != 1 && v[i] != -1) {
                    model_fail("invalid non-expert sign tensor '" + st + "'");
                }
            }
        }
    }
    return L;
}

// The embedding tensors, checked (src/model.cpp:316-363, 836-849).
struct EmbeddingTensors {
    const adi_hip_gguf_tensor *packed, *minimum, *maximum, *indexes, *bits;
    uint32_t rows, columns;
};

EmbeddingTensors check_embedding(const adi_hip_gguf &f) {
    const uint32_t hidden = required_u32(f, "qwen35moe.embedding_length");
    const adi_hip_gguf_tensor *q = f.tensor("mach.embedding.q_packed");
    if (q == nullptr || q->type != ADI_HIP_GGML_I8) {
        model_fail("missing or invalid tensor 'mach.embedding.q_packed'");
    }
    if (q->dimension_count != 2 || q->dimensions[0] * 2 != hidden || hidden % 64 != 0 ||
        q->dimensions[1] > 0xFFFFFFFFull ||
        static_cast<uint64_t>(hidden) * q->dimensions[1] > 0xFFFFFFFFull) {
        model_fail("malformed embedding geometry");
    }
    EmbeddingTensors t{};
    t.rows = static_cast<uint32_t>(q->dimensions[1]);
    t.columns = hidden;
    t.packed = &required_tensor(f, "mach.embedding.q_packed", ADI_HIP_GGML_I8, {hidden / 2u, t.rows});
    t.minimum = &required_tensor(f, "mach.embedding.mn", ADI_HIP_GGML_F16, {hidden / 64u, t.rows});
    t.maximum = &required_tensor(f, "mach.embedding.mx", ADI_HIP_GGML_F16, {hidden / 64u, t.rows});
    const adi_hip_gguf_tensor *ix = f.tensor("mach.embedding.exc_idx");
    const adi_hip_gguf_tensor *bx = f.tensor("mach.embedding.exc_bits");
    if (ix == nullptr || ix->type != ADI_HIP_GGML_I32 || bx == nullptr ||
        bx->type != ADI_HIP_GGML_I16 || ix->dimension_count != 1 || bx->dimension_count != 1 ||
        ix->dimensions[0] != bx->dimensions[0]) {
        model_fail("malformed embedding tensors");
    }
    t.indexes = &required_tensor(f, "mach.embedding.exc_idx", ADI_HIP_GGML_I32, {ix->dimensions[0]});
    t.bits = &required_tensor(f, "mach.embedding.exc_bits", ADI_HIP_GGML_I16, {bx->dimensions[0]});
    const uint32_t *idx = static_cast<const uint32_t *>(t.indexes->data);
    const uint64_t total = static_cast<uint64_t>(t.rows) * t.columns;
    for (uint64_t i = 0; i < t.indexes->elements; ++i) {
        if ((i > 0 && idx[i] <= idx[i - 1]) || idx[i] >= total) {
            model_fail("malformed embedding tensors");
        }
    }
    require_finite(*t.minimum, finite_f16, "mach.embedding.mn");
    require_finite(*t.maximum, finite_f16, "mach.embedding.mx");
    require_finite(*t.bits, finite_bf16, "mach.embedding.exc_bits");
    const uint16_t *mn = static_cast<const uint16_t *>(t.minimum->data);
    const uint16_t *mx = static_cast<const uint16_t *>(t.maximum->data);
    for (uint64_t i = 0; i < t.minimum->elements; ++i) {
        if (f16_bits_to_float_host(mn[i]) > f16_bits_to_float_host(mx[i])) {
            model_fail("embedding minimum exceeds maximum");
        }
    }
    return t;
}

}  // namespace
}  // namespace adi_hip

struct adi_hip_weights {
    int device = 0;
    void *base = nullptr;
};

extern "C" {

int adi_hip_gguf_open(const char *path, adi_hip_gguf **out) {
    return file_call([&] {
        if (out == nullptr || path == nullptr) {
            fail(ADI_HIP_INVALID_ARGUMENT, "GGUF: null path or output pointer");
        }
        *out = nullptr;
        auto *file = new adi_hip_gguf;
        try {
            file->open(path);
        } catch (...) {
            delete file;
            throw;
        }
        *out = file;
        return ADI_HIP_OK;
    });
}

void adi_hip_gguf_close(adi_hip_gguf *file) { delete file; }

const char *adi_hip_gguf_error(void) { return g_gguf_error.c_str(); }

uint32_t adi_hip_gguf_version(const adi_hip_gguf *file) { return file ? file->version : 0; }
uint64_t adi_hip_gguf_alignment(const adi_hip_gguf *file) { return file ? file->alignment : 0; }
uint64_t adi_hip_gguf_metadata_count(const adi_hip_gguf *file) {
    return file ? file->metadata_count : 0;
}
uint64_t adi_hip_gguf_tensor_count(const adi_hip_gguf *file) {
    return file ? file->tensors.size() : 0;
}

int adi_hip_gguf_find_tensor(const adi_hip_gguf *file, const char *name, adi_hip_gguf_tensor *out) {
    return file_call([&] {
        if (file == nullptr || name == nullptr || out == nullptr) {
            fail(ADI_HIP_INVALID_ARGUMENT, "GGUF: null argument");
        }
        const adi_hip_gguf_tensor *t = file->tensor(name);
        if (t == nullptr) {
            return not_found(std::string("tensor '") + name + "'");
        }
        *out = *t;
        return ADI_HIP_OK;
    });
}

int adi_hip_gguf_integer(const adi_hip_gguf *file, const char *key, uint64_t *out) {
    return file_call([&] {
        uint64_t v = 0;
        if (file == nullptr || out == nullptr || !file->integer(key, v)) {
            return not_found(std::string("integer '") + (key ? key : "") + "'");
        }
        *out = v;
        return ADI_HIP_OK;
    });
}

int adi_hip_gguf_number(const adi_hip_gguf *file, const char *key, double *out) {
    return file_call([&] {
        double v = 0.0;
        if (file == nullptr || out == nullptr || !file->number(key, v)) {
            return not_found(std::string("number '") + (key ? key : "") + "'");
        }
        *out = v;
        return ADI_HIP_OK;
    });
}

int adi_hip_gguf_boolean(const adi_hip_gguf *file, const char *key, int *out) {
    return file_call([&] {
        bool v = false;
        if (file == nullptr || out == nullptr || !file->boolean(key, v)) {
            return not_found(std::string("boolean '") + (key ? key : "") + "'");
        }
        *out = v ? 1 : 0;
        return ADI_HIP_OK;
    });
}

int adi_hip_gguf_string(const adi_hip_gguf *file, const char *key, const char **data,
                        uint64_t *length) {
    return file_call([&] {
        std::string_view v;
        if (file == nullptr || data == nullptr || length == nullptr || !file->string(key, v)) {
            return not_found(std::string("string '") + (key ? key : "") + "'");
        }
        *data = v.data();
        *length = v.size();
        return ADI_HIP_OK;
    });
}

int adi_hip_gguf_string_array(const adi_hip_gguf *file, const char *key, uint64_t index,
                              uint64_t *count, const char **data, uint64_t *length) {
    return file_call([&] {
        const adi_hip_gguf::Entry *e = file ? file->entry(key) : nullptr;
        if (e == nullptr || e->type != kArray || count == nullptr) {
            return not_found(std::string("string array '") + (key ? key : "") + "'");
        }
        Reader r = file->reader(e->value_at);
        if (r.value_type() != kString) {
            return not_found(std::string("string array '") + key + "'");
        }
        const uint64_t n = r.get<uint64_t>();
        if (n > r.left()) {
            gguf_fail("metadata string array count is invalid");
        }
        *count = n;
        if (index < n && data != nullptr && length != nullptr) {
            for (uint64_t i = 0; i < index; ++i) {
                (void)r.text();
            }
            const std::string_view v = r.text();
            *data = v.data();
            *length = v.size();
        }
        return ADI_HIP_OK;
    });
}

int adi_hip_gguf_integer_array(const adi_hip_gguf *file, const char *key, uint64_t index,
                               uint64_t *count, uint64_t *value) {
    return file_call([&] {
        const adi_hip_gguf::Entry *e = file ? file->entry(key) : nullptr;
        if (e == nullptr || e->type != kArray || count == nullptr) {
            return not_found(std::string("integer array '") + (key ? key : "") + "'");
        }
        Reader r = file->reader(e->value_at);
        const uint32_t type = r.value_type();
        const uint64_t n = r.get<uint64_t>();
        // unsigned element types only, as GgufFile::integer_array
        if ((type != kU8 && type != kU16 && type != kU32 && type != kU64) || n > r.left()) {
            return not_found(std::string("integer array '") + key + "'");
        }
        *count = n;
        if (index < n && value != nullptr) {
            const uint64_t size = scalar_bytes(type);
            r.skip(index * size);
            switch (type) {
            case kU8: *value = r.get<uint8_t>(); break;
            case kU16: *value = r.get<uint16_t>(); break;
            case kU32: *value = r.get<uint32_t>(); break;
            default: *value = r.get<uint64_t>(); break;
            }
        }
        return ADI_HIP_OK;
    });
}

int adi_hip_gguf_moe_geometry(const adi_hip_gguf *file, adi_hip_moe_geometry *out) {
    return file_call([&] {
        if (file == nullptr || out == nullptr) {
            fail(ADI_HIP_INVALID_ARGUMENT, "model: null argument");
        }
        *out = read_geometry(*file);
        return ADI_HIP_OK;
    });
}

int adi_hip_gguf_check_moe_layer(const adi_hip_gguf *file, uint32_t layer) {
    return file_call([&] {
        if (file == nullptr) {
            fail(ADI_HIP_INVALID_ARGUMENT, "model: null file");
        }
        (void)check_layer(*file, read_geometry(*file), layer);
        return ADI_HIP_OK;
    });
}

int adi_hip_gguf_upload_codebooks(adi_hip_context *ctx, const adi_hip_gguf *file,
                                  adi_hip_codebook **expert_codebook,
                                  adi_hip_codebook **ne_codebook) {
    if (ctx == nullptr) {
        return ADI_HIP_INVALID_ARGUMENT;
    }
    const float *et = nullptr, *nt = nullptr;
    const int status = guarded(ctx, [&] {
        require(file != nullptr && expert_codebook != nullptr && ne_codebook != nullptr,
                "GGUF codebooks: null argument");
        *expert_codebook = nullptr;
        *ne_codebook = nullptr;
        (void)read_geometry(*file);
        et = static_cast<const float *>(file->tensor("mach.tlut.expert.tlut")->data);
        nt = static_cast<const float *>(file->tensor("mach.tlut.ne.tlut")->data);
    });
    if (status != ADI_HIP_OK) {
        return status;
    }
    int s = adi_hip_codebook_create_expert(ctx, et, expert_codebook);
    if (s != ADI_HIP_OK) {
        return s;
    }
    s = adi_hip_codebook_create_ne(ctx, nt, ne_codebook);
    if (s != ADI_HIP_OK) {
        adi_hip_codebook_destroy(*expert_codebook);
        *expert_codebook = nullptr;
    }
    return s;
}

int adi_hip_gguf_upload_moe_layer(adi_hip_context *ctx, const adi_hip_gguf *file, uint32_t layer,
                                  const adi_hip_codebook *expert_codebook,
                                  const adi_hip_codebook *ne_codebook,
                                  adi_hip_weights **weights,
                                  adi_hip_moe_layer *descriptor) {
    return guarded(ctx, [&] {
        require(file != nullptr && weights != nullptr && descriptor != nullptr,
                "GGUF layer upload: null argument");
        require(expert_codebook != nullptr && expert_codebook->kind == adi_hip_codebook::expert &&
                    ne_codebook != nullptr && ne_codebook->kind == adi_hip_codebook::ne,
                "GGUF layer upload: expert and NE codebooks required");
        *weights = nullptr;
        const adi_hip_moe_geometry g = read_geometry(*file);
        const LayerTensors L = check_layer(*file, g, layer);

        // one allocation, every piece 256-byte aligned; the chunks of a stack
        // field are laid end to end (expert-major, as the stack expects)
        struct Piece {
            const adi_hip_gguf_tensor *tensor;
            size_t at;
        };
        std::vector<Piece> pieces;
        size_t total = 0;
        auto place = [&](std::initializer_list<const adi_hip_gguf_tensor *> run) {
            const size_t start = total;
            for (const adi_hip_gguf_tensor *t : run) {
                pieces.push_back({t, total});
                total += static_cast<size_t>(t->bytes);
            }
            total = (total + 255) & ~size_t(255);
            return start;
        };
        auto place_chunks = [&](const std::vector<const adi_hip_gguf_tensor *> &chunks) {
            const size_t start = total;
            for (const adi_hip_gguf_tensor *t : chunks) {
                pieces.push_back({t, total});
                total += static_cast<size_t>(t->bytes);
            }
            total = (total + 255) & ~size_t(255);
            return start;
        };
        const size_t router_at = place({L.router});
        const size_t gate_row_at = place({L.gate_row});
        size_t stack_at[3][4], shared_at[3][3];
        for (int pr = 0; pr < 3; ++pr) {
            for (int fi = 0; fi < 4; ++fi) {
                stack_at[pr][fi] = place_chunks(L.expert[pr][fi]);
            }
            for (int fi = 0; fi < 3; ++fi) {
                shared_at[pr][fi] = place({L.shared[pr][fi]});
            }
        }
        auto *w = new adi_hip_weights;
        w->device = ctx->device;
        if (hipMalloc(&w->base, total) != hipSuccess) {
            delete w;
            fail(ADI_HIP_OUT_OF_MEMORY, "GGUF layer upload: device allocation failed");
        }
        try {
            for (const Piece &p : pieces) {
                check_hip(hipMemcpy(static_cast<char *>(w->base) + p.at, p.tensor->data,
                                    static_cast<size_t>(p.tensor->bytes), hipMemcpyHostToDevice),
                          "GGUF layer upload copy");
            }
        } catch (...) {
            (void)hipFree(w->base);
            delete w;
            throw;
        }
        char *base = static_cast<char *>(w->base);
        adi_hip_moe_layer d{};
        d.hidden = g.hidden;
        d.expert_hidden = g.expert_hidden;
        d.experts = g.experts;
        d.router = adi_hip_bf16_matrix{g.experts, g.hidden, reinterpret_cast<const uint16_t *>(base + router_at)};
        d.shared_expert_gate = adi_hip_bf16_matrix{1, g.hidden, reinterpret_cast<const uint16_t *>(base + gate_row_at)};
        adi_hip_expert_stack *stacks[3] = {&d.gate, &d.up, &d.down};
        adi_hip_ne_matrix *shared[3] = {&d.shared_gate, &d.shared_up, &d.shared_down};
        for (int pr = 0; pr < 3; ++pr) {
            stacks[pr]->trellis = reinterpret_cast<const uint16_t *>(base + stack_at[pr][0]);
            stacks[pr]->su_f16 = reinterpret_cast<const uint16_t *>(base + stack_at[pr][1]);
            stacks[pr]->sv_f16 = reinterpret_cast<const uint16_t *>(base + stack_at[pr][2]);
            stacks[pr]->wave_gamma_f16 = reinterpret_cast<const uint16_t *>(base + stack_at[pr][3]);
            adi_hip_ne_matrix &n = *shared[pr];
            n.rows = pr == 2 ? g.hidden : g.shared_hidden;
            n.columns = pr == 2 ? g.shared_hidden : g.hidden;
            n.trellis = reinterpret_cast<const uint16_t *>(base + shared_at[pr][0]);
            n.su = reinterpret_cast<const int8_t *>(base + shared_at[pr][1]);
            n.sv = reinterpret_cast<const int8_t *>(base + shared_at[pr][2]);
            n.weight_scale = L.wscale[pr];
            n.codebook = ne_codebook;
        }
        d.expert_codebook = expert_codebook;
        *descriptor = d;
        *weights = w;
    });
}

int adi_hip_gguf_check_embedding(const adi_hip_gguf *file) {
    return file_call([&] {
        if (file == nullptr) {
            fail(ADI_HIP_INVALID_ARGUMENT, "model: null file");
        }
        (void)check_embedding(*file);
        return ADI_HIP_OK;
    });
}

int adi_hip_gguf_upload_embedding(adi_hip_context *ctx, const adi_hip_gguf *file,
                                  adi_hip_weights **weights, adi_hip_embedding *descriptor) {
    return guarded(ctx, [&] {
        require(file != nullptr && weights != nullptr && descriptor != nullptr,
                "GGUF embedding upload: null argument");
        *weights = nullptr;
        const EmbeddingTensors t = check_embedding(*file);
        const adi_hip_gguf_tensor *parts[5] = {t.packed, t.minimum, t.maximum, t.indexes, t.bits};
        size_t at[5], total = 0;
        for (int i = 0; i < 5; ++i) {
            at[i] = total;
            total = (total + static_cast<size_t>(parts[i]->bytes) + 255) & ~size_t(255);
        }
        auto *w = new adi_hip_weights;
        w->device = ctx->device;
        if (hipMalloc(&w->base, total) != hipSuccess) {
            delete w;
            fail(ADI_HIP_OUT_OF_MEMORY, "GGUF embedding upload: device allocation failed");
        }
        try {
            for (int i = 0; i < 5; ++i) {
                check_hip(hipMemcpy(static_cast<char *>(w->base) + at[i], parts[i]->data,
                                    static_cast<size_t>(parts[i]->bytes), hipMemcpyHostToDevice),
                          "GGUF embedding upload copy");
            }
        } catch (...) {
            (void)hipFree(w->base);
            delete w;
            throw;
        }
        const char *base = static_cast<const char *>(w->base);
        adi_hip_embedding d{};
        d.rows = t.rows;
        d.columns = t.columns;
        d.packed = reinterpret_cast<const uint8_t *>(base + at[0]);
        d.minimum_f16 = reinterpret_cast<const uint16_t *>(base + at[1]);
        d.maximum_f16 = reinterpret_cast<const uint16_t *>(base + at[2]);
        d.exception_indexes = reinterpret_cast<const uint32_t *>(base + at[3]);
        d.exception_bf16 = reinterpret_cast<const uint16_t *>(base + at[4]);
        d.exception_count = static_cast<uint32_t>(t.indexes->elements);
        *descriptor = d;
        *weights = w;
    });
}

void adi_hip_weights_destroy(adi_hip_weights *weights) {
    if (weights == nullptr) {
        return;
    }
    int previous = 0;
    (void)hipGetDevice(&previous);
    (void)hipSetDevice(weights->device);
    (void)hipFree(weights->base);
    (void)hipSetDevice(previous);
    delete weights;
}

}  // extern "C"
