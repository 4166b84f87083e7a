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

// ---- attention, norms and the output head ---------------------------------

// A bf16 tensor by its source name, stored as "hf." + name
// (MachModel::bf16_vector / bf16_matrix / bf16_data, src/model.cpp:440-470),
// with the shape and finite values validate_manifest requires
// (src/model.cpp:140-148, 808-900).
const adi_hip_gguf_tensor &bf16_tensor(const adi_hip_gguf &f, const std::string &source,
                                       std::initializer_list<uint64_t> dims) {
    const std::string name = "hf." + source;
    const adi_hip_gguf_tensor &t = required_tensor(f, name, ADI_HIP_GGML_BF16, dims);
    require_finite(t, finite_bf16, name);
    return t;
}

// One NE matrix (MachModel::non_expert, src/model.cpp:267-314, with
// require_ne_shape, src/model.cpp:150-175): trellis i16 {64, tiles}, SU i8
// {columns}, SV i8 {rows}, Wscale f32 {1}; +-1 signs, finite positive Wscale.
struct NeTensors {
    const adi_hip_gguf_tensor *trellis, *su, *sv;
    float wscale;
    uint32_t rows, columns;
};

NeTensors check_ne(const adi_hip_gguf &f, uint32_t layer, const std::string &source, uint32_t rows,
                   uint32_t columns) {
    const std::string p = "mach.ne." + std::to_string(layer) + "." + source + "|";
    NeTensors n{};
    n.rows = rows;
    n.columns = columns;
    n.trellis = &required_tensor(f, p + "trellis", ADI_HIP_GGML_I16,
                                 {64, static_cast<uint64_t>(rows / 16) * (columns / 16)});
    n.su = &required_tensor(f, p + "SU", ADI_HIP_GGML_I8, {columns});
    n.sv = &required_tensor(f, p + "SV", ADI_HIP_GGML_I8, {rows});
    n.wscale = *static_cast<const float *>(required_tensor(f, p + "Wscale", ADI_HIP_GGML_F32, {1}).data);
    if (!std::isfinite(n.wscale) || n.wscale <= 0.0f) {
        model_fail("unexpected non-expert shape '" + source + "'");
    }
    for (const adi_hip_gguf_tensor *t : {n.su, n.sv}) {
        const int8_t *v = static_cast<const int8_t *>(t->data);
        for (uint64_t i = 0; i < t->elements; ++i) {
            if (v[i] != 1 && v[i] != -1) {
                model_fail("invalid non-expert sign tensor '" + source + "'");
            }
        }
    }
    return n;
}

// The attention half of a decoder layer and its two norms
// (MachModel::cache_descriptors, src/model.cpp:619-683, with the shapes of
// validate_manifest, src/model.cpp:808-880): every fourth layer (layer + 1
// divisible by 4) full attention, the others Gated DeltaNet.
struct AttentionTensors {
    bool full;
    NeTensors ne[4];                    // full: q, k, v, o; linear: qkv, z, out
    const adi_hip_gguf_tensor *bf[6];  // full: q_norm, k_norm; linear: a, b, conv1d, dt_bias, A_log, norm
    const adi_hip_gguf_tensor *input_norm, *post_norm;
};

AttentionTensors check_attention(const adi_hip_gguf &f, const adi_hip_moe_geometry &g, uint32_t layer) {
    if (layer >= g.layers) {
        model_fail("layer index is out of range");
    }
    AttentionTensors A{};
    const std::string prefix = layer_prefix(layer);
    A.input_norm = &bf16_tensor(f, prefix + "input_layernorm.weight", {g.hidden});
    A.post_norm = &bf16_tensor(f, prefix + "post_attention_layernorm.weight", {g.hidden});
    A.full = (layer + 1) % 4 == 0;
    if (A.full) {
        const std::string a = prefix + "self_attn.";
        A.ne[0] = check_ne(f, layer, a + "q_proj.weight", 8192, g.hidden);
        A.ne[1] = check_ne(f, layer, a + "k_proj.weight", 512, g.hidden);
        A.ne[2] = check_ne(f, layer, a + "v_proj.weight", 512, g.hidden);
        A.ne[3] = check_ne(f, layer, a + "o_proj.weight", g.hidden, 4096);
        A.bf[0] = &bf16_tensor(f, a + "q_norm.weight", {256});
        A.bf[1] = &bf16_tensor(f, a + "k_norm.weight", {256});
    } else {
        const std::string a = prefix + "linear_attn.";
        A.ne[0] = check_ne(f, layer, a + "in_proj_qkv.weight", 8192, g.hidden);
        A.ne[1] = check_ne(f, layer, a + "in_proj_z.weight", 4096, g.hidden);
        A.ne[2] = check_ne(f, layer, a + "out_proj.weight", g.hidden, 4096);
        A.bf[0] = &bf16_tensor(f, a + "in_proj_a.weight", {g.hidden, 32});
        A.bf[1] = &bf16_tensor(f, a + "in_proj_b.weight", {g.hidden, 32});
        A.bf[2] = &bf16_tensor(f, a + "conv1d.weight", {4, 1, 8192});
        A.bf[3] = &bf16_tensor(f, a + "dt_bias", {32});
        A.bf[4] = &bf16_tensor(f, a + "A_log", {32});
        A.bf[5] = &bf16_tensor(f, a + "norm.weight", {128});
    }
    return A;
}

// The output head: eight chunks of vocabulary / 8 rows (MachModel::head_chunk,
// src/model.cpp:367-420): qp i8 {hidden/8*5, rows}, gscale f16 {hidden/64,
// rows} finite, and optionally prot_rows i32 {n} with prot_dense bf16
// {hidden, n} (both or neither; rows inside the chunk, finite values); then
// the final norm (bf16 {hidden}, src/model.cpp:604, 884-887). The vocabulary
// and hidden width are the embedding's.
struct HeadTensors {
    uint32_t vocabulary, hidden, chunk_rows;
    const adi_hip_gguf_tensor *qp[8], *scale[8], *rows[8], *dense[8];
    const adi_hip_gguf_tensor *final_norm;
};

HeadTensors check_head(const adi_hip_gguf &f) {
    const EmbeddingTensors e = check_embedding(f);
    HeadTensors h{};
    h.vocabulary = e.rows;
    h.hidden = e.columns;
    if (h.vocabulary % 8 != 0 || h.hidden % 64 != 0) {
        model_fail("output chunk index is out of range");
    }
    h.chunk_rows = h.vocabulary / 8;
    for (uint32_t c = 0; c < 8; ++c) {
        const uint32_t begin = c * h.chunk_rows, end = begin + h.chunk_rows;
        const std::string p = "mach.output." + std::to_string(c) + ".LMHEADCHUNK:" + std::to_string(begin) +
                              ":" + std::to_string(end) + "|";
        h.qp[c] = &required_tensor(f, p + "qp", ADI_HIP_GGML_I8, {h.hidden / 8u * 5u, h.chunk_rows});
        h.scale[c] = &required_tensor(f, p + "gscale", ADI_HIP_GGML_F16, {h.hidden / 64u, h.chunk_rows});
        require_finite(*h.scale[c], finite_f16, "output head scale");
        const adi_hip_gguf_tensor *r = f.tensor(p + "prot_rows");
        const adi_hip_gguf_tensor *d = f.tensor(p + "prot_dense");
        if ((r == nullptr) != (d == nullptr)) {
            model_fail("incomplete protected output rows");
        }
        if (r != nullptr) {
            if (r->type != ADI_HIP_GGML_I32 || r->dimension_count != 1) {
                model_fail("invalid protected output row indexes");
            }
            h.rows[c] = &required_tensor(f, p + "prot_rows", ADI_HIP_GGML_I32, {r->dimensions[0]});
            h.dense[c] = &required_tensor(f, p + "prot_dense", ADI_HIP_GGML_BF16, {h.hidden, r->dimensions[0]});
            require_finite(*h.dense[c], finite_bf16, "protected output rows");
            const uint32_t *v = static_cast<const uint32_t *>(h.rows[c]->data);
            for (uint64_t i = 0; i < h.rows[c]->elements; ++i) {
                if (v[i] >= h.chunk_rows) {
                    model_fail("protected output row is out of range");
                }
            }
        }
    }
    h.final_norm = &bf16_tensor(f, "model.language_model.norm.weight", {h.hidden});
    return h;
}

// One device allocation for a set of host pieces, each 256-byte aligned (a
// run of pieces can be laid end to end).
struct Upload {
    struct Piece {
        const void *data;
        size_t bytes;
        size_t at;
    };
    std::vector<Piece> pieces;
    size_t total = 0;
    size_t add(const void *data, size_t bytes) {
        const size_t at = total;
        pieces.push_back({data, bytes, at});
        total = (total + bytes + 255) & ~size_t(255);
        return at;
    }
    size_t add(const adi_hip_gguf_tensor *t) { return add(t->data, static_cast<size_t>(t->bytes)); }
    size_t add_run(const std::vector<const adi_hip_gguf_tensor *> &run) {
        const size_t start = total;
        for (const adi_hip_gguf_tensor *t : run) {
            pieces.push_back({t->data, static_cast<size_t>(t->bytes), total});
            total += static_cast<size_t>(t->bytes);
        }
        total = (total + 255) & ~size_t(255);
        return start;
    }
    adi_hip_weights *commit(adi_hip_context *ctx, const char *what);
};

// Offsets of a layer's MoE tensors in an Upload.
struct MoeAt {
    size_t router, gate_row, stack[3][4], shared[3][3];
};

MoeAt place_moe(Upload &u, const LayerTensors &L) {
    MoeAt at{};
    at.router = u.add(L.router);
    at.gate_row = u.add(L.gate_row);
    for (int pr = 0; pr < 3; ++pr) {
        for (int fi = 0; fi < 4; ++fi) {
            at.stack[pr][fi] = u.add_run(L.expert[pr][fi]);
        }
        for (int fi = 0; fi < 3; ++fi) {
            at.shared[pr][fi] = u.add(L.shared[pr][fi]);
        }
    }
    return at;
}

adi_hip_ne_matrix ne_descriptor(const char *base, size_t trellis, size_t su, size_t sv, uint32_t rows,
                                uint32_t columns, float wscale, const adi_hip_codebook *ne_codebook) {
    adi_hip_ne_matrix n{};
    n.rows = rows;
    n.columns = columns;
    n.trellis = reinterpret_cast<const uint16_t *>(base + trellis);
    n.su = reinterpret_cast<const int8_t *>(base + su);
    n.sv = reinterpret_cast<const int8_t *>(base + sv);
    n.weight_scale = wscale;
    n.codebook = ne_codebook;
    return n;
}

adi_hip_moe_layer moe_descriptor(const char *base, const MoeAt &at, const adi_hip_moe_geometry &g,
                                 const LayerTensors &L, const adi_hip_codebook *expert_codebook,
                                 const adi_hip_codebook *ne_codebook) {
    adi_hip_moe_layer d{};
    d.hidden = g.hidden;
    d.expert_hidden = g.expert_hidden;
    d.experts = g.experts;
    d.router = adi_hip_bf16_matrix{g.experts, g.hidden, reinterpret_cast<const uint16_t *>(base + at.router)};
    d.shared_expert_gate = adi_hip_bf16_matrix{1, g.hidden, reinterpret_cast<const uint16_t *>(base + at.gate_row)};
    adi_hip_expert_stack *stacks[3] = {&d.gate, &d.up, &d.down};
    adi_hip_ne_matrix *shared[3] = {&d.shared_gate, &d.shared_up, &d.shared_down};
    for (int pr = 0; pr < 3; ++pr) {
        stacks[pr]->trellis = reinterpret_cast<const uint16_t *>(base + at.stack[pr][0]);
        stacks[pr]->su_f16 = reinterpret_cast<const uint16_t *>(base + at.stack[pr][1]);
        stacks[pr]->sv_f16 = reinterpret_cast<const uint16_t *>(base + at.stack[pr][2]);
        stacks[pr]->wave_gamma_f16 = reinterpret_cast<const uint16_t *>(base + at.stack[pr][3]);
        *shared[pr] = ne_descriptor(base, at.shared[pr][0], at.shared[pr][1], at.shared[pr][2],
                                    pr == 2 ? g.hidden : g.shared_hidden, pr == 2 ? g.shared_hidden : g.hidden,
                                    L.wscale[pr], ne_codebook);
    }
    d.expert_codebook = expert_codebook;
    return d;
}

}  // namespace
}  // namespace adi_hip

struct adi_hip_weights {
    int device = 0;
    void *base = nullptr;
};

adi_hip_weights *adi_hip::Upload::commit(adi_hip_context *ctx, const char *what) {
    auto *w = new adi_hip_weights;
    w->device = ctx->device;
    if (hipMalloc(&w->base, total == 0 ? 256 : total) != hipSuccess) {
        (void)hipGetLastError();
        delete w;
        fail(ADI_HIP_OUT_OF_MEMORY, std::string(what) + ": device allocation failed");
    }
    try {
        for (const Piece &p : pieces) {
            check_hip(hipMemcpy(static_cast<char *>(w->base) + p.at, p.data, p.bytes, hipMemcpyHostToDevice),
                      (std::string(what) + " copy").c_str());
        }
    } catch (...) {
        (void)hipFree(w->base);
        delete w;
        throw;
    }
    return w;
}

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
        // one allocation; the chunks of a stack field are laid end to end
        // (expert-major, as the stack expects)
        Upload u;
        const MoeAt at = place_moe(u, L);
        adi_hip_weights *w = u.commit(ctx, "GGUF layer upload");
        *descriptor = moe_descriptor(static_cast<const char *>(w->base), at, g, L, expert_codebook, ne_codebook);
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
            (void)hipGetLastError();
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

int adi_hip_gguf_check_decoder_layer(const adi_hip_gguf *file, uint32_t layer) {
    return file_call([&] {
        if (file == nullptr) {
            fail(ADI_HIP_INVALID_ARGUMENT, "model: null file");
        }
        const adi_hip_moe_geometry g = read_geometry(*file);
        (void)check_layer(*file, g, layer);
        (void)check_attention(*file, g, layer);
        return ADI_HIP_OK;
    });
}

int adi_hip_gguf_upload_decoder_layer(adi_hip_context *ctx, const adi_hip_gguf *file, uint32_t layer,
                                      const adi_hip_codebook *expert_codebook,
                                      const adi_hip_codebook *ne_codebook, adi_hip_weights **weights,
                                      adi_hip_decoder_layer *descriptor) {
    return guarded(ctx, [&] {
        require(file != nullptr && weights != nullptr && descriptor != nullptr,
                "GGUF decoder layer upload: null argument");
        require(expert_codebook != nullptr && expert_codebook->kind == adi_hip_codebook::expert &&
                    ne_codebook != nullptr && ne_codebook->kind == adi_hip_codebook::ne,
                "GGUF decoder layer upload: expert and NE codebooks required");
        *weights = nullptr;
        const adi_hip_moe_geometry g = read_geometry(*file);
        const LayerTensors L = check_layer(*file, g, layer);
        const AttentionTensors A = check_attention(*file, g, layer);
        Upload u;
        const MoeAt moe = place_moe(u, L);
        const size_t input_norm = u.add(A.input_norm), post_norm = u.add(A.post_norm);
        size_t ne[4][3] = {};
        const int ne_count = A.full ? 4 : 3;
        for (int i = 0; i < ne_count; ++i) {
            ne[i][0] = u.add(A.ne[i].trellis);
            ne[i][1] = u.add(A.ne[i].su);
            ne[i][2] = u.add(A.ne[i].sv);
        }
        size_t bf[6] = {};
        const int bf_count = A.full ? 2 : 6;
        for (int i = 0; i < bf_count; ++i) {
            bf[i] = u.add(A.bf[i]);
        }
        adi_hip_weights *w = u.commit(ctx, "GGUF decoder layer upload");
        const char *base = static_cast<const char *>(w->base);
        auto ne_at = [&](int i) {
            return ne_descriptor(base, ne[i][0], ne[i][1], ne[i][2], A.ne[i].rows, A.ne[i].columns, A.ne[i].wscale,
                                 ne_codebook);
        };
        auto bf_at = [&](int i) { return reinterpret_cast<const uint16_t *>(base + bf[i]); };
        adi_hip_decoder_layer d{};
        d.input_norm = reinterpret_cast<const uint16_t *>(base + input_norm);
        d.post_attention_norm = reinterpret_cast<const uint16_t *>(base + post_norm);
        d.full_attention = A.full ? 1 : 0;
        if (A.full) {
            d.full.query = ne_at(0);
            d.full.key = ne_at(1);
            d.full.value = ne_at(2);
            d.full.output = ne_at(3);
            d.full.query_norm = bf_at(0);
            d.full.key_norm = bf_at(1);
        } else {
            d.linear.qkv = ne_at(0);
            d.linear.gate = ne_at(1);
            d.linear.output = ne_at(2);
            d.linear.alpha = adi_hip_bf16_matrix{32, g.hidden, bf_at(0)};
            d.linear.beta = adi_hip_bf16_matrix{32, g.hidden, bf_at(1)};
            d.linear.convolution = bf_at(2);
            d.linear.alpha_bias = bf_at(3);
            d.linear.a_log = bf_at(4);
            d.linear.norm = bf_at(5);
        }
        d.moe = moe_descriptor(base, moe, g, L, expert_codebook, ne_codebook);
        *descriptor = d;
        *weights = w;
    });
}

int adi_hip_gguf_check_head(const adi_hip_gguf *file) {
    return file_call([&] {
        if (file == nullptr) {
            fail(ADI_HIP_INVALID_ARGUMENT, "model: null file");
        }
        (void)check_head(*file);
        return ADI_HIP_OK;
    });
}

int adi_hip_gguf_upload_head(adi_hip_context *ctx, const adi_hip_gguf *file, adi_hip_weights **weights,
                             adi_hip_head_chunk *head, const uint16_t **final_norm) {
    return guarded(ctx, [&] {
        require(file != nullptr && weights != nullptr && head != nullptr && final_norm != nullptr,
                "GGUF head upload: null argument");
        *weights = nullptr;
        const HeadTensors h = check_head(*file);
        // the chunks end to end: packed rows, scales, then the protected rows
        // renumbered to the whole head and their dense rows
        std::vector<const adi_hip_gguf_tensor *> qp(h.qp, h.qp + 8), scale(h.scale, h.scale + 8), dense;
        std::vector<uint32_t> protected_rows;
        for (uint32_t c = 0; c < 8; ++c) {
            if (h.rows[c] != nullptr) {
                const uint32_t *v = static_cast<const uint32_t *>(h.rows[c]->data);
                for (uint64_t i = 0; i < h.rows[c]->elements; ++i) {
                    protected_rows.push_back(c * h.chunk_rows + v[i]);
                }
                dense.push_back(h.dense[c]);
            }
        }
        Upload u;
        const size_t packed = u.add_run(qp);
        const size_t scales = u.add_run(scale);
        const size_t rows = protected_rows.empty() ? 0 : u.add(protected_rows.data(), protected_rows.size() * 4);
        const size_t bf = dense.empty() ? 0 : u.add_run(dense);
        const size_t norm = u.add(h.final_norm);
        adi_hip_weights *w = u.commit(ctx, "GGUF head upload");
        const char *base = static_cast<const char *>(w->base);
        adi_hip_head_chunk d{};
        d.rows = h.vocabulary;
        d.columns = h.hidden;
        d.packed = reinterpret_cast<const uint8_t *>(base + packed);
        d.group_scale_f16 = reinterpret_cast<const uint16_t *>(base + scales);
        d.protected_count = static_cast<uint32_t>(protected_rows.size());
        d.protected_rows = protected_rows.empty() ? nullptr : reinterpret_cast<const uint32_t *>(base + rows);
        d.protected_bf16 = dense.empty() ? nullptr : reinterpret_cast<const uint16_t *>(base + bf);
        *head = d;
        *final_norm = reinterpret_cast<const uint16_t *>(base + norm);
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
