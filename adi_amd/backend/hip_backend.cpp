// hip_backend.cpp -- adi::Backend over the adi_hip C ABI.
//
// Each entry checks its arguments exactly as the reference entry it replaces
// (same conditions, same std::invalid_argument messages: src/kernels.cpp:385-
// 1073), finds or creates the device copy of the weights, copies the host
// span in, launches, and copies the result out. Weights are views into the
// model file (include/adi/kernels.hpp:9-77) and never change while mapped, so
// their device copies are cached by host address and shape, as ExpertScratch
// caches the derived tables by source pointer (src/kernels.cpp:33-94). Each
// entry also keeps a hash of the buffer's full contents, taken at upload and
// compared on every call: a different buffer met at the same address (a
// remapped model) replaces the entry (its device copies are freed and the new
// contents uploaded), so the cache holds one copy per live address and never
// serves stale weights. The hash reads every byte of the weights a call uses
// (four independent 64-bit lanes, about 10-20 GB/s on one core): a parity
// cost of this host-span path, which copies activations in and out per call
// anyway. hip_backend_release_weights() frees every copy. Calls are serialised
// on one context:
// moe_forward calls the projections from worker threads
// (src/executor.cpp:261, 1321-1371), and the GPU runs them in turn anyway.
#include "hip_backend.hpp"

#include "adi_hip.h"

#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <stdexcept>
#include <string>
#include <tuple>
#include <utility>
#include <vector>

namespace adi {
namespace {

bool is_power_of_two(std::uint32_t v) { return v != 0 && (v & (v - 1)) == 0; }
constexpr std::uint32_t kTile = 16;

// 64-bit hash of a buffer's full contents: four independent multiply-rotate
// lanes over 8-byte words (so the loads pipeline), the tail bytes and the
// size folded in at the end.
inline std::uint64_t mix_lane(std::uint64_t lane, std::uint64_t word) {
    lane ^= word * 0x9E3779B97F4A7C15ull;
    lane = (lane << 31) | (lane >> 33);
    return lane * 0xC2B2AE3D27D4EB4Full;
}

template <typename T>
std::uint64_t fingerprint(std::span<const T> values) {
    const auto *bytes = reinterpret_cast<const unsigned char *>(values.data());
    const std::size_t size = values.size_bytes();
    std::uint64_t lane[4] = {0x243F6A8885A308D3ull, 0x13198A2E03707344ull, 0xA4093822299F31D0ull,
                             0x082EFA98EC4E6C89ull};
    std::size_t at = 0;
    for (; at + 32 <= size; at += 32) {
        std::uint64_t w[4];
        std::memcpy(w, bytes + at, 32);
        for (int i = 0; i < 4; ++i) {
            lane[i] = mix_lane(lane[i], w[i]);
        }
    }
    std::uint64_t tail = 0;
    for (std::size_t b = 0; at + b < size; ++b) {
        tail |= static_cast<std::uint64_t>(bytes[at + b]) << (8 * (b & 7));
        if ((b & 7) == 7 || at + b + 1 == size) {
            lane[0] = mix_lane(lane[0], tail);
            tail = 0;
        }
    }
    std::uint64_t h = size * 0xFF51AFD7ED558CCDull;
    for (int i = 0; i < 4; ++i) {
        h = mix_lane(h ^ lane[i], static_cast<std::uint64_t>(i) + 1);
    }
    return h;
}

class Runtime {
  public:
    static Runtime &get() {
        // never destroyed: device memory stays valid until the process ends
        static Runtime *runtime = new Runtime();
        return *runtime;
    }

    std::mutex mutex;
    adi_hip_context *ctx = nullptr;

    // cache keys: host address and shape (matrices) or address and length
    using Key = std::tuple<const void *, std::uint32_t, std::uint32_t>;
    using TableKey = std::pair<const void *, std::size_t>;

    void check(int status) const {
        if (status == ADI_HIP_OK) {
            return;
        }
        const std::string message = adi_hip_last_error(ctx);
        if (status == ADI_HIP_INVALID_ARGUMENT) {
            throw std::invalid_argument(message);
        }
        throw std::runtime_error("adi_hip: " + message);
    }

    template <typename T>
    const T *upload(std::span<const T> host) {
        void *device = nullptr;
        check(adi_hip_device_alloc(ctx, host.size_bytes(), &device));
        check(adi_hip_copy_to_device(ctx, device, host.data(), host.size_bytes()));
        return static_cast<const T *>(device);
    }

    // Grow-only staging buffers for the activations of one call.
    float *staging(int which, std::size_t count) {
        Buffer &b = buffers_[which];
        if (b.bytes < count * sizeof(float)) {
            adi_hip_device_free(ctx, b.pointer);
            b.pointer = nullptr;
            b.bytes = 0;
            check(adi_hip_device_alloc(ctx, count * sizeof(float), &b.pointer));
            b.bytes = count * sizeof(float);
        }
        return static_cast<float *>(b.pointer);
    }

    void to_device(float *device, std::span<const float> host) {
        check(adi_hip_copy_to_device(ctx, device, host.data(), host.size_bytes()));
    }
    void to_host(std::span<float> host, const float *device) {
        check(adi_hip_copy_to_host(ctx, host.data(), device, host.size_bytes()));
    }

    // An entry of a cache: the descriptor, the contents' full hash and the
    // device buffers it owns.
    template <typename T>
    struct Entry {
        std::uint64_t fingerprint = 0;
        T value{};
        std::vector<void *> owned;
    };

    // The entry of `key`, (re)built by make(entry) when it is missing or its
    // contents' hash differs from `fp` (the old copies are freed first).
    template <typename K, typename T, typename Make>
    const T &cached(std::map<K, Entry<T>> &cache, const K &key, std::uint64_t fp, Make &&make) {
        auto found = cache.find(key);
        if (found != cache.end() && found->second.fingerprint == fp) {
            return found->second.value;
        }
        if (found != cache.end()) {
            release(found->second);
            cache.erase(found);
        }
        Entry<T> entry;
        entry.fingerprint = fp;
        make(entry);
        return cache.emplace(key, std::move(entry)).first->second.value;
    }

    template <typename U, typename T>
    const U *upload_into(Entry<T> &entry, std::span<const U> host) {
        const U *device = upload(host);
        entry.owned.push_back(const_cast<U *>(device));
        return device;
    }

    template <typename T>
    void release(Entry<T> &entry) {
        check(adi_hip_synchronize(ctx));
        for (void *p : entry.owned) {
            adi_hip_device_free(ctx, p);
        }
        entry.owned.clear();
    }

    template <typename K, typename T>
    void release_all(std::map<K, Entry<T>> &cache) {
        for (auto &kv : cache) {
            release(kv.second);
        }
        cache.clear();
    }

    void release_books(std::map<TableKey, Entry<adi_hip_codebook *>> &books) {
        check(adi_hip_synchronize(ctx));
        for (auto &kv : books) {
            adi_hip_codebook_destroy(kv.second.value);
        }
        books.clear();
    }

    void release_weights() {
        release_all(experts_);
        release_all(nes_);
        release_all(heads_);
        release_all(bf16s_);
        release_all(embeddings_);
        release_all(weights_);
        release_books(expert_books_);
        release_books(ne_books_);
    }

    const adi_hip_codebook *book(std::map<TableKey, Entry<adi_hip_codebook *>> &books,
                                 std::span<const float> tlut, bool expert) {
        const TableKey key{tlut.data(), tlut.size()};
        auto found = books.find(key);
        const std::uint64_t fp = fingerprint(tlut);
        if (found != books.end() && found->second.fingerprint == fp) {
            return found->second.value;
        }
        if (found != books.end()) {
            check(adi_hip_synchronize(ctx));
            adi_hip_codebook_destroy(found->second.value);
            books.erase(found);
        }
        Entry<adi_hip_codebook *> entry;
        entry.fingerprint = fp;
        check(expert ? adi_hip_codebook_create_expert(ctx, tlut.data(), &entry.value)
                     : adi_hip_codebook_create_ne(ctx, tlut.data(), &entry.value));
        return books.emplace(key, std::move(entry)).first->second.value;
    }
    const adi_hip_codebook *expert_book(std::span<const float> tlut) {
        return book(expert_books_, tlut, true);
    }
    const adi_hip_codebook *ne_book(std::span<const float> tlut) {
        return book(ne_books_, tlut, false);
    }

    const adi_hip_expert_matrix &expert(const MachExpertMatrix &m) {
        const std::uint64_t fp = fingerprint(m.trellis) ^ fingerprint(m.su_f16) * 3 ^
                                 fingerprint(m.sv_f16) * 5 ^ fingerprint(m.wave_gamma_f16) * 7 ^
                                 fingerprint(m.tlut) * 11;
        return cached(experts_, Key{m.trellis.data(), m.rows, m.columns}, fp,
                      [&](Entry<adi_hip_expert_matrix> &e) {
                          adi_hip_expert_matrix &d = e.value;
                          d.rows = m.rows;
                          d.columns = m.columns;
                          d.trellis = upload_into(e, m.trellis);
                          d.su_f16 = upload_into(e, m.su_f16);
                          d.sv_f16 = upload_into(e, m.sv_f16);
                          d.wave_gamma_f16 = upload_into(e, m.wave_gamma_f16);
                          d.codebook = expert_book(m.tlut);
                      });
    }

    const adi_hip_ne_matrix &ne(const MachNeMatrix &m) {
        std::uint32_t scale_bits = 0;
        std::memcpy(&scale_bits, &m.weight_scale, sizeof(scale_bits));
        const std::uint64_t fp = fingerprint(m.trellis) ^ fingerprint(m.su) * 3 ^
                                 fingerprint(m.sv) * 5 ^ fingerprint(m.tlut) * 7 ^
                                 static_cast<std::uint64_t>(scale_bits) * 13;
        return cached(nes_, Key{m.trellis.data(), m.rows, m.columns}, fp,
                      [&](Entry<adi_hip_ne_matrix> &e) {
                          adi_hip_ne_matrix &d = e.value;
                          d.rows = m.rows;
                          d.columns = m.columns;
                          d.trellis = upload_into(e, m.trellis);
                          d.su = upload_into(e, m.su);
                          d.sv = upload_into(e, m.sv);
                          d.weight_scale = m.weight_scale;
                          d.codebook = ne_book(m.tlut);
                      });
    }

    const adi_hip_head_chunk &head(const MachHeadChunk &h) {
        const std::uint64_t fp = fingerprint(h.packed) ^ fingerprint(h.group_scale_f16) * 3 ^
                                 fingerprint(h.protected_rows) * 5 ^
                                 fingerprint(h.protected_bf16) * 7;
        return cached(heads_, Key{h.packed.data(), h.rows, h.columns}, fp,
                      [&](Entry<adi_hip_head_chunk> &e) {
                          adi_hip_head_chunk &d = e.value;
                          d.rows = h.rows;
                          d.columns = h.columns;
                          d.packed = upload_into(e, h.packed);
                          d.group_scale_f16 = upload_into(e, h.group_scale_f16);
                          d.protected_count = static_cast<std::uint32_t>(h.protected_rows.size());
                          if (d.protected_count != 0) {
                              d.protected_rows = upload_into(e, h.protected_rows);
                              d.protected_bf16 = upload_into(e, h.protected_bf16);
                          }
                      });
    }

    const adi_hip_bf16_matrix &bf16(const Bf16Matrix &m) {
        return cached(bf16s_, Key{m.values.data(), m.rows, m.columns}, fingerprint(m.values),
                      [&](Entry<adi_hip_bf16_matrix> &e) {
                          e.value.rows = m.rows;
                          e.value.columns = m.columns;
                          e.value.values = upload_into(e, m.values);
                      });
    }

    const adi_hip_embedding &embedding(const MachEmbedding &e) {
        const std::uint64_t fp = fingerprint(e.packed) ^ fingerprint(e.minimum_f16) * 3 ^
                                 fingerprint(e.maximum_f16) * 5 ^
                                 fingerprint(e.exception_indexes) * 7 ^
                                 fingerprint(e.exception_bf16) * 11;
        return cached(embeddings_, Key{e.packed.data(), e.rows, e.columns}, fp,
                      [&](Entry<adi_hip_embedding> &entry) {
                          adi_hip_embedding &d = entry.value;
                          d.rows = e.rows;
                          d.columns = e.columns;
                          d.packed = upload_into(entry, e.packed);
                          d.minimum_f16 = upload_into(entry, e.minimum_f16);
                          d.maximum_f16 = upload_into(entry, e.maximum_f16);
                          d.exception_count = static_cast<std::uint32_t>(e.exception_indexes.size());
                          if (d.exception_count != 0) {
                              d.exception_indexes = upload_into(entry, e.exception_indexes);
                              d.exception_bf16 = upload_into(entry, e.exception_bf16);
                          }
                      });
    }

    const std::uint16_t *weights(std::span<const std::uint16_t> w) {
        return cached(weights_, TableKey{w.data(), w.size()}, fingerprint(w),
                      [&](Entry<const std::uint16_t *> &e) { e.value = upload_into(e, w); });
    }

    std::string name;

  private:
    Runtime() {
        int device = 0;
        if (const char *value = std::getenv("ADI_HIP_DEVICE")) {
            device = std::atoi(value);
        }
        if (adi_hip_context_create(device, &ctx) != ADI_HIP_OK) {
            throw std::runtime_error(std::string("adi_hip: ") + adi_hip_last_error(nullptr));
        }
        // follow the host CPU's reduction order (cpu_backend().name)
        const std::string_view isa = cpu_backend().name;
        const std::uint32_t lanes = isa == "avx512" ? 16u : (isa == "avx2" ? 8u : 1u);
        check(adi_hip_set_reduction_isa(ctx, lanes));
        name = "hip:" + std::string(isa);
    }

    struct Buffer {
        void *pointer = nullptr;
        std::size_t bytes = 0;
    };
    Buffer buffers_[2];
    std::map<TableKey, Entry<adi_hip_codebook *>> expert_books_;
    std::map<TableKey, Entry<adi_hip_codebook *>> ne_books_;
    std::map<Key, Entry<adi_hip_expert_matrix>> experts_;
    std::map<Key, Entry<adi_hip_ne_matrix>> nes_;
    std::map<Key, Entry<adi_hip_head_chunk>> heads_;
    std::map<Key, Entry<adi_hip_bf16_matrix>> bf16s_;
    std::map<Key, Entry<adi_hip_embedding>> embeddings_;
    std::map<TableKey, Entry<const std::uint16_t *>> weights_;
};

// ---- argument checks: the reference's conditions and messages -------------

void check_expert_codec(const MachExpertMatrix &m) {
    const std::size_t tiles = static_cast<std::size_t>(m.rows / kTile) * (m.columns / kTile);
    if (m.trellis.size() != tiles * 24 || m.wave_gamma_f16.size() != m.rows / kTile + m.columns / kTile ||
        m.tlut.size() != 32768u * 8u) {
        throw std::invalid_argument("Mach expert codec tensor shape mismatch");
    }
}

void check_ne_codec(const MachNeMatrix &m) {
    const std::size_t tiles = static_cast<std::size_t>(m.rows / kTile) * (m.columns / kTile);
    if (m.trellis.size() != tiles * 64 || m.tlut.size() != 512u * 2u) {
        throw std::invalid_argument("Mach NE codec tensor shape mismatch");
    }
}

bool tiled_powers(std::uint32_t rows, std::uint32_t columns) {
    return is_power_of_two(rows) && is_power_of_two(columns) && rows % kTile == 0 &&
           columns % kTile == 0;
}

void check_head(const MachHeadChunk &h, std::size_t inputs, std::size_t outputs, std::uint32_t batch) {
    constexpr std::uint32_t group = 64;
    const bool shape_ok = h.columns % group == 0 && inputs == std::size_t(batch) * h.columns &&
                          outputs == std::size_t(batch) * h.rows &&
                          h.packed.size() == std::size_t(h.rows) * h.columns / 8 * 5 &&
                          h.group_scale_f16.size() == std::size_t(h.rows) * h.columns / group;
    if (batch == 1 && !shape_ok) {
        throw std::invalid_argument("Mach output head shape mismatch");
    }
    if (batch != 1 && (batch == 0 || !shape_ok)) {
        throw std::invalid_argument("Mach output head batch shape mismatch");
    }
    if (!h.protected_rows.empty()) {
        if (h.protected_bf16.size() != h.protected_rows.size() * h.columns) {
            throw std::invalid_argument("Mach protected output row shape mismatch");
        }
        for (const auto row : h.protected_rows) {
            if (row >= h.rows) {
                throw std::invalid_argument("Mach protected output row is out of range");
            }
        }
    }
}

// ---- the entries ---------------------------------------------------------------

void hip_expert_matmul(const MachExpertMatrix &m, std::span<const float> inputs, std::uint32_t batch,
                       std::span<float> outputs, ExpertScratch &) {
    if (batch == 1) {
        if (!tiled_powers(m.rows, m.columns)) {
            throw std::invalid_argument("Mach expert dimensions must be tiled powers of two");
        }
        if (inputs.size() != m.columns || outputs.size() != m.rows || m.su_f16.size() != m.columns ||
            m.sv_f16.size() != m.rows) {
            throw std::invalid_argument("Mach expert vector or scale shape mismatch");
        }
    } else if (batch == 0 || !tiled_powers(m.rows, m.columns) ||
               inputs.size() != std::size_t(batch) * m.columns ||
               outputs.size() != std::size_t(batch) * m.rows || m.su_f16.size() != m.columns ||
               m.sv_f16.size() != m.rows) {
        throw std::invalid_argument("Mach expert batch shape mismatch");
    }
    check_expert_codec(m);
    Runtime &rt = Runtime::get();
    std::lock_guard<std::mutex> lock(rt.mutex);
    const adi_hip_expert_matrix &d = rt.expert(m);
    float *in = rt.staging(0, inputs.size());
    float *out = rt.staging(1, outputs.size());
    rt.to_device(in, inputs);
    rt.check(adi_hip_expert_matmul(rt.ctx, &d, in, batch, out));
    rt.to_host(outputs, out);
}

void hip_expert_matvec(const MachExpertMatrix &m, std::span<const float> input, std::span<float> output,
                       ExpertScratch &scratch) {
    hip_expert_matmul(m, input, 1, output, scratch);
}

void hip_ne_matmul(const MachNeMatrix &m, std::span<const float> inputs, std::uint32_t batch,
                   std::span<float> outputs, ExpertScratch &) {
    if (batch == 1) {
        if (!tiled_powers(m.rows, m.columns)) {
            throw std::invalid_argument("Mach NE dimensions must be tiled powers of two");
        }
        if (inputs.size() != m.columns || outputs.size() != m.rows || m.su.size() != m.columns ||
            m.sv.size() != m.rows) {
            throw std::invalid_argument("Mach NE vector or sign shape mismatch");
        }
    } else if (batch == 0 || !tiled_powers(m.rows, m.columns) ||
               inputs.size() != std::size_t(batch) * m.columns ||
               outputs.size() != std::size_t(batch) * m.rows || m.su.size() != m.columns ||
               m.sv.size() != m.rows) {
        throw std::invalid_argument("Mach NE batch shape mismatch");
    }
    check_ne_codec(m);
    Runtime &rt = Runtime::get();
    std::lock_guard<std::mutex> lock(rt.mutex);
    const adi_hip_ne_matrix &d = rt.ne(m);
    float *in = rt.staging(0, inputs.size());
    float *out = rt.staging(1, outputs.size());
    rt.to_device(in, inputs);
    rt.check(adi_hip_ne_matmul(rt.ctx, &d, in, batch, out));
    rt.to_host(outputs, out);
}

void hip_ne_matvec(const MachNeMatrix &m, std::span<const float> input, std::span<float> output,
                   ExpertScratch &scratch) {
    hip_ne_matmul(m, input, 1, output, scratch);
}

void hip_head_matmul(const MachHeadChunk &h, std::span<const float> inputs, std::uint32_t batch,
                     std::span<float> outputs) {
    check_head(h, inputs.size(), outputs.size(), batch);
    Runtime &rt = Runtime::get();
    std::lock_guard<std::mutex> lock(rt.mutex);
    const adi_hip_head_chunk &d = rt.head(h);
    float *in = rt.staging(0, inputs.size());
    float *out = rt.staging(1, outputs.size());
    rt.to_device(in, inputs);
    rt.check(adi_hip_head_matmul(rt.ctx, &d, in, batch, out));
    rt.to_host(outputs, out);
}

void hip_head_matvec(const MachHeadChunk &h, std::span<const float> input, std::span<float> output) {
    hip_head_matmul(h, input, 1, output);
}

void hip_bf16_matmul(const Bf16Matrix &m, std::span<const float> inputs, std::uint32_t batch,
                     std::span<float> outputs) {
    const bool values_ok = m.values.size() == std::size_t(m.rows) * m.columns;
    if (batch == 1 && (inputs.size() != m.columns || outputs.size() != m.rows || !values_ok)) {
        throw std::invalid_argument("BF16 matrix-vector shape mismatch");
    }
    if (batch != 1 && (batch == 0 || inputs.size() != std::size_t(batch) * m.columns ||
                       outputs.size() != std::size_t(batch) * m.rows || !values_ok)) {
        throw std::invalid_argument("BF16 matrix batch shape mismatch");
    }
    Runtime &rt = Runtime::get();
    std::lock_guard<std::mutex> lock(rt.mutex);
    const adi_hip_bf16_matrix &d = rt.bf16(m);
    float *in = rt.staging(0, inputs.size());
    float *out = rt.staging(1, outputs.size());
    rt.to_device(in, inputs);
    rt.check(adi_hip_bf16_matmul(rt.ctx, &d, in, batch, out));
    rt.to_host(outputs, out);
}

void hip_bf16_matvec(const Bf16Matrix &m, std::span<const float> input, std::span<float> output) {
    hip_bf16_matmul(m, input, 1, output);
}

void hip_rms_norm(std::span<const float> input, std::span<const std::uint16_t> weight_bf16,
                  float weight_offset, float epsilon, std::span<float> output) {
    if (input.size() != weight_bf16.size() || output.size() != input.size() || input.empty()) {
        throw std::invalid_argument("RMS norm shape mismatch");
    }
    Runtime &rt = Runtime::get();
    std::lock_guard<std::mutex> lock(rt.mutex);
    const std::uint16_t *w = rt.weights(weight_bf16);
    float *in = rt.staging(0, input.size());
    float *out = rt.staging(1, output.size());
    rt.to_device(in, input);
    rt.check(adi_hip_rms_norm(rt.ctx, in, w, static_cast<std::uint32_t>(input.size()), 1,
                              weight_offset, epsilon, out));
    rt.to_host(output, out);
}

// mach_embedding_row's checks and messages (src/kernels.cpp:806-818); the
// token goes to the device, the row comes back.
void hip_embedding_row(const MachEmbedding &e, std::uint32_t token, std::span<float> output) {
    constexpr std::uint32_t group = 64;
    if (token >= e.rows || output.size() != e.columns || e.columns % group != 0 ||
        e.packed.size() != static_cast<std::size_t>(e.rows) * e.columns / 2) {
        throw std::invalid_argument("Mach embedding shape mismatch");
    }
    const std::size_t groups = e.columns / group;
    if (e.minimum_f16.size() != static_cast<std::size_t>(e.rows) * groups ||
        e.maximum_f16.size() != static_cast<std::size_t>(e.rows) * groups ||
        e.exception_indexes.size() != e.exception_bf16.size()) {
        throw std::invalid_argument("Mach embedding scale or exception shape mismatch");
    }
    Runtime &rt = Runtime::get();
    std::lock_guard<std::mutex> lock(rt.mutex);
    const adi_hip_embedding &d = rt.embedding(e);
    float *staged = rt.staging(0, 1);
    float *out = rt.staging(1, output.size());
    rt.check(adi_hip_copy_to_device(rt.ctx, staged, &token, sizeof(token)));
    rt.check(adi_hip_embedding_rows(rt.ctx, &d, reinterpret_cast<const std::uint32_t *>(staged), 1,
                                    out));
    rt.to_host(output, out);
}

}  // namespace

const Backend &hip_backend() {
    static const Backend backend = [] {
        Runtime &rt = Runtime::get();
        return Backend{
            rt.name,
            hip_expert_matvec,
            hip_expert_matmul,
            hip_ne_matvec,
            hip_ne_matmul,
            hip_embedding_row,
            hip_head_matvec,
            hip_head_matmul,
            hip_bf16_matvec,
            hip_bf16_matmul,
            hip_rms_norm,
        };
    }();
    return backend;
}

void hip_backend_release_weights() {
    Runtime &rt = Runtime::get();
    const std::lock_guard<std::mutex> lock(rt.mutex);
    rt.release_weights();
}

}  // namespace adi
