// ref_shim.cpp -- C entry points over the reference's own compiled CPU path.
//
// TEST INFRASTRUCTURE ONLY. oracle/Makefile compiles the reference's sources
// where they lie (its src/*.cpp with the per-file ISA flags of its
// CMakeLists.txt:93-126) together with this file into oracle/_ref/. Tests use
// it to pin the C restatement in adi_oracle.c, and the benchmark times it as
// the CPU baseline. Nothing in the product links it.
//
// The MoE composition below calls only the reference's model-free entry
// points (bf16_matmul, top_experts, mach_expert_matmul/matvec,
// mach_ne_matmul/matvec, silu, sigmoid, and its worker pool) in the order of
// moe_forward (src/executor.cpp:242-330) for one row and moe_forward_batch
// (src/executor.cpp:1181-1453) otherwise: MachModel itself cannot be built
// without the full GGUF checkpoint. Codec caches are prepared once per layer
// the way MachModel::cache_descriptors does (src/model.cpp:542-691).
#include "adi/backend.hpp"
#include "adi/executor.hpp"
#include "adi/generation.hpp"
#include "adi/gguf.hpp"
#include "adi/kernels.hpp"
#include "adi/profiling.hpp"
#include "attention.hpp"
#include "codec_cache.hpp"
#include "expert_trellis.hpp"
#include "ne_trellis.hpp"
#include "parallel.hpp"
#include "simd.hpp"

#include "adi_oracle.h"

#include <algorithm>
#include <array>
#include <cstring>
#include <exception>
#include <memory>
#include <vector>

namespace {

std::span<const std::uint16_t> u16(const std::uint16_t *data, std::size_t n) {
    return {data, n};
}

adi::MachExpertMatrix expert_view(const ao_expert_matrix &m) {
    const std::size_t tiles =
        static_cast<std::size_t>(m.rows / 16) * (m.columns / 16);
    return {
        m.rows,
        m.columns,
        u16(m.trellis, tiles * 24),
        u16(m.su_f16, m.columns),
        u16(m.sv_f16, m.rows),
        u16(m.wave_gamma_f16, m.rows / 16 + m.columns / 16),
        std::span<const float>(m.tlut, 32768 * 8),
    };
}

adi::MachNeMatrix ne_view(const ao_ne_matrix &m) {
    const std::size_t tiles =
        static_cast<std::size_t>(m.rows / 16) * (m.columns / 16);
    return {
        m.rows,
        m.columns,
        u16(m.trellis, tiles * 64),
        std::span<const std::int8_t>(m.su, m.columns),
        std::span<const std::int8_t>(m.sv, m.rows),
        m.weight_scale,
        std::span<const float>(m.tlut, 512 * 2),
    };
}

adi::Bf16Matrix bf16_view(const ao_bf16_matrix &m) {
    return {m.rows, m.columns,
            u16(m.values, static_cast<std::size_t>(m.rows) * m.columns)};
}

template <typename F>
int guarded(F &&function) {
    try {
        function();
        return 0;
    } catch (const std::invalid_argument &) {
        return -1;
    } catch (const std::exception &) {
        return -3;
    }
}

adi::detail::CpuIsa isa_for_lanes(int lanes) {
    switch (lanes) {
    case 1:
        return adi::detail::CpuIsa::scalar;
    case 8:
        return adi::detail::CpuIsa::avx2;
    default:
        return adi::detail::CpuIsa::avx512;
    }
}

int lanes_for_isa(adi::detail::CpuIsa isa) {
    switch (isa) {
    case adi::detail::CpuIsa::avx2:
        return 8;
    case adi::detail::CpuIsa::avx512:
        return 16;
    default:
        return 1;
    }
}

// A prepared MoE layer: the views plus the caches MachModel builds at load.
struct RefLayer {
    std::uint32_t hidden = 0;
    std::uint32_t expert_hidden = 0;
    std::uint32_t experts = 0;
    adi::Bf16Matrix router{};
    adi::Bf16Matrix shared_expert_gate{};
    std::vector<std::array<adi::MachExpertMatrix, 3>> matrices;
    adi::MachNeMatrix shared[3]{};
    std::vector<float> expert_state_values;
    std::vector<float> ne_state_values;
    std::vector<float> ne_signed_tlut;
    std::vector<std::uint16_t> waves_forward;
    std::vector<std::uint16_t> waves_reverse;
    std::vector<float> gamma;
    // persistent scratch, as MoeScratch / DecoderBatchScratch are
    adi::MoeScratch moe_scratch;
    adi::DecoderBatchScratch batch_scratch;
};

} // namespace

extern "C" {

int ref_selected_isa_lanes(void) {
    return lanes_for_isa(adi::detail::selected_cpu_isa());
}

// lanes 0 clears the override; 1/8/16 force scalar/AVX2/AVX-512.
void ref_force_isa_lanes(int lanes) {
    if (lanes == 0) {
        adi::detail::clear_cpu_isa_for_testing();
    } else {
        adi::detail::force_cpu_isa_for_testing(isa_for_lanes(lanes));
    }
}

int ref_avx512_vbmi(void) {
    return adi::detail::detected_cpu_features().avx512vbmi ? 1 : 0;
}

std::uint32_t ref_worker_threads(void) {
    return adi::worker_threads();
}

// The reference's per-kind kernel profile (include/adi/profiling.hpp:9-40),
// as its bench commands print it (src/main.cpp:199-227): enabling resets it.
void ref_kernel_profiling(int enabled) {
    if (enabled != 0) {
        adi::reset_kernel_profiles();
    }
    adi::set_kernel_profiling_enabled(enabled != 0);
}

// Kind `kind`'s name (up to `capacity` bytes with the terminator), calls,
// nanoseconds and work items; returns the number of kinds.
std::uint32_t ref_kernel_profile(std::uint32_t kind, char *name, std::uint32_t capacity,
                                 std::uint64_t *calls, std::uint64_t *nanoseconds,
                                 std::uint64_t *work_items) {
    const auto profiles = adi::kernel_profiles();
    const auto count = static_cast<std::uint32_t>(profiles.size());
    if (kind < count) {
        const auto text = adi::kernel_name(static_cast<adi::KernelKind>(kind));
        const std::size_t n = std::min<std::size_t>(text.size(), capacity > 0 ? capacity - 1 : 0);
        if (capacity > 0) {
            std::memcpy(name, text.data(), n);
            name[n] = '\0';
        }
        *calls = profiles[kind].calls;
        *nanoseconds = profiles[kind].nanoseconds;
        *work_items = profiles[kind].work_items;
    }
    return count;
}

float ref_f16_to_f32(std::uint16_t bits) { return adi::f16_to_f32(bits); }
std::uint16_t ref_f32_to_f16(float value) { return adi::f32_to_f16(value); }
float ref_silu(float value) { return adi::silu(value); }
float ref_sigmoid(float value) { return adi::sigmoid(value); }

void ref_expert_tile_states(const std::uint16_t *words, std::uint16_t *states) {
    adi::detail::for_each_expert_state(
        words, [&](std::uint32_t i, std::uint32_t s) {
            states[i] = static_cast<std::uint16_t>(s);
        });
}

void ref_expert_row_states(const std::uint16_t *words, std::uint16_t *states) {
    adi::detail::for_each_expert_row_state(
        words, [&](std::uint32_t row, std::uint32_t step, std::uint32_t s) {
            states[row * 2 + step] = static_cast<std::uint16_t>(s);
        });
}

void ref_ne_tile_states(const std::uint16_t *words, std::uint16_t *states) {
    adi::detail::for_each_ne_state(
        words, [&](std::uint32_t i, std::uint32_t s) {
            states[i] = static_cast<std::uint16_t>(s);
        });
}

void ref_ne_row_states(const std::uint16_t *words, std::uint16_t *states) {
    adi::detail::for_each_ne_row_state(
        words, [&](std::uint32_t row, std::uint32_t step, std::uint32_t s) {
            states[row * 8 + step] = static_cast<std::uint16_t>(s);
        });
}

void ref_build_expert_state_values(const float *tlut, float *out) {
    const auto v = adi::detail::build_expert_state_values({tlut, 32768 * 8});
    std::memcpy(out, v.data(), v.size() * sizeof(float));
}

void ref_build_ne_state_values(const float *tlut, float *out) {
    const auto v = adi::detail::build_ne_state_values({tlut, 512 * 2});
    std::memcpy(out, v.data(), v.size() * sizeof(float));
}

void ref_build_ne_signed_tlut(const float *tlut, float *out) {
    const auto v = adi::detail::build_ne_signed_tlut({tlut, 512 * 2});
    std::memcpy(out, v.data(), v.size() * sizeof(float));
}

int ref_build_wave_indexes(std::uint32_t tile_rows, std::uint32_t tile_columns,
                           std::uint16_t *out) {
    return guarded([&] {
        const auto v = adi::detail::build_wave_indexes(tile_rows, tile_columns);
        std::memcpy(out, v.data(), v.size() * sizeof(std::uint16_t));
    });
}

void ref_hadamard(float *values, std::uint32_t count) {
    adi::detail::hadamard_transform({values, count});
}

int ref_expert_matmul(const ao_expert_matrix *m, const float *inputs,
                      std::uint32_t batch, float *outputs) {
    return guarded([&] {
        thread_local adi::ExpertScratch scratch;
        adi::mach_expert_matmul(
            expert_view(*m),
            {inputs, static_cast<std::size_t>(batch) * m->columns}, batch,
            {outputs, static_cast<std::size_t>(batch) * m->rows}, scratch);
    });
}

int ref_ne_matmul(const ao_ne_matrix *m, const float *inputs,
                  std::uint32_t batch, float *outputs) {
    return guarded([&] {
        thread_local adi::ExpertScratch scratch;
        adi::mach_ne_matmul(
            ne_view(*m),
            {inputs, static_cast<std::size_t>(batch) * m->columns}, batch,
            {outputs, static_cast<std::size_t>(batch) * m->rows}, scratch);
    });
}

int ref_head_matmul(const ao_head_chunk *h, const float *inputs,
                    std::uint32_t batch, float *outputs) {
    return guarded([&] {
        const std::size_t packed =
            static_cast<std::size_t>(h->rows) * h->columns / 8 * 5;
        const std::size_t scales =
            static_cast<std::size_t>(h->rows) * (h->columns / 64);
        const adi::MachHeadChunk head{
            h->rows,
            h->columns,
            {h->packed, packed},
            u16(h->group_scale_f16, scales),
            {h->protected_rows, h->protected_count},
            u16(h->protected_bf16,
                static_cast<std::size_t>(h->protected_count) * h->columns),
        };
        adi::mach_head_matmul(
            head, {inputs, static_cast<std::size_t>(batch) * h->columns}, batch,
            {outputs, static_cast<std::size_t>(batch) * h->rows});
    });
}

int ref_bf16_matmul(const ao_bf16_matrix *m, const float *inputs,
                    std::uint32_t batch, float *outputs) {
    return guarded([&] {
        adi::bf16_matmul(
            bf16_view(*m),
            {inputs, static_cast<std::size_t>(batch) * m->columns}, batch,
            {outputs, static_cast<std::size_t>(batch) * m->rows});
    });
}

int ref_rms_norm(const float *input, const std::uint16_t *weight_bf16,
                 std::uint32_t count, float weight_offset, float epsilon,
                 float *output) {
    return guarded([&] {
        adi::rms_norm({input, count}, {weight_bf16, count}, weight_offset,
                      epsilon, {output, count});
    });
}

int ref_embedding_row(const ao_embedding *e, std::uint32_t token, float *output) {
    return guarded([&] {
        const std::size_t groups = e->columns / 64;
        const adi::MachEmbedding view{
            e->rows,
            e->columns,
            {e->packed, static_cast<std::size_t>(e->rows) * e->columns / 2},
            u16(e->minimum_f16, e->rows * groups),
            u16(e->maximum_f16, e->rows * groups),
            {e->exception_indexes, e->exception_count},
            u16(e->exception_bf16, e->exception_count),
        };
        adi::mach_embedding_row(view, token, {output, e->columns});
    });
}

/* sample_token (src/generation.cpp:161-225) with a std::mt19937_64 seeded
 * with `seed`; *first_word receives the engine's first output, the one word a
 * draw at temperature > 0 consumes. */
int ref_sample_token(const float *logits, std::uint32_t count, float temperature, float top_p,
                     std::uint64_t seed, std::uint64_t *first_word, std::uint32_t *token) {
    return guarded([&] {
        std::mt19937_64 random(seed);
        std::mt19937_64 copy = random;
        *first_word = copy();
        *token = adi::sample_token({logits, count}, temperature, top_p, random);
    });
}

/* GgufFile (src/gguf.cpp:232-330) on `path`: AO_OK with the counts, or
 * AO_INVALID_ARGUMENT when the reader rejects the file. */
int ref_gguf_summary(const char *path, std::uint64_t *tensors, std::uint64_t *metadata,
                     std::uint64_t *alignment) {
    return guarded([&] {
        const adi::GgufFile file(path);
        *tensors = file.tensors().size();
        *metadata = file.metadata().size();
        *alignment = file.alignment();
    });
}

int ref_top_experts(const float *logits, std::uint32_t count,
                    std::uint32_t *experts, float *weights) {
    return guarded([&] {
        const auto routes = adi::top_experts({logits, count});
        for (std::size_t i = 0; i < routes.size(); ++i) {
            experts[i] = routes[i].expert;
            weights[i] = routes[i].weight;
        }
    });
}

void *ref_moe_layer_create(const ao_moe_layer *desc) {
    try {
        auto layer = std::make_unique<RefLayer>();
        layer->hidden = desc->hidden;
        layer->expert_hidden = desc->expert_hidden;
        layer->experts = desc->experts;
        layer->router = bf16_view(desc->router);
        layer->shared_expert_gate = bf16_view(desc->shared_expert_gate);
        const auto *first = &desc->expert_matrices[0];
        layer->expert_state_values =
            adi::detail::build_expert_state_values({first->tlut, 32768 * 8});
        layer->ne_state_values =
            adi::detail::build_ne_state_values({desc->shared_gate.tlut, 512 * 2});
        layer->ne_signed_tlut =
            adi::detail::build_ne_signed_tlut({desc->shared_gate.tlut, 512 * 2});
        layer->waves_forward = adi::detail::build_wave_indexes(
            desc->expert_hidden / 16, desc->hidden / 16);
        layer->waves_reverse = adi::detail::build_wave_indexes(
            desc->hidden / 16, desc->expert_hidden / 16);
        const std::size_t gamma_per = (desc->hidden + desc->expert_hidden) / 16;
        layer->gamma.resize(static_cast<std::size_t>(desc->experts) * 3 * gamma_per);
        layer->matrices.resize(desc->experts);
        for (std::uint32_t e = 0; e < desc->experts; ++e) {
            for (int p = 0; p < 3; ++p) {
                const auto &src = desc->expert_matrices[e * 3 + p];
                auto view = expert_view(src);
                float *g = layer->gamma.data() + (static_cast<std::size_t>(e) * 3 + p) * gamma_per;
                for (std::size_t i = 0; i < gamma_per; ++i) {
                    g[i] = adi::f16_to_f32(src.wave_gamma_f16[i]);
                }
                view.state_values = layer->expert_state_values;
                view.wave_indexes = p == 2 ? std::span<const std::uint16_t>(layer->waves_reverse)
                                           : std::span<const std::uint16_t>(layer->waves_forward);
                view.wave_gamma = {g, gamma_per};
                layer->matrices[e][p] = view;
            }
        }
        const ao_ne_matrix *shared[3] = {&desc->shared_gate, &desc->shared_up,
                                         &desc->shared_down};
        for (int p = 0; p < 3; ++p) {
            layer->shared[p] = ne_view(*shared[p]);
            layer->shared[p].state_values = layer->ne_state_values;
            layer->shared[p].signed_tlut = layer->ne_signed_tlut;
        }
        return layer.release();
    } catch (const std::exception &) {
        return nullptr;
    }
}

void ref_moe_layer_destroy(void *handle) {
    delete static_cast<RefLayer *>(handle);
}

// One MoE block. logit_bias (nullable, [experts]) is added between the router
// and top_experts. route_expert/route_weight (nullable) receive [batch*8].
int ref_moe_forward(void *handle, const float *inputs, std::uint32_t batch,
                    const float *logit_bias, float *outputs,
                    std::uint32_t *route_expert, float *route_weight) {
    return guarded([&] {
        auto &L = *static_cast<RefLayer *>(handle);
        const auto H = L.hidden, I = L.expert_hidden, E = L.experts;
        if (batch == 0) {
            throw std::invalid_argument("MoE batch shape mismatch");
        }
        if (batch == 1) {
            // moe_forward (src/executor.cpp:242-330)
            auto &s = L.moe_scratch;
            const std::span<const float> input(inputs, H);
            const std::span<float> output(outputs, H);
            s.router_logits.resize(E);
            adi::bf16_matvec(L.router, input, s.router_logits);
            if (logit_bias != nullptr) {
                for (std::uint32_t e = 0; e < E; ++e) {
                    s.router_logits[e] += logit_bias[e];
                }
            }
            const auto routes = adi::top_experts(s.router_logits);
            std::fill(output.begin(), output.end(), 0.0F);
            adi::detail::parallel_tasks(8, [&](std::uint32_t r) {
                auto &w = s.experts[r];
                w.gate.resize(I);
                w.up.resize(I);
                w.activated.resize(I);
                w.projected.resize(H);
                const auto &m = L.matrices[routes[r].expert];
                adi::mach_expert_matvec(m[0], input, w.gate, w.codec);
                adi::mach_expert_matvec(m[1], input, w.up, w.codec);
                for (std::size_t i = 0; i < I; ++i) {
                    w.activated[i] = adi::silu(w.gate[i]) * w.up[i];
                }
                adi::mach_expert_matvec(m[2], w.activated, w.projected, w.codec);
            });
            for (std::size_t r = 0; r < 8; ++r) {
                for (std::size_t i = 0; i < H; ++i) {
                    output[i] += routes[r].weight * s.experts[r].projected[i];
                }
            }
            s.shared_gate.resize(I);
            s.shared_up.resize(I);
            s.shared_down.resize(H);
            adi::mach_ne_matvec(L.shared[0], input, s.shared_gate, s.shared_codec);
            adi::mach_ne_matvec(L.shared[1], input, s.shared_up, s.shared_codec);
            for (std::size_t i = 0; i < I; ++i) {
                s.shared_gate[i] = adi::silu(s.shared_gate[i]) * s.shared_up[i];
            }
            adi::mach_ne_matvec(L.shared[2], s.shared_gate, s.shared_down, s.shared_codec);
            float shared_weight = 0.0F;
            adi::bf16_matvec(L.shared_expert_gate, input, {&shared_weight, 1});
            shared_weight = adi::sigmoid(shared_weight);
            for (std::size_t i = 0; i < H; ++i) {
                output[i] += shared_weight * s.shared_down[i];
            }
            for (std::size_t r = 0; r < 8; ++r) {
                if (route_expert) route_expert[r] = routes[r].expert;
                if (route_weight) route_weight[r] = routes[r].weight;
            }
            return;
        }

        // moe_forward_batch (src/executor.cpp:1181-1453)
        constexpr std::uint32_t routes_per_token = 8;
        constexpr std::uint32_t rows_per_task = 32;
        auto &bs = L.batch_scratch;
        auto &s = bs.moe;
        const std::size_t positions = static_cast<std::size_t>(batch) * routes_per_token;
        const std::span<const float> in(inputs, static_cast<std::size_t>(batch) * H);
        const std::span<float> out(outputs, static_cast<std::size_t>(batch) * H);
        s.router_logits.resize(static_cast<std::size_t>(batch) * E);
        adi::bf16_matmul(L.router, in, batch, s.router_logits);
        if (logit_bias != nullptr) {
            for (std::uint32_t b = 0; b < batch; ++b) {
                for (std::uint32_t e = 0; e < E; ++e) {
                    s.router_logits[static_cast<std::size_t>(b) * E + e] += logit_bias[e];
                }
            }
        }
        s.routes.resize(batch);
        s.counts.assign(E, 0);
        s.offsets.resize(static_cast<std::size_t>(E) + 1);
        s.cursors.resize(E);
        s.active.clear();
        s.grouped_batch.resize(positions);
        s.route_to_grouped.resize(positions);
        for (std::uint32_t b = 0; b < batch; ++b) {
            s.routes[b] = adi::top_experts(
                std::span<const float>(s.router_logits).subspan(static_cast<std::size_t>(b) * E, E),
                s.route_order);
            for (std::uint32_t r = 0; r < routes_per_token; ++r) {
                ++s.counts[s.routes[b][r].expert];
            }
        }
        std::uint32_t total = 0;
        for (std::uint32_t e = 0; e < E; ++e) {
            s.offsets[e] = total;
            s.cursors[e] = total;
            total += s.counts[e];
            if (s.counts[e] != 0) {
                s.active.push_back(e);
            }
        }
        s.offsets[E] = total;
        for (std::uint32_t b = 0; b < batch; ++b) {
            for (std::uint32_t r = 0; r < routes_per_token; ++r) {
                const auto e = s.routes[b][r].expert;
                const auto position = s.cursors[e]++;
                s.grouped_batch[position] = b;
                s.route_to_grouped[static_cast<std::size_t>(b) * routes_per_token + r] = position;
            }
        }
        s.gathered.resize(positions * H);
        s.gate.resize(positions * I);
        s.up.resize(s.gate.size());
        s.activated.resize(s.gate.size());
        s.projected.resize(s.gathered.size());
        adi::detail::parallel_ranges(
            static_cast<std::uint32_t>(positions), 64,
            [&](std::uint32_t begin, std::uint32_t end) {
                for (auto p = begin; p < end; ++p) {
                    std::copy_n(in.begin() + static_cast<std::size_t>(s.grouped_batch[p]) * H, H,
                                s.gathered.begin() + static_cast<std::size_t>(p) * H);
                }
            });
        s.tasks.clear();
        for (const auto e : s.active) {
            const auto rows = s.counts[e];
            const auto begin = s.offsets[e];
            const auto chunks = (rows + rows_per_task - 1) / rows_per_task;
            std::uint32_t placed = 0;
            for (std::uint32_t c = 0; c < chunks; ++c) {
                const auto chunk_rows = (rows - placed) / (chunks - c);
                s.tasks.push_back({e, begin + placed, chunk_rows});
                placed += chunk_rows;
            }
        }
        adi::detail::parallel_dynamic(
            static_cast<std::uint32_t>(s.tasks.size()), [&](std::uint32_t t) {
                const auto task = s.tasks[t];
                const auto ho = static_cast<std::size_t>(task.begin) * H;
                const auto eo = static_cast<std::size_t>(task.begin) * I;
                const auto hs = static_cast<std::size_t>(task.rows) * H;
                const auto es = static_cast<std::size_t>(task.rows) * I;
                thread_local adi::ExpertScratch codec;
                const auto gathered = std::span<const float>(s.gathered).subspan(ho, hs);
                auto gate = std::span<float>(s.gate).subspan(eo, es);
                auto up = std::span<float>(s.up).subspan(eo, es);
                auto act = std::span<float>(s.activated).subspan(eo, es);
                auto proj = std::span<float>(s.projected).subspan(ho, hs);
                const auto &m = L.matrices[task.expert];
                adi::mach_expert_matmul(m[0], gathered, task.rows, gate, codec);
                adi::mach_expert_matmul(m[1], gathered, task.rows, up, codec);
                for (std::size_t i = 0; i < act.size(); ++i) {
                    act[i] = adi::silu(gate[i]) * up[i];
                }
                adi::mach_expert_matmul(m[2], act, task.rows, proj, codec);
            });
        std::fill(out.begin(), out.end(), 0.0F);
        for (std::uint32_t b = 0; b < batch; ++b) {
            for (std::uint32_t r = 0; r < routes_per_token; ++r) {
                const auto position = s.route_to_grouped[static_cast<std::size_t>(b) * routes_per_token + r];
                const float w = s.routes[b][r].weight;
                const float *src = s.projected.data() + static_cast<std::size_t>(position) * H;
                float *dst = outputs + static_cast<std::size_t>(b) * H;
                for (std::uint32_t i = 0; i < H; ++i) {
                    dst[i] += w * src[i];
                }
            }
        }
        bs.projection_0.resize(static_cast<std::size_t>(batch) * I);
        bs.projection_1.resize(static_cast<std::size_t>(batch) * I);
        adi::mach_ne_matmul(L.shared[0], in, batch, bs.projection_0, bs.codec);
        adi::mach_ne_matmul(L.shared[1], in, batch, bs.projection_1, bs.codec);
        for (std::size_t i = 0; i < bs.projection_0.size(); ++i) {
            bs.projection_0[i] = adi::silu(bs.projection_0[i]) * bs.projection_1[i];
        }
        bs.projection_2.resize(static_cast<std::size_t>(batch) * H);
        adi::mach_ne_matmul(L.shared[2], bs.projection_0, batch, bs.projection_2, bs.codec);
        bs.projection_3.resize(batch);
        adi::bf16_matmul(L.shared_expert_gate, in, batch, bs.projection_3);
        for (std::uint32_t b = 0; b < batch; ++b) {
            const float w = adi::sigmoid(bs.projection_3[b]);
            for (std::uint32_t i = 0; i < H; ++i) {
                outputs[static_cast<std::size_t>(b) * H + i] +=
                    w * bs.projection_2[static_cast<std::size_t>(b) * H + i];
            }
        }
        for (std::uint32_t b = 0; b < batch; ++b) {
            for (std::uint32_t r = 0; r < routes_per_token; ++r) {
                const std::size_t k = static_cast<std::size_t>(b) * routes_per_token + r;
                if (route_expert) route_expert[k] = s.routes[b][r].expert;
                if (route_weight) route_weight[k] = s.routes[b][r].weight;
            }
        }
    });
}

// detail::grouped_query_online_attention (src/attention.cpp:38-229), heads
// in one pass (its sequential form).
int ref_grouped_attention(const float *queries, const float *keys, const float *values,
                          std::uint32_t tokens, std::uint32_t query_heads,
                          std::uint32_t kv_heads, std::uint32_t head_size,
                          std::uint32_t query_stride, float *output) {
    return guarded([&] {
        const std::size_t kv = static_cast<std::size_t>(tokens) * kv_heads * head_size;
        adi::detail::grouped_query_online_attention(
            {queries, static_cast<std::size_t>(query_heads) * query_stride}, {keys, kv},
            {values, kv}, query_heads, kv_heads, head_size, query_stride, false,
            {output, static_cast<std::size_t>(query_heads) * head_size});
    });
}

// detail::gated_delta_update (src/simd.cpp) of the selected ISA.
float ref_gated_delta_update(float *state, const float *query, const float *key, float value,
                             float beta, float decay, std::uint32_t count) {
    return adi::detail::gated_delta_update({state, count}, {query, count}, {key, count}, value,
                                           beta, decay);
}

int ref_l2_normalize(float *values, std::uint32_t count, float epsilon) {
    return guarded([&] { adi::l2_normalize({values, count}, epsilon); });
}

// gated_delta_key_head (src/executor.cpp:231-240); UINT32_MAX where it throws.
uint32_t ref_gated_delta_key_head(uint32_t value_head, uint32_t value_heads, uint32_t key_heads) {
    try {
        return adi::gated_delta_key_head(value_head, value_heads, key_heads);
    } catch (const std::exception &) {
        return UINT32_MAX;
    }
}

} // extern "C"
