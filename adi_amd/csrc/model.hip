// model.hip -- the model-level entry points: a decode step over many
// sequences (decode_batch, src/executor.cpp:1592-1825; decode_token is its
// one-sequence case) and the prefill of a prompt in micro-batches
// (prefill_prompt, src/generation.cpp:131-159, over prefill,
// src/executor.cpp:1827-2101). Every argument is checked before anything is
// launched, so a rejected call leaves the states and outputs as they were.
#include "attention.hpp"
#include "dense.hpp"

#include <vector>

namespace adi_hip {
namespace {

constexpr uint32_t kDefaultUbatch = 128;  // ExecutionOptions::prefill_ubatch
constexpr uint32_t kMaxUbatch = 4096;
constexpr uint32_t kTokenWords = 64;
constexpr uint32_t kSpanStep = 512;  // a captured step covers positions in steps of this

struct TokenWords {
    uint32_t token[kTokenWords];
};

// Host tokens reach the device as kernel arguments, in stream order with
// the kernels that read them.
__global__ __launch_bounds__(64) void k_store_tokens(uint32_t *dst, TokenWords words,
                                                     uint32_t count) {
    const uint32_t i = threadIdx.x;
    if (i < count) {
        dst[i] = words.token[i];
    }
}

// The last launch of a captured decode step: every sequence's position
// advances by one, so the next replay runs at the next positions.
__global__ __launch_bounds__(256) void k_advance_positions(uint32_t *positions, uint32_t count) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < count) {
        positions[i] += 1u;
    }
}

// A decode step's tokens and positions, 32 rows a launch.
__global__ __launch_bounds__(64) void k_store_step(uint32_t *tokens, uint32_t *positions,
                                                   TokenWords words, uint32_t count) {
    const uint32_t i = threadIdx.x;
    if (i < count) {
        tokens[i] = words.token[i];
    } else if (i >= kTokenWords / 2 && i - kTokenWords / 2 < count) {
        positions[i - kTokenWords / 2] = words.token[i];
    }
}

void upload_step(adi_hip_context *ctx, uint32_t *device_tokens, uint32_t *device_positions,
                 const uint32_t *tokens, const uint32_t *positions, uint32_t count) {
    constexpr uint32_t kRows = kTokenWords / 2;
    for (uint32_t first = 0; first < count; first += kRows) {
        const uint32_t n = count - first < kRows ? count - first : kRows;
        TokenWords words{};
        for (uint32_t i = 0; i < n; ++i) {
            words.token[i] = tokens[first + i];
            words.token[kRows + i] = positions[first + i];
        }
        launch(ctx, "store_step", k_store_step, dim3(1), dim3(64), 0, device_tokens + first,
               device_positions + first, words, n);
    }
}

void upload_tokens(adi_hip_context *ctx, uint32_t *dst, const uint32_t *tokens, uint32_t count) {
    for (uint32_t first = 0; first < count; first += kTokenWords) {
        const uint32_t n = count - first < kTokenWords ? count - first : kTokenWords;
        TokenWords words{};
        for (uint32_t i = 0; i < n; ++i) {
            words.token[i] = tokens[first + i];
        }
        launch(ctx, "store_tokens", k_store_tokens, dim3(1), dim3(64), 0, dst + first, words, n);
    }
}

void forward_status(adi_hip_context *ctx, int status) {
    if (status != ADI_HIP_OK) {
        fail(status, ctx->last_error());
    }
}

struct ModelShape {
    uint32_t hidden;
    uint32_t vocabulary;
    uint32_t widest_chunk;
};

ModelShape validate_model(const adi_hip_model *m) {
    require(m != nullptr && m->layers > 0 && m->layer != nullptr && m->embedding != nullptr &&
                m->final_norm != nullptr && m->head_chunks > 0 && m->head != nullptr &&
                m->context > 0,
            "model descriptor is incomplete");
    ModelShape shape{m->embedding->columns, m->embedding->rows, 0};
    require(shape.hidden > 0 && shape.vocabulary > 0, "model embedding shape mismatch");
    uint64_t rows = 0;
    for (uint32_t c = 0; c < m->head_chunks; ++c) {
        require(m->head[c].columns == shape.hidden && m->head[c].rows > 0,
                "model head chunk shape mismatch");
        rows += m->head[c].rows;
        shape.widest_chunk = m->head[c].rows > shape.widest_chunk ? m->head[c].rows : shape.widest_chunk;
    }
    require(rows == shape.vocabulary, "model head chunks do not cover the vocabulary");
    for (uint32_t l = 0; l < m->layers; ++l) {
        require(m->layer[l].moe.hidden == shape.hidden, "model layer hidden size mismatch");
    }
    return shape;
}

// Every layer state of a sequence about to take `tokens` tokens.
void validate_state(const adi_hip_model *m, const adi_hip_decoder_state &s, uint32_t tokens,
                    const char *message) {
    require(s.layers != nullptr, message);
    for (uint32_t l = 0; l < m->layers; ++l) {
        const adi_hip_layer_state &st = s.layers[l];
        if (m->layer[l].full_attention != 0) {
            require(st.keys != nullptr && st.values != nullptr && st.capacity >= tokens &&
                        s.position <= st.capacity - tokens,
                    message);
        } else {
            require(st.convolution != nullptr && st.recurrent != nullptr, message);
        }
    }
}

// The final norm of rows[rows][hidden] + pending (the last layer's MoE
// rows, added in place first) and the head chunks into
// logits[rows][vocabulary].
void model_logits(adi_hip_context *ctx, const adi_hip_model *m, const ModelShape &shape,
                  float *hidden, const float *pending, uint32_t rows, float *normalized,
                  float *staging, float *logits) {
    launch_add_rms_norm(ctx, hidden, pending, m->final_norm, shape.hidden, rows, normalized);
    size_t offset = 0;
    for (uint32_t c = 0; c < m->head_chunks; ++c) {
        const adi_hip_head_chunk &h = m->head[c];
        if (rows == 1 || m->head_chunks == 1) {
            forward_status(ctx, adi_hip_head_matmul(ctx, &h, normalized, rows, logits + offset));
        } else {
            forward_status(ctx, adi_hip_head_matmul(ctx, &h, normalized, rows, staging));
            if (!ctx->dry_run) {
                check_hip(hipMemcpy2DAsync(logits + offset, size_t(shape.vocabulary) * 4, staging,
                                           size_t(h.rows) * 4, size_t(h.rows) * 4, rows,
                                           hipMemcpyDeviceToDevice, ctx->stream),
                          "head chunk copy");
            }
        }
        offset += h.rows;
    }
}

// The launches of one decode step over `batch` sequences (everything after
// the tokens and positions reach the device): embedding rows of
// device_tokens, every layer at device_positions, the final norm and the
// head. positions[] are the same positions on the host (checks, the RoPE
// table); the attention launches cover positions below `span`.
void decode_body(adi_hip_context *ctx, const adi_hip_model *m, const ModelShape &shape,
                 const uint32_t *device_tokens, const uint32_t *device_positions,
                 const uint32_t *positions, uint32_t batch, const adi_hip_decoder_state *states,
                 float *logits, uint32_t span, float *hidden, float *normalized, float *moe_rows,
                 float *staging) {
    forward_status(ctx, adi_hip_embedding_rows(ctx, m->embedding, device_tokens, batch, hidden));
    std::vector<const adi_hip_layer_state *> layer_states(batch);
    // each layer's MoE rows are added by the next layer's first norm, the
    // last layer's by the final norm (not at all without logits: nothing
    // reads the hidden rows then)
    for (uint32_t l = 0; l < m->layers; ++l) {
        for (uint32_t b = 0; b < batch; ++b) {
            layer_states[b] = &states[b].layers[l];
        }
        decoder_rows(ctx, &m->layer[l], batch, hidden, l > 0 ? moe_rows : nullptr, moe_rows,
                     layer_states.data(), positions, device_positions, span);
    }
    if (logits != nullptr) {
        model_logits(ctx, m, shape, hidden, moe_rows, batch, normalized, staging, logits);
    }
}

// The step's device buffers in the sequence workspace.
struct StepBuffers {
    uint32_t *tokens;
    uint32_t *positions;
    float *hidden;
    float *normalized;
    float *moe_rows;
    float *staging;
};

StepBuffers step_buffers(adi_hip_context *ctx, const adi_hip_model *m, const ModelShape &shape,
                         uint32_t batch, bool with_logits) {
    auto &ws = ctx->sequence_workspace;
    ws.used = 0;
    const size_t rows = batch;
    const bool staged = with_logits && batch > 1 && m->head_chunks > 1;
    ws.ensure(Workspace::round(rows * 4) * 2 + Workspace::round(rows * shape.hidden * 4) * 3 +
              (staged ? Workspace::round(rows * shape.widest_chunk * 4) : 0));
    StepBuffers b{};
    b.tokens = ws.take<uint32_t>(rows);
    b.positions = ws.take<uint32_t>(rows);
    b.hidden = ws.take<float>(rows * shape.hidden);
    b.normalized = ws.take<float>(rows * shape.hidden);
    b.moe_rows = ws.take<float>(rows * shape.hidden);
    b.staging = staged ? ws.take<float>(rows * shape.widest_chunk) : nullptr;
    return b;
}

void decode_rows(adi_hip_context *ctx, const adi_hip_model *m, const ModelShape &shape,
                 const uint32_t *tokens, uint32_t batch, adi_hip_decoder_state *states,
                 float *logits) {
    const StepBuffers buf = step_buffers(ctx, m, shape, batch, logits != nullptr);
    std::vector<uint32_t> positions(batch);
    for (uint32_t b = 0; b < batch; ++b) {
        positions[b] = states[b].position;
    }
    upload_step(ctx, buf.tokens, buf.positions, tokens, positions.data(), batch);
    decode_body(ctx, m, shape, buf.tokens, buf.positions, positions.data(), batch, states, logits,
                0, buf.hidden, buf.normalized, buf.moe_rows, buf.staging);
}

void check_decode_step(const adi_hip_model *model, const ModelShape &shape, uint32_t batch,
                       const adi_hip_decoder_state *states) {
    require(batch > 0 && states != nullptr, "decoder batch shape mismatch");
    for (uint32_t b = 0; b < batch; ++b) {
        if (states[b].position >= model->context) {
            fail(ADI_HIP_OUT_OF_RANGE, "decoder context is exhausted");
        }
    }
    for (uint32_t b = 0; b < batch; ++b) {
        validate_state(model, states[b], 1, "decoder batch state mismatch");
    }
    (void)shape;
}

}  // namespace
}  // namespace adi_hip

using namespace adi_hip;

// A decode step captured as a HIP graph: the launches of adi_hip_decode_batch
// for one set of sequences, reading the step's tokens from the caller's
// device array and the positions from the graph's own, which the graph's
// last launch advances.
struct adi_hip_decode_graph {
    adi_hip_context *ctx = nullptr;
    // copies of the model descriptor and of each sequence's layer states, as
    // captured (the device memory they point to belongs to the caller)
    adi_hip_model model{};
    std::vector<adi_hip_decoder_layer> layers;
    std::vector<adi_hip_head_chunk> heads;
    adi_hip_embedding embedding{};
    ModelShape shape{};
    uint32_t batch = 0;
    std::vector<std::vector<adi_hip_layer_state>> sequences;
    std::vector<adi_hip_decoder_state> states;
    std::vector<uint32_t> positions;  // the positions the next replay runs at
    uint32_t *device_positions = nullptr;
    const uint32_t *tokens = nullptr;  // the caller's device array
    float *logits = nullptr;
    uint32_t span = 0;
    std::vector<void *> bases;  // the context's arenas when captured
    hipStream_t stream = nullptr;  // the capture stream when the context's is the null stream
    hipGraphExec_t exec = nullptr;
    uint32_t captures = 0;
};

namespace adi_hip {
namespace {

void release_capture(adi_hip_decode_graph *g) {
    if (g->exec != nullptr) {
        (void)hipGraphExecDestroy(g->exec);
        g->exec = nullptr;
    }
}

void free_decode_graph(adi_hip_decode_graph *g) {
    release_capture(g);
    if (g->device_positions != nullptr) {
        (void)hipFree(g->device_positions);
    }
    if (g->stream != nullptr) {
        (void)hipStreamDestroy(g->stream);
    }
    delete g;
}

// Records one step at the graph's positions. A planning pass runs the host
// side of the step first without launching (checks, workspace and RoPE
// growth), so nothing allocates or synchronizes while the stream captures.
void capture(adi_hip_decode_graph *g) {
    adi_hip_context *ctx = g->ctx;
    release_capture(g);
    uint32_t last = 0;
    for (uint32_t p : g->positions) {
        last = p + 1 > last ? p + 1 : last;
    }
    g->span = ((last + kSpanStep - 1) / kSpanStep) * kSpanStep;
    const StepBuffers buf = step_buffers(ctx, &g->model, g->shape, g->batch, g->logits != nullptr);
    ctx->dry_run = true;
    try {
        decode_body(ctx, &g->model, g->shape, g->tokens, g->device_positions, g->positions.data(),
                    g->batch, g->states.data(), g->logits, g->span, buf.hidden, buf.normalized,
                    buf.moe_rows, buf.staging);
    } catch (...) {
        ctx->dry_run = false;
        throw;
    }
    ctx->dry_run = false;
    const hipStream_t saved = ctx->stream;
    if (saved == nullptr && g->stream == nullptr) {
        check_hip(hipStreamCreateWithFlags(&g->stream, hipStreamNonBlocking), "graph stream");
    }
    const hipStream_t stream = saved != nullptr ? saved : g->stream;
    if (saved == nullptr) {
        // the capture stream starts after the work already queued
        check_hip(hipStreamSynchronize(nullptr), "graph capture synchronize");
    }
    const auto arenas = ctx->arenas();
    g->bases.clear();
    for (Workspace *w : arenas) {
        g->bases.push_back(w->base);
        w->frozen = true;
    }
    hipGraph_t graph = nullptr;
    ctx->stream = stream;
    check_hip(hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal), "graph capture");
    try {
        const StepBuffers again = step_buffers(ctx, &g->model, g->shape, g->batch,
                                               g->logits != nullptr);
        decode_body(ctx, &g->model, g->shape, g->tokens, g->device_positions, g->positions.data(),
                    g->batch, g->states.data(), g->logits, g->span, again.hidden,
                    again.normalized, again.moe_rows, again.staging);
        launch(ctx, "advance_positions", k_advance_positions, dim3(ceil_div(g->batch, 256)),
               dim3(256), 0, g->device_positions, g->batch);
    } catch (...) {
        (void)hipStreamEndCapture(stream, &graph);
        if (graph != nullptr) {
            (void)hipGraphDestroy(graph);
        }
        ctx->stream = saved;
        for (Workspace *w : arenas) {
            w->frozen = false;
        }
        throw;
    }
    ctx->stream = saved;
    for (Workspace *w : arenas) {
        w->frozen = false;
    }
    check_hip(hipStreamEndCapture(stream, &graph), "graph capture end");
    const hipError_t made = hipGraphInstantiate(&g->exec, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    check_hip(made, "graph instantiate");
    ++g->captures;
}

bool arenas_moved(adi_hip_decode_graph *g) {
    const auto arenas = g->ctx->arenas();
    for (size_t i = 0; i < arenas.size(); ++i) {
        if (arenas[i]->base != g->bases[i]) {
            return true;
        }
    }
    return false;
}

bool same_layer_state(const adi_hip_layer_state &a, const adi_hip_layer_state &b) {
    return a.keys == b.keys && a.values == b.values && a.capacity == b.capacity &&
           a.convolution == b.convolution && a.recurrent == b.recurrent;
}

}  // namespace
}  // namespace adi_hip

extern "C" {

int adi_hip_decode_batch(adi_hip_context *ctx, const adi_hip_model *model, const uint32_t *tokens,
                         uint32_t batch, adi_hip_decoder_state *states, float *logits) {
    return guarded(ctx, [&] {
        const ModelShape shape = validate_model(model);
        require(batch > 0 && tokens != nullptr && states != nullptr, "decoder batch shape mismatch");
        for (uint32_t b = 0; b < batch; ++b) {
            require(tokens[b] < shape.vocabulary, "decoder batch token is out of range");
        }
        check_decode_step(model, shape, batch, states);
        decode_rows(ctx, model, shape, tokens, batch, states, logits);
        for (uint32_t b = 0; b < batch; ++b) {
            ++states[b].position;
        }
    });
}

int adi_hip_prefill(adi_hip_context *ctx, const adi_hip_model *model, const uint32_t *tokens,
                    uint32_t count, uint32_t ubatch, adi_hip_decoder_state *state, float *logits) {
    return guarded(ctx, [&] {
        const ModelShape shape = validate_model(model);
        require(tokens != nullptr && state != nullptr && count > 0 &&
                    state->position < model->context && count <= model->context - state->position,
                "prefill shape or context is invalid");
        for (uint32_t i = 0; i < count; ++i) {
            require(tokens[i] < shape.vocabulary, "prefill token is out of range");
        }
        const uint32_t chunk = ubatch == 0 ? kDefaultUbatch : ubatch;
        require(chunk <= kMaxUbatch, "prefill_ubatch must be in [1, 4096]");
        validate_state(model, *state, count, "prefill state mismatch");
        auto &ws = ctx->sequence_workspace;
        ws.used = 0;
        const uint32_t rows = count < chunk ? count : chunk;
        ws.ensure(Workspace::round(size_t(count) * 4) +
                  Workspace::round(size_t(rows) * shape.hidden * 4) * 2 +
                  Workspace::round(size_t(shape.hidden) * 4));
        uint32_t *device_tokens = ws.take<uint32_t>(count);
        float *hidden = ws.take<float>(size_t(rows) * shape.hidden);
        float *moe_rows = ws.take<float>(size_t(rows) * shape.hidden);
        float *normalized = ws.take<float>(shape.hidden);
        const uint32_t start = state->position;
        upload_tokens(ctx, device_tokens, tokens, count);
        uint32_t n = 0;
        for (uint32_t offset = 0; offset < count; offset += n) {
            n = count - offset < chunk ? count - offset : chunk;
            forward_status(ctx, adi_hip_embedding_rows(ctx, model->embedding, device_tokens + offset,
                                                       n, hidden));
            for (uint32_t l = 0; l < model->layers; ++l) {
                prefill_chunk(ctx, &model->layer[l], start + offset, n, hidden,
                              l > 0 ? moe_rows : nullptr, moe_rows, &state->layers[l]);
            }
        }
        if (logits != nullptr) {
            const size_t last = size_t(n - 1) * shape.hidden;
            model_logits(ctx, model, shape, hidden + last, moe_rows + last, 1, normalized, nullptr,
                         logits);
        }
        state->position += count;
    });
}

int adi_hip_decode_graph_create(adi_hip_context *ctx, const adi_hip_model *model, uint32_t batch,
                                const adi_hip_decoder_state *states, const uint32_t *tokens,
                                float *logits, adi_hip_decode_graph **out) {
    return guarded(ctx, [&] {
        require(out != nullptr, "decode graph: null argument");
        *out = nullptr;
        require(!ctx->profiling, "decode graph: kernel profiling is on (its events cannot be captured)");
        const ModelShape shape = validate_model(model);
        require(tokens != nullptr, "decoder batch shape mismatch");
        check_decode_step(model, shape, batch, states);
        auto *g = new adi_hip_decode_graph;
        try {
            g->ctx = ctx;
            g->layers.assign(model->layer, model->layer + model->layers);
            g->heads.assign(model->head, model->head + model->head_chunks);
            g->embedding = *model->embedding;
            g->model = *model;
            g->model.layer = g->layers.data();
            g->model.head = g->heads.data();
            g->model.embedding = &g->embedding;
            g->shape = shape;
            g->batch = batch;
            g->tokens = tokens;
            g->logits = logits;
            g->sequences.resize(batch);
            g->states.resize(batch);
            for (uint32_t b = 0; b < batch; ++b) {
                g->sequences[b].assign(states[b].layers, states[b].layers + model->layers);
                g->states[b].layers = g->sequences[b].data();
                g->states[b].position = states[b].position;
                g->positions.push_back(states[b].position);
            }
            check_hip(hipMalloc(&g->device_positions, size_t(batch) * 4), "decode graph allocation");
            upload_tokens(ctx, g->device_positions, g->positions.data(), batch);
            capture(g);
        } catch (...) {
            free_decode_graph(g);
            throw;
        }
        *out = g;
    });
}

int adi_hip_decode_graph_launch(adi_hip_decode_graph *g, adi_hip_decoder_state *states) {
    if (g == nullptr) {
        return ADI_HIP_INVALID_ARGUMENT;
    }
    adi_hip_context *ctx = g->ctx;
    return guarded(ctx, [&] {
        require(states != nullptr, "decoder batch shape mismatch");
        require(!ctx->profiling, "decode graph: kernel profiling is on (its events cannot be captured)");
        for (uint32_t b = 0; b < g->batch; ++b) {
            require(states[b].layers != nullptr, "decoder batch state mismatch");
            for (uint32_t l = 0; l < g->model.layers; ++l) {
                require(same_layer_state(states[b].layers[l], g->sequences[b][l]),
                        "decode graph: the sequences differ from the captured ones");
            }
        }
        check_decode_step(&g->model, g->shape, g->batch, states);
        bool moved = false;
        uint32_t last = 0;
        for (uint32_t b = 0; b < g->batch; ++b) {
            moved = moved || states[b].position != g->positions[b];
            last = states[b].position + 1 > last ? states[b].position + 1 : last;
        }
        if (moved) {
            // positions set by the caller (a reset sequence): the graph's
            // array follows them
            for (uint32_t b = 0; b < g->batch; ++b) {
                g->positions[b] = states[b].position;
                g->states[b].position = states[b].position;
            }
            upload_tokens(ctx, g->device_positions, g->positions.data(), g->batch);
        }
        if (last > g->span || arenas_moved(g)) {
            capture(g);
        }
        const hipStream_t stream = ctx->stream;
        check_hip(hipGraphLaunch(g->exec, stream), "graph launch");
        if (g->batch == 1 && ctx->fused_moe) {
            ctx->moe_sync_pending = true;  // the one-launch MoE block's error word
        }
        for (uint32_t b = 0; b < g->batch; ++b) {
            ++g->positions[b];
            g->states[b].position = g->positions[b];
            states[b].position = g->positions[b];
        }
    });
}

uint32_t adi_hip_decode_graph_captures(const adi_hip_decode_graph *graph) {
    return graph == nullptr ? 0u : graph->captures;
}

void adi_hip_decode_graph_destroy(adi_hip_decode_graph *graph) {
    if (graph == nullptr) {
        return;
    }
    (void)hipStreamSynchronize(graph->ctx->stream);
    free_decode_graph(graph);
}

}  // extern "C"
