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
            check_hip(hipMemcpy2DAsync(logits + offset, size_t(shape.vocabulary) * 4, staging,
                                       size_t(h.rows) * 4, size_t(h.rows) * 4, rows,
                                       hipMemcpyDeviceToDevice, ctx->stream),
                      "head chunk copy");
        }
        offset += h.rows;
    }
}

void decode_rows(adi_hip_context *ctx, const adi_hip_model *m, const ModelShape &shape,
                 const uint32_t *tokens, uint32_t batch, adi_hip_decoder_state *states,
                 float *logits) {
    auto &ws = ctx->sequence_workspace;
    ws.used = 0;
    const size_t rows = batch;
    const bool staged = logits != nullptr && batch > 1 && m->head_chunks > 1;
    ws.ensure(Workspace::round(rows * 4) + Workspace::round(rows * shape.hidden * 4) * 3 +
              (staged ? Workspace::round(rows * shape.widest_chunk * 4) : 0));
    uint32_t *device_tokens = ws.take<uint32_t>(rows);
    float *hidden = ws.take<float>(rows * shape.hidden);
    float *normalized = ws.take<float>(rows * shape.hidden);
    float *moe_rows = ws.take<float>(rows * shape.hidden);
    float *staging = staged ? ws.take<float>(rows * shape.widest_chunk) : nullptr;
    upload_tokens(ctx, device_tokens, tokens, batch);
    forward_status(ctx, adi_hip_embedding_rows(ctx, m->embedding, device_tokens, batch, hidden));
    std::vector<const adi_hip_layer_state *> layer_states(batch);
    std::vector<uint32_t> positions(batch);
    for (uint32_t b = 0; b < batch; ++b) {
        positions[b] = states[b].position;
    }
    // each layer's MoE rows are added by the next layer's first norm, the
    // last layer's by the final norm (not at all without logits: nothing
    // reads the hidden rows then)
    for (uint32_t l = 0; l < m->layers; ++l) {
        for (uint32_t b = 0; b < batch; ++b) {
            layer_states[b] = &states[b].layers[l];
        }
        decoder_rows(ctx, &m->layer[l], batch, hidden, l > 0 ? moe_rows : nullptr, moe_rows,
                     layer_states.data(), positions.data());
    }
    if (logits != nullptr) {
        model_logits(ctx, m, shape, hidden, moe_rows, batch, normalized, staging, logits);
    }
}

}  // namespace
}  // namespace adi_hip

using namespace adi_hip;

extern "C" {

int adi_hip_decode_batch(adi_hip_context *ctx, const adi_hip_model *model, const uint32_t *tokens,
                         uint32_t batch, adi_hip_decoder_state *states, float *logits) {
    return guarded(ctx, [&] {
        const ModelShape shape = validate_model(model);
        require(batch > 0 && tokens != nullptr && states != nullptr, "decoder batch shape mismatch");
        for (uint32_t b = 0; b < batch; ++b) {
            require(tokens[b] < shape.vocabulary, "decoder batch token is out of range");
        }
        for (uint32_t b = 0; b < batch; ++b) {
            if (states[b].position >= model->context) {
                fail(ADI_HIP_OUT_OF_RANGE, "decoder context is exhausted");
            }
        }
        for (uint32_t b = 0; b < batch; ++b) {
            validate_state(model, states[b], 1, "decoder batch state mismatch");
        }
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

}  // extern "C"
