// attention.hip -- the attention half of a decode step on the device, for one
// token of one sequence:
//   full_attention_forward   (src/executor.cpp:332-418, src/attention.cpp)
//   linear_attention_forward (src/executor.cpp:420-557, Gated DeltaNet)
//
// Full attention, after the q/k/v projections:
//   norm_rope   one block per head: RMS norm with (1 + w), then RoPE on the
//               first 64 dimensions from a cos/sin table the host computes
//               with the same libm calls as the reference (prepare_rope);
//               the key lands in its cache slot, the value is projected there
//   partial     flash-decoding: block (head, split) runs the online softmax
//               over its share of the history, one wave per token stream,
//               and merges its four waves
//   combine     per head: merge the splits, times sigmoid(gate)
// Linear attention, after the projections:
//   conv        per 128-channel group: the width-4 causal convolution, SiLU,
//               the state shift, and the L2 norm of the query and key heads
//   delta       block (value head, 16 rows): the gated delta update of each
//               state row, one wave per row, state read and written once
//   norm_gate   per value head: RMS norm (weight offset 0) times SiLU(gate)
// The sums run in a different order from the CPU's (wave and block
// reductions); results agree to float rounding.
#include "dense.hpp"

#include <cmath>

namespace adi_hip {
namespace {

constexpr uint32_t kQueryHeads = 16;
constexpr uint32_t kKvHeads = 2;
constexpr uint32_t kHeadSize = 256;
constexpr uint32_t kQueryStride = 2 * kHeadSize;  // query then gate, per head
constexpr uint32_t kRopeHalf = 32;
constexpr uint32_t kMaxSplits = 64;
constexpr uint32_t kPartialStride = kHeadSize + 2;  // acc[256], maximum, denominator

constexpr uint32_t kKeyHeads = 16;
constexpr uint32_t kValueHeads = 32;
constexpr uint32_t kLinearHead = 128;
constexpr uint32_t kQkSize = kKeyHeads * kLinearHead;      // 2048
constexpr uint32_t kValueSize = kValueHeads * kLinearHead; // 4096
constexpr uint32_t kChannels = 2 * kQkSize + kValueSize;   // 8192
constexpr uint32_t kDeltaRows = 16;                        // state rows per block

constexpr float kEpsilon = 1.0e-6f;

struct RopeTable {
    float cosine[kRopeHalf];
    float sine[kRopeHalf];
};

__device__ __forceinline__ float wave_sum(float v) {
    v += lane_xor<1>(v);
    v += lane_xor<2>(v);
    v += lane_xor<4>(v);
    v += lane_xor<8>(v);
    v += lane_xor<16>(v);
    v += lane_xor<32>(v);
    return v;
}

// Sum over the block (blockDim.x a multiple of 64, at most 1024); every
// thread receives it. `partial` holds 16 floats.
__device__ __forceinline__ float block_sum(float v, float *partial) {
    v = wave_sum(v);
    const uint32_t waves = blockDim.x >> 6;
    if ((threadIdx.x & 63u) == 0) {
        partial[threadIdx.x >> 6] = v;
    }
    __syncthreads();
    float total = 0.0f;
    for (uint32_t w = 0; w < waves; ++w) {
        total += partial[w];
    }
    __syncthreads();
    return total;
}

__device__ __forceinline__ float silu_of(float v) { return v / (1.0f + expf(-v)); }
__device__ __forceinline__ float sigmoid_of(float v) { return 1.0f / (1.0f + expf(-v)); }

// normalize_head then apply_rope (src/executor.cpp:25-41, 60-72, 376-390):
// blocks 0-15 the query heads (stride 512), 16-17 the new key heads.
__global__ __launch_bounds__(kHeadSize) void k_norm_rope(float *query_gate, float *key,
                                                         const uint16_t *query_norm,
                                                         const uint16_t *key_norm, RopeTable rope) {
#pragma clang fp contract(off)
    __shared__ float partial[16];
    __shared__ float head[kHeadSize];
    const uint32_t h = blockIdx.x, t = threadIdx.x;
    float *v = h < kQueryHeads ? query_gate + static_cast<size_t>(h) * kQueryStride
                               : key + static_cast<size_t>(h - kQueryHeads) * kHeadSize;
    const uint16_t *w = h < kQueryHeads ? query_norm : key_norm;
    float x = v[t];
    const float squares = block_sum(x * x, partial);
    const float scale = 1.0f / sqrtf(squares / static_cast<float>(kHeadSize) + kEpsilon);
    x *= scale * (1.0f + bf16_bits_to_float(w[t]));
    head[t] = x;
    __syncthreads();
    if (t < kRopeHalf) {
        const float first = head[t], second = head[t + kRopeHalf];
        v[t] = first * rope.cosine[t] - second * rope.sine[t];
        v[t + kRopeHalf] = second * rope.cosine[t] + first * rope.sine[t];
    } else if (t >= 2 * kRopeHalf) {
        v[t] = x;
    }
}

// update_online_softmax (src/attention.cpp:15-35) on a lane's four values.
__device__ __forceinline__ void online_step(float score, float4 value, float &maximum,
                                            float &denominator, float4 &acc) {
#pragma clang fp contract(off)
    if (score <= maximum) {
        const float weight = expf(score - maximum);
        denominator += weight;
        acc.x += value.x * weight;
        acc.y += value.y * weight;
        acc.z += value.z * weight;
        acc.w += value.w * weight;
        return;
    }
    const float previous = expf(maximum - score);
    denominator = denominator * previous + 1.0f;
    acc.x = acc.x * previous + value.x;
    acc.y = acc.y * previous + value.y;
    acc.z = acc.z * previous + value.z;
    acc.w = acc.w * previous + value.w;
    maximum = score;
}

// Block (query head, split): tokens [split * chunk, min(tokens, ...)) of the
// head's KV stream, wave w taking every fourth. Lane l holds dimensions
// 4l..4l+3. Writes the split's accumulator, maximum and denominator.
__global__ __launch_bounds__(256) void k_attention_partial(const float *query_gate,
                                                           const float *keys, const float *values,
                                                           uint32_t tokens, uint32_t chunk,
                                                           float *partial) {
#pragma clang fp contract(off)
    __shared__ __align__(16) float wave_acc[4][kHeadSize];
    __shared__ float wave_max[4], wave_den[4];
    const uint32_t h = blockIdx.x, split = blockIdx.y, splits = gridDim.y;
    const uint32_t kv = h / (kQueryHeads / kKvHeads);
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const float4 q = reinterpret_cast<const float4 *>(query_gate + static_cast<size_t>(h) * kQueryStride)[lane];
    const float score_scale = 1.0f / 16.0f;  // 1 / sqrt(256)
    const uint32_t begin = split * chunk;
    const uint32_t end = begin + chunk < tokens ? begin + chunk : tokens;
    float maximum = -__builtin_huge_valf(), denominator = 0.0f;
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (uint32_t t = begin + wave; t < end; t += 4) {
        const size_t at = (static_cast<size_t>(t) * kKvHeads + kv) * kHeadSize;
        const float4 k = reinterpret_cast<const float4 *>(keys + at)[lane];
        const float4 v = reinterpret_cast<const float4 *>(values + at)[lane];
        const float dot = wave_sum(((q.x * k.x + q.y * k.y) + q.z * k.z) + q.w * k.w);
        online_step(dot * score_scale, v, maximum, denominator, acc);
    }
    reinterpret_cast<float4 *>(wave_acc[wave])[lane] = acc;
    if (lane == 0) {
        wave_max[wave] = maximum;
        wave_den[wave] = denominator;
    }
    __syncthreads();
    // every split holds at least one token, so the block maximum is finite
    float m = wave_max[0];
    for (uint32_t w = 1; w < 4; ++w) {
        m = fmaxf(m, wave_max[w]);
    }
    float a = 0.0f, d = 0.0f;
    for (uint32_t w = 0; w < 4; ++w) {
        const float f = expf(wave_max[w] - m);  // 0 for a wave without tokens
        a += wave_acc[w][threadIdx.x] * f;
        d += wave_den[w] * f;
    }
    float *out = partial + (static_cast<size_t>(h) * splits + split) * kPartialStride;
    out[threadIdx.x] = a;
    if (threadIdx.x == 0) {
        out[kHeadSize] = m;
        out[kHeadSize + 1] = d;
    }
}

// Per query head: the splits merged, divided by the denominator, times the
// head's sigmoid gate (src/executor.cpp:403-411).
__global__ __launch_bounds__(kHeadSize) void k_attention_combine(const float *partial,
                                                                 uint32_t splits,
                                                                 const float *query_gate,
                                                                 float *attended) {
#pragma clang fp contract(off)
    const uint32_t h = blockIdx.x, t = threadIdx.x;
    const float *p = partial + static_cast<size_t>(h) * splits * kPartialStride;
    float m = p[kHeadSize];
    for (uint32_t s = 1; s < splits; ++s) {
        m = fmaxf(m, p[s * kPartialStride + kHeadSize]);
    }
    float a = 0.0f, d = 0.0f;
    for (uint32_t s = 0; s < splits; ++s) {
        const float f = expf(p[s * kPartialStride + kHeadSize] - m);
        a += p[s * kPartialStride + t] * f;
        d += p[s * kPartialStride + kHeadSize + 1] * f;
    }
    const float gate = query_gate[static_cast<size_t>(h) * kQueryStride + kHeadSize + t];
    attended[static_cast<size_t>(h) * kHeadSize + t] = a * (1.0f / d) * sigmoid_of(gate);
}

// The causal convolution of 128 channels (src/executor.cpp:480-496) and, for
// the query and key groups (blocks 0-31), their L2 norm (497-505).
__global__ __launch_bounds__(kLinearHead) void k_linear_conv(const float *qkv,
                                                             const uint16_t *weights,
                                                             float *state, float *convolved) {
#pragma clang fp contract(off)
    __shared__ float partial[16];
    const uint32_t c = blockIdx.x * kLinearHead + threadIdx.x;
    float *history = state + static_cast<size_t>(c) * 3u;
    const uint2 packed = *reinterpret_cast<const uint2 *>(weights + static_cast<size_t>(c) * 4u);
    const float w0 = bf16_bits_to_float(packed.x & 0xFFFFu), w1 = bf16_bits_to_float(packed.x >> 16);
    const float w2 = bf16_bits_to_float(packed.y & 0xFFFFu), w3 = bf16_bits_to_float(packed.y >> 16);
    const float h0 = history[0], h1 = history[1], h2 = history[2];
    const float x = qkv[c];
    float v = 0.0f;
    v += h0 * w0;
    v += h1 * w1;
    v += h2 * w2;
    v += x * w3;
    float y = silu_of(v);
    history[0] = h1;
    history[1] = h2;
    history[2] = x;
    if (blockIdx.x < 2u * kKeyHeads) {  // uniform over the block
        const float squares = block_sum(y * y, partial);
        y *= 1.0f / sqrtf(squares + kEpsilon);
    }
    convolved[c] = y;
}

// gated_delta_head (src/executor.cpp:121-155) for rows [16 y, 16 y + 16) of
// value head x: each wave updates four state rows in turn, a lane holding two
// of a row's 128 values (src/simd.cpp:108-127).
__global__ __launch_bounds__(256) void k_gated_delta(const float *convolved, const float *alpha,
                                                     const float *beta, const uint16_t *alpha_bias,
                                                     const uint16_t *a_log, float *recurrent,
                                                     float *output) {
#pragma clang fp contract(off)
    const uint32_t h = blockIdx.x;
    const uint32_t kh = h / (kValueHeads / kKeyHeads);
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const float2 q = reinterpret_cast<const float2 *>(convolved + static_cast<size_t>(kh) * kLinearHead)[lane];
    const float2 k = reinterpret_cast<const float2 *>(convolved + kQkSize + static_cast<size_t>(kh) * kLinearHead)[lane];
    const float *v = convolved + 2u * kQkSize + static_cast<size_t>(h) * kLinearHead;
    const float beta_value = sigmoid_of(beta[h]);
    const float biased = alpha[h] + bf16_bits_to_float(alpha_bias[h]);
    const float softplus = biased > 20.0f ? biased : log1pf(expf(biased));
    const float decay = expf(-expf(bf16_bits_to_float(a_log[h])) * softplus);
    const float output_scale = 1.0f / sqrtf(static_cast<float>(kLinearHead));
    for (uint32_t j = 0; j < kDeltaRows / 4u; ++j) {
        const uint32_t row = blockIdx.y * kDeltaRows + wave * (kDeltaRows / 4u) + j;
        float2 *state = reinterpret_cast<float2 *>(
            recurrent + (static_cast<size_t>(h) * kLinearHead + row) * kLinearHead);
        float2 s = state[lane];
        s.x *= decay;
        s.y *= decay;
        const float prediction = wave_sum(s.x * k.x + s.y * k.y);
        const float delta = (v[row] - prediction) * beta_value;
        s.x += k.x * delta;
        s.y += k.y * delta;
        const float attended = wave_sum(s.x * q.x + s.y * q.y);
        state[lane] = s;
        if (lane == 0) {
            output[static_cast<size_t>(h) * kLinearHead + row] = attended * output_scale;
        }
    }
}

// rms_norm (weight offset 0, src/kernels.cpp:1052-1073) of each value head,
// times SiLU of the gate (src/executor.cpp:538-550).
__global__ __launch_bounds__(kLinearHead) void k_linear_norm_gate(const float *recurrent_output,
                                                                  const uint16_t *norm,
                                                                  const float *gate,
                                                                  float *normalized) {
#pragma clang fp contract(off)
    __shared__ float partial[16];
    const size_t i = static_cast<size_t>(blockIdx.x) * kLinearHead + threadIdx.x;
    const float x = recurrent_output[i];
    const float squares = block_sum(x * x, partial);
    const float scale = 1.0f / sqrtf(squares / static_cast<float>(kLinearHead) + kEpsilon);
    normalized[i] = x * scale * (0.0f + bf16_bits_to_float(norm[threadIdx.x])) * silu_of(gate[i]);
}

// hidden += branch (the residual adds of decode_layer).
__global__ __launch_bounds__(256) void k_residual_add(float *hidden, const float *branch,
                                                      uint32_t count) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < count) {
        hidden[i] = hidden[i] + branch[i];
    }
}

// prepare_rope (src/executor.cpp:43-58) with MachModel's divisors
// (src/model.cpp:606-615), on the host with the reference's float libm calls.
RopeTable rope_table(uint32_t position) {
    RopeTable t{};
    for (uint32_t i = 0; i < kRopeHalf; ++i) {
        const float divisor = std::pow(10000000.0F, 2.0F * static_cast<float>(i) / 64.0F);
        const float theta = static_cast<float>(position) / divisor;
        t.cosine[i] = std::cos(theta);
        t.sine[i] = std::sin(theta);
    }
    return t;
}

// A nested entry's status becomes this call's failure.
void forward(adi_hip_context *ctx, int status) {
    if (status != ADI_HIP_OK) {
        fail(status, ctx->last_error);
    }
}

bool ne_shaped(const adi_hip_ne_matrix &m, uint32_t rows, uint32_t columns) {
    return m.rows == rows && m.columns == columns && m.trellis != nullptr;
}

}  // namespace
}  // namespace adi_hip

using namespace adi_hip;

extern "C" {

int adi_hip_full_attention_forward(adi_hip_context *ctx, const adi_hip_full_attention *L,
                                   uint32_t position, const float *input, float *output,
                                   float *keys, float *values, uint32_t capacity) {
    return guarded(ctx, [&] {
        require(L != nullptr && input != nullptr && output != nullptr && keys != nullptr &&
                    values != nullptr,
                "full attention state or input shape mismatch");
        const uint32_t hidden = L->query.columns;
        require(ne_shaped(L->query, kQueryHeads * kQueryStride, hidden) &&
                    ne_shaped(L->key, kKvHeads * kHeadSize, hidden) &&
                    ne_shaped(L->value, kKvHeads * kHeadSize, hidden) &&
                    ne_shaped(L->output, hidden, kQueryHeads * kHeadSize) &&
                    L->query_norm != nullptr && L->key_norm != nullptr && position < capacity,
                "full attention state or input shape mismatch");
        require(aligned_to(keys, 16) && aligned_to(values, 16),
                "attention caches must be 16-byte aligned");
        auto &ws = ctx->layer_workspace;
        ws.used = 0;
        const uint32_t tokens = position + 1;
        uint32_t splits = ceil_div(tokens, 32);
        splits = splits < 1 ? 1 : (splits > kMaxSplits ? kMaxSplits : splits);
        const uint32_t chunk = ceil_div(tokens, splits);
        splits = ceil_div(tokens, chunk);  // every split holds a token
        ws.ensure(Workspace::round(kQueryHeads * kQueryStride * 4) +
                  Workspace::round(kQueryHeads * kHeadSize * 4) +
                  Workspace::round(size_t(kQueryHeads) * kMaxSplits * kPartialStride * 4));
        float *query_gate = ws.take<float>(kQueryHeads * kQueryStride);
        float *attended = ws.take<float>(kQueryHeads * kHeadSize);
        float *partial = ws.take<float>(size_t(kQueryHeads) * splits * kPartialStride);
        float *key = keys + static_cast<size_t>(position) * kKvHeads * kHeadSize;
        float *value = values + static_cast<size_t>(position) * kKvHeads * kHeadSize;
        forward(ctx, adi_hip_ne_matvec(ctx, &L->query, input, query_gate));
        forward(ctx, adi_hip_ne_matvec(ctx, &L->key, input, key));
        forward(ctx, adi_hip_ne_matvec(ctx, &L->value, input, value));
        launch(ctx, "attention_norm_rope", k_norm_rope, dim3(kQueryHeads + kKvHeads),
               dim3(kHeadSize), 0, query_gate, key, L->query_norm, L->key_norm,
               rope_table(position));
        launch(ctx, "attention_partial", k_attention_partial, dim3(kQueryHeads, splits), dim3(256),
               0, static_cast<const float *>(query_gate), static_cast<const float *>(keys),
               static_cast<const float *>(values), tokens, chunk, partial);
        launch(ctx, "attention_combine", k_attention_combine, dim3(kQueryHeads), dim3(kHeadSize), 0,
               static_cast<const float *>(partial), splits,
               static_cast<const float *>(query_gate), attended);
        forward(ctx, adi_hip_ne_matvec(ctx, &L->output, attended, output));
    });
}

int adi_hip_linear_attention_forward(adi_hip_context *ctx, const adi_hip_linear_attention *L,
                                     const float *input, float *output, float *convolution_state,
                                     float *recurrent_state) {
    return guarded(ctx, [&] {
        require(L != nullptr && input != nullptr && output != nullptr &&
                    convolution_state != nullptr && recurrent_state != nullptr,
                "linear attention input shape mismatch");
        const uint32_t hidden = L->qkv.columns;
        require(ne_shaped(L->qkv, kChannels, hidden) && ne_shaped(L->gate, kValueSize, hidden) &&
                    ne_shaped(L->output, hidden, kValueSize),
                "linear attention input shape mismatch");
        require(L->alpha.rows == kValueHeads && L->alpha.columns == hidden &&
                    L->beta.rows == kValueHeads && L->beta.columns == hidden &&
                    L->alpha.values != nullptr && L->beta.values != nullptr &&
                    L->alpha_bias != nullptr && L->a_log != nullptr,
                "linear attention decay shape mismatch");
        require(L->convolution != nullptr && aligned_to(L->convolution, 8),
                "linear attention convolution shape mismatch");
        require(L->norm != nullptr, "linear attention input shape mismatch");
        require(aligned_to(recurrent_state, 8), "linear attention state must be 8-byte aligned");
        auto &ws = ctx->layer_workspace;
        ws.used = 0;
        ws.ensure(Workspace::round(kChannels * 4) * 2 + Workspace::round(kValueSize * 4) * 3 +
                  Workspace::round(kValueHeads * 4) * 2);
        float *qkv = ws.take<float>(kChannels);
        float *convolved = ws.take<float>(kChannels);
        float *gate = ws.take<float>(kValueSize);
        float *recurrent_output = ws.take<float>(kValueSize);
        float *normalized = ws.take<float>(kValueSize);
        float *alpha = ws.take<float>(kValueHeads);
        float *beta = ws.take<float>(kValueHeads);
        forward(ctx, adi_hip_ne_matvec(ctx, &L->qkv, input, qkv));
        forward(ctx, adi_hip_ne_matvec(ctx, &L->gate, input, gate));
        forward(ctx, adi_hip_bf16_matvec(ctx, &L->alpha, input, alpha));
        forward(ctx, adi_hip_bf16_matvec(ctx, &L->beta, input, beta));
        launch(ctx, "linear_conv", k_linear_conv, dim3(kChannels / kLinearHead), dim3(kLinearHead),
               0, static_cast<const float *>(qkv), L->convolution, convolution_state, convolved);
        launch(ctx, "gated_delta", k_gated_delta, dim3(kValueHeads, kLinearHead / kDeltaRows),
               dim3(256), 0, static_cast<const float *>(convolved),
               static_cast<const float *>(alpha), static_cast<const float *>(beta), L->alpha_bias,
               L->a_log, recurrent_state, recurrent_output);
        launch(ctx, "linear_norm_gate", k_linear_norm_gate, dim3(kValueHeads), dim3(kLinearHead), 0,
               static_cast<const float *>(recurrent_output), L->norm,
               static_cast<const float *>(gate), normalized);
        forward(ctx, adi_hip_ne_matvec(ctx, &L->output, normalized, output));
    });
}

int adi_hip_decode_layer(adi_hip_context *ctx, const adi_hip_decoder_layer *L, uint32_t position,
                         float *hidden, const adi_hip_layer_state *state) {
    return guarded(ctx, [&] {
        require(L != nullptr && hidden != nullptr && state != nullptr && L->input_norm != nullptr &&
                    L->post_attention_norm != nullptr,
                "decoder layer input is null");
        const uint32_t n = L->moe.hidden;
        require(n > 0 && aligned_to(hidden, 16), "decoder hidden row must be 16-byte aligned");
        auto &ws = ctx->decoder_workspace;
        ws.used = 0;
        ws.ensure(Workspace::round(size_t(n) * 4) * 2);
        float *normalized = ws.take<float>(n);
        float *branch = ws.take<float>(n);
        const dim3 grid(ceil_div(n, 256));
        forward(ctx, adi_hip_rms_norm(ctx, hidden, L->input_norm, n, 1, 1.0f, 1.0e-6f, normalized));
        if (L->full_attention != 0) {
            forward(ctx, adi_hip_full_attention_forward(ctx, &L->full, position, normalized, branch,
                                                        state->keys, state->values,
                                                        state->capacity));
        } else {
            forward(ctx, adi_hip_linear_attention_forward(ctx, &L->linear, normalized, branch,
                                                          state->convolution, state->recurrent));
        }
        launch(ctx, "residual_add", k_residual_add, grid, dim3(256), 0, hidden,
               static_cast<const float *>(branch), n);
        forward(ctx, adi_hip_rms_norm(ctx, hidden, L->post_attention_norm, n, 1, 1.0f, 1.0e-6f,
                                      normalized));
        forward(ctx, adi_hip_moe_forward(ctx, &L->moe, normalized, 1, nullptr, branch, nullptr,
                                         nullptr));
        launch(ctx, "residual_add", k_residual_add, grid, dim3(256), 0, hidden,
               static_cast<const float *>(branch), n);
    });
}

}  // extern "C"
