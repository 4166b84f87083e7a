// attention.hip -- the attention half of a decoder layer on the device, for a
// chunk of consecutive tokens of one sequence (one token when decoding):
//   full_attention_forward   (src/executor.cpp:332-418, src/attention.cpp)
//   linear_attention_forward (src/executor.cpp:420-557, Gated DeltaNet)
// A chunk gives what decoding its tokens one after another gives (token b sees
// the cache up to its own position; the recurrence runs over the chunk in
// order); its projections and MoE run batched.
//
// Full attention, after the q/k/v projections:
//   norm_rope   one block per head: RMS norm with (1 + w), then RoPE on the
//               first 64 dimensions from a cos/sin table the host computes
//               with the same libm calls as the reference (prepare_rope):
//               a kernel argument for one token, a cached device table of
//               every position for a chunk; the key lands in its cache slot,
//               the value is projected there
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
#include "attention.hpp"
#include "dense.hpp"
#include "projection.hpp"

#include <algorithm>
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

// Sequences per launch of the per-sequence kernels of a decode step over
// many sequences; their state pointers travel as kernel arguments, their
// positions in a device array (so a captured step replays at new positions).
constexpr uint32_t kRowGroup = 32;

struct FullRows {
    float *keys[kRowGroup];
    float *values[kRowGroup];
};

// Splits of the history of a row at `tokens` entries: one per 32 entries, at
// most `cap`. Each row's split count follows from its own position alone, so
// its result does not depend on the launch's grid (any grid with at least
// this many splits gives the same bits) or on the other rows.
__host__ __device__ __forceinline__ uint32_t row_splits(uint32_t tokens, uint32_t cap) {
    const uint32_t s = (tokens + 31u) / 32u;
    return s < 1u ? 1u : (s > cap ? cap : s);
}

// Blocks of the flash-decoding partial kernels (block b runs on XCD b % 8).
// Under kPairSplits splits block b is query head b % 16 of split b / 16: all
// splits of a head on one XCD, whose L2 then still holds them for the
// combine. From kPairSplits splits the history is long and the eight query
// heads of a KV head, which read the same cache entries, are dealt to one
// XCD instead, so the entries pass through that XCD's L2 once rather than
// once per XCD: block b (k = b / 8) takes pair g = 8 (k / 8) + b % 8,
// g = kKvHeads split + kv, and query head 8 kv + k % 8; the grid of
// partial_blocks(splits) covers every pair, and blocks of pairs past the
// last split return at once.
static_assert(kQueryHeads == 8 * kKvHeads, "eight query heads to a KV head");
constexpr uint32_t kPairSplits = 32;
__host__ __device__ __forceinline__ uint32_t partial_blocks(uint32_t splits) {
    return splits < kPairSplits ? kQueryHeads * splits : (kKvHeads * splits + 7u) / 8u * 64u;
}
struct PartialBlock {
    uint32_t head, split;
    bool live;
};
__device__ __forceinline__ PartialBlock partial_block(uint32_t b, uint32_t splits) {
    if (splits < kPairSplits) {
        return {b % kQueryHeads, b / kQueryHeads, true};
    }
    const uint32_t k = b >> 3;
    const uint32_t g = ((k >> 3) << 3) | (b & 7u);
    const uint32_t kv = g % kKvHeads;
    return {kv * 8u + (k & 7u), g / kKvHeads, g < kKvHeads * splits};
}

struct LinearRows {
    float *convolution[kRowGroup];
    float *recurrent[kRowGroup];
};

struct RopeTable {
    float cosine[kRopeHalf];
    float sine[kRopeHalf];
};

// MachModel's RoPE divisors (src/model.cpp:606-615), computed on the host.
struct RopeDivisors {
    float divisor[kRopeHalf];
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

// normalize_head then apply_rope (src/executor.cpp:25-41, 60-72, 376-390)
// of one 256-value head by a block of kHeadSize threads: RMS norm with
// (1 + w), then thread t < 32 rotates the pair (t, t + 32) by its cosine and
// sine. src and dst may be the same.
__device__ __forceinline__ void norm_rope_head(const float *src, float *dst, const uint16_t *w,
                                               float cosine, float sine, float *partial,
                                               float *head) {
#pragma clang fp contract(off)
    const uint32_t t = threadIdx.x;
    float x = src[t];
    const float squares = block_sum(x * x, partial);
    const float scale = 1.0f / sqrtf(squares / static_cast<float>(kHeadSize) + kEpsilon);
    x *= scale * (1.0f + bf16_bits_to_float(w[t]));
    head[t] = x;
    __syncthreads();
    if (t < kRopeHalf) {
        const float first = head[t], second = head[t + kRopeHalf];
        dst[t] = first * cosine - second * sine;
        dst[t + kRopeHalf] = second * cosine + first * sine;
    } else if (t >= 2 * kRopeHalf) {
        dst[t] = x;
    }
}

// Block (h, b) of token b of a chunk: h 0-15 the query heads (stride 512),
// 16-17 the new key heads, in place. One token takes the host's table `rope`;
// in a chunk, token b reads the host-computed table of position + b from
// `rope_rows` ([position][32 cosines, 32 sines]), so every token of a chunk
// rotates exactly as it would alone (the reference builds its prefill table
// on the host too, src/executor.cpp:1853-1866).
__global__ __launch_bounds__(kHeadSize) void k_norm_rope(float *query_gate, float *key,
                                                         const uint16_t *query_norm,
                                                         const uint16_t *key_norm, RopeTable rope,
                                                         const float *rope_rows, uint32_t position) {
    __shared__ float partial[16];
    __shared__ float head[kHeadSize];
    const uint32_t h = blockIdx.x, b = blockIdx.y, t = threadIdx.x;
    query_gate += static_cast<size_t>(b) * kQueryHeads * kQueryStride;
    key += static_cast<size_t>(b) * kKvHeads * kHeadSize;
    float *v = h < kQueryHeads ? query_gate + static_cast<size_t>(h) * kQueryStride
                               : key + static_cast<size_t>(h - kQueryHeads) * kHeadSize;
    float cosine = 0.0f, sine = 0.0f;
    if (t < kRopeHalf) {
        cosine = rope.cosine[t];
        sine = rope.sine[t];
        if (rope_rows != nullptr) {
            const float *row = rope_rows + static_cast<size_t>(position + b) * (2 * kRopeHalf);
            cosine = row[t];
            sine = row[kRopeHalf + t];
        }
    }
    norm_rope_head(v, v, h < kQueryHeads ? query_norm : key_norm, cosine, sine, partial, head);
}

// The same for one decode token of each of up to kRowGroup sequences: block
// (h, r), h 0-15 the query heads of row r (in place), 16-17 its key heads,
// normalized and rotated into the sequence's cache entry positions[r], and
// 18-19 its value heads, copied into that entry. The RoPE table row is the
// row's position.
__global__ __launch_bounds__(kHeadSize) void k_norm_rope_rows(float *query_gate, const float *key,
                                                              const float *value,
                                                              const uint16_t *query_norm,
                                                              const uint16_t *key_norm,
                                                              const float *rope_rows, FullRows rows,
                                                              const uint32_t *positions) {
    __shared__ float partial[16];
    __shared__ float head[kHeadSize];
    const uint32_t h = blockIdx.x, r = blockIdx.y, t = threadIdx.x;
    const uint32_t position = positions[r];
    const size_t entry = static_cast<size_t>(position) * kKvHeads * kHeadSize;
    if (h >= kQueryHeads + kKvHeads) {  // uniform over the block
        const uint32_t kv = h - kQueryHeads - kKvHeads;
        rows.values[r][entry + kv * kHeadSize + t] =
            value[(static_cast<size_t>(r) * kKvHeads + kv) * kHeadSize + t];
        return;
    }
    float cosine = 0.0f, sine = 0.0f;
    if (t < kRopeHalf) {
        const float *row = rope_rows + static_cast<size_t>(position) * (2 * kRopeHalf);
        cosine = row[t];
        sine = row[kRopeHalf + t];
    }
    if (h < kQueryHeads) {
        float *q = query_gate + static_cast<size_t>(r) * kQueryHeads * kQueryStride +
                   static_cast<size_t>(h) * kQueryStride;
        norm_rope_head(q, q, query_norm, cosine, sine, partial, head);
    } else {
        const uint32_t kv = h - kQueryHeads;
        norm_rope_head(key + (static_cast<size_t>(r) * kKvHeads + kv) * kHeadSize,
                       rows.keys[r] + entry + kv * kHeadSize, key_norm, cosine, sine, partial,
                       head);
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

// Block (query head, split) of one token's query row: cache entries
// [split * chunk, ...) below `tokens` of the head's KV stream, wave w taking
// every fourth. Lane l holds dimensions 4l..4l+3. Writes the split's
// accumulator, maximum and denominator to the token's partial rows
// (maximum -inf and denominator 0 when the split lies past the token).
// With COHERENT the partial row is written through to memory (a later block
// of the same launch reads it). The query head is at `query` (global or LDS);
// entry `fresh` (when below `tokens`) is taken from fresh_key / fresh_value
// (LDS) instead of the cache.
template <bool COHERENT = false>
__device__ __forceinline__ void attention_partial_span(const float *query, const float *keys,
                                                       const float *values, uint32_t tokens,
                                                       uint32_t chunk, float *partial, uint32_t h,
                                                       uint32_t split, uint32_t splits,
                                                       uint32_t fresh = 0xFFFFFFFFu,
                                                       const float *fresh_key = nullptr,
                                                       const float *fresh_value = nullptr) {
#pragma clang fp contract(off)
    __shared__ __align__(16) float wave_acc[4][kHeadSize];
    __shared__ float wave_max[4], wave_den[4];
    const uint32_t kv = h / (kQueryHeads / kKvHeads);
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const float4 q = reinterpret_cast<const float4 *>(query)[lane];
    const float score_scale = 1.0f / 16.0f;  // 1 / sqrt(256)
    const uint32_t begin = split * chunk;
    const uint32_t end = begin + chunk < tokens ? begin + chunk : tokens;
    float maximum = -__builtin_huge_valf(), denominator = 0.0f;
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    // the wave's tokens t0, t0 + 4, ... in batches of eight: the batch's
    // entries are loaded together (a token past the span reloads t0, unused),
    // its dot products reduced together, then the online updates in order
    constexpr uint32_t kBatch = 8;
    for (uint32_t t0 = begin + wave; t0 < end; t0 += 4u * kBatch) {
        // every entry from the cache, with no branch around a load (so the
        // batch's loads are counted and waited for once); the fresh entry's
        // cache slot is read too and then replaced by its LDS copy
        float4 k[kBatch], v[kBatch];
#pragma unroll
        for (uint32_t j = 0; j < kBatch; ++j) {
            const uint32_t t = t0 + 4u * j < end ? t0 + 4u * j : t0;
            const size_t at = (static_cast<size_t>(t) * kKvHeads + kv) * kHeadSize;
            k[j] = reinterpret_cast<const float4 *>(keys + at)[lane];
            v[j] = reinterpret_cast<const float4 *>(values + at)[lane];
        }
#pragma unroll
        for (uint32_t j = 0; j < kBatch; ++j) {
            const uint32_t t = t0 + 4u * j < end ? t0 + 4u * j : t0;
            if (t == fresh) {  // wave-uniform
                k[j] = reinterpret_cast<const float4 *>(fresh_key)[lane];
                v[j] = reinterpret_cast<const float4 *>(fresh_value)[lane];
            }
        }
        float dot[kBatch];
#pragma unroll
        for (uint32_t j = 0; j < kBatch; ++j) {
            dot[j] = wave_sum(((q.x * k[j].x + q.y * k[j].y) + q.z * k[j].z) + q.w * k[j].w);
        }
#pragma unroll
        for (uint32_t j = 0; j < kBatch; ++j) {
            if (t0 + 4u * j < end) {
                online_step(dot[j] * score_scale, v[j], maximum, denominator, acc);
            }
        }
    }
    reinterpret_cast<float4 *>(wave_acc[wave])[lane] = acc;
    if (lane == 0) {
        wave_max[wave] = maximum;
        wave_den[wave] = denominator;
    }
    __syncthreads();
    float m = wave_max[0];
    for (uint32_t w = 1; w < 4; ++w) {
        m = fmaxf(m, wave_max[w]);
    }
    float a = 0.0f, d = 0.0f;
    if (m != -__builtin_huge_valf()) {  // else no token in this split
        for (uint32_t w = 0; w < 4; ++w) {
            const float f = expf(wave_max[w] - m);  // 0 for a wave without tokens
            a += wave_acc[w][threadIdx.x] * f;
            d += wave_den[w] * f;
        }
    }
    float *out = partial + (static_cast<size_t>(h) * splits + split) * kPartialStride;
    if constexpr (COHERENT) {
        coherent_store(out + threadIdx.x, a);
        if (threadIdx.x == 0) {
            coherent_store(out + kHeadSize, m);
            coherent_store(out + kHeadSize + 1, d);
        }
    } else {
        out[threadIdx.x] = a;
        if (threadIdx.x == 0) {
            out[kHeadSize] = m;
            out[kHeadSize + 1] = d;
        }
    }
}

// Token b of a chunk at `position` sees entries 0 .. position + b.
__global__ __launch_bounds__(256) void k_attention_partial(const float *query_gate,
                                                           const float *keys, const float *values,
                                                           uint32_t position, uint32_t chunk,
                                                           uint32_t splits, float *partial) {
    const PartialBlock pb = partial_block(blockIdx.x, splits);
    if (!pb.live) {
        return;
    }
    const uint32_t b = blockIdx.z;
    attention_partial_span(query_gate + static_cast<size_t>(b) * kQueryHeads * kQueryStride +
                               static_cast<size_t>(pb.head) * kQueryStride,
                           keys,
                           values, position + b + 1, chunk,
                           partial + static_cast<size_t>(b) * kQueryHeads * splits * kPartialStride, pb.head,
                           pb.split, splits);
}

// Row r of a decode step over sequences sees its own cache's entries
// 0 .. positions[r], split evenly over row_splits(positions[r] + 1, cap)
// splits; the grid's further splits lie past the row's tokens and come out
// empty (skipped by the combine).
__global__ __launch_bounds__(256) void k_attention_partial_rows(const float *query_gate,
                                                                FullRows rows,
                                                                const uint32_t *positions,
                                                                uint32_t cap, uint32_t grid_splits,
                                                                float *partial) {
    const PartialBlock pb = partial_block(blockIdx.x, grid_splits);
    if (!pb.live) {
        return;
    }
    const uint32_t r = blockIdx.z;
    const uint32_t tokens = positions[r] + 1;
    const uint32_t splits = row_splits(tokens, cap);
    attention_partial_span(query_gate + static_cast<size_t>(r) * kQueryHeads * kQueryStride +
                               static_cast<size_t>(pb.head) * kQueryStride,
                           rows.keys[r], rows.values[r], tokens, (tokens + splits - 1u) / splits,
                           partial + static_cast<size_t>(r) * kQueryHeads * grid_splits * kPartialStride,
                           pb.head, pb.split, grid_splits);
}

// The splits of one query head merged (splits <= N): every split's
// accumulator, then the splits' maxima and denominators (through LDS),
// loaded in one round, then the accumulators added in split order.
template <uint32_t N, bool COHERENT = false>
__device__ __forceinline__ void combine_splits(const float *p, uint32_t splits, uint32_t t, float *split_max,
                                               float *split_den, float *split_factor, float &a, float &d) {
#pragma clang fp contract(off)
    const auto load = [](const float *at) { return COHERENT ? coherent_load(at) : *at; };
    float acc[N];
#pragma unroll
    for (uint32_t s = 0; s < N; ++s) {
        acc[s] = s < splits ? load(p + s * kPartialStride + t) : 0.0f;
    }
    static_assert(N <= kHeadSize, "a thread's split");
    // both words of the thread's split loaded before either is stored (one
    // round trip with the accumulators')
    if (t < splits) {
        const float mx = load(p + t * kPartialStride + kHeadSize);
        const float dn = load(p + t * kPartialStride + kHeadSize + 1);
        split_max[t] = mx;
        split_den[t] = dn;
    }
    __syncthreads();
    // split 0 always holds token 0, so the maximum is finite
    float m = split_max[0];
    for (uint32_t s = 1; s < splits; ++s) {
        m = fmaxf(m, split_max[s]);
    }
    for (uint32_t s = t; s < splits; s += kHeadSize) {
        split_factor[s] = expf(split_max[s] - m);
    }
    __syncthreads();
    a = 0.0f;
    d = 0.0f;
#pragma unroll
    for (uint32_t s = 0; s < N; ++s) {
        const float den = s < splits ? split_den[s] : 0.0f;
        if (den == 0.0f) {
            continue;  // a split past the token (or past the splits)
        }
        const float f = split_factor[s];
        a += acc[s] * f;
        d += den * f;
    }
}

// Per query head: the splits merged, divided by the denominator, times the
// head's sigmoid gate (src/executor.cpp:403-411).
__global__ __launch_bounds__(kHeadSize) void k_attention_combine(const float *partial,
                                                                 uint32_t splits,
                                                                 const float *query_gate,
                                                                 float *attended) {
#pragma clang fp contract(off)
    const uint32_t h = blockIdx.x, t = threadIdx.x, b = blockIdx.y;
    query_gate += static_cast<size_t>(b) * kQueryHeads * kQueryStride;
    attended += static_cast<size_t>(b) * kQueryHeads * kHeadSize;
    __shared__ float split_max[kMaxSplits], split_den[kMaxSplits], split_factor[kMaxSplits];
    const float *p = partial + (static_cast<size_t>(b) * kQueryHeads + h) * splits * kPartialStride;
    const float gate = query_gate[static_cast<size_t>(h) * kQueryStride + kHeadSize + t];
    float a, d;
    if (splits <= 16u) {
        combine_splits<16>(p, splits, t, split_max, split_den, split_factor, a, d);
    } else {
        combine_splits<kMaxSplits>(p, splits, t, split_max, split_den, split_factor, a, d);
    }
    attended[static_cast<size_t>(h) * kHeadSize + t] = a * (1.0f / d) * sigmoid_of(gate);
}

// One decode token of each of up to kRowGroup sequences through full
// attention's core in one launch, with the arithmetic of k_norm_rope_rows,
// k_attention_partial_rows and k_attention_combine. Block (query head h,
// split, sequence r), dealt as partial_block deals them:
// - normalizes and rotates its query head into LDS itself (every split of a
//   head does);
// - the splits holding the row's new entry (position) normalize and rotate
//   its key and take its value themselves, and one of them per KV head (the
//   first query head of the KV head) writes both into the cache: no block
//   reads that entry from the cache;
// - writes its split's partial row through to memory; the last block of the
//   head's grid_splits through the head's ticket merges them and applies the
//   sigmoid gate.
// `tickets` holds kQueryHeads words a sequence, zero between calls.
__global__ __launch_bounds__(256) void k_attention_rows_one(const float *query_gate, const float *key,
                                                            const float *value, const uint16_t *query_norm,
                                                            const uint16_t *key_norm, const float *rope_rows,
                                                            FullRows rows, const uint32_t *positions,
                                                            uint32_t cap, uint32_t grid_splits, float *partial,
                                                            float *attended, uint32_t *tickets) {
    __shared__ float sums[16];
    __shared__ float head[kHeadSize];
    __shared__ __align__(16) float q_lds[kHeadSize];
    __shared__ __align__(16) float key_lds[kHeadSize];
    __shared__ __align__(16) float value_lds[kHeadSize];
    __shared__ float split_max[kMaxSplits], split_den[kMaxSplits], split_factor[kMaxSplits];
    __shared__ uint32_t last;
    const PartialBlock pb = partial_block(blockIdx.x, grid_splits);
    if (!pb.live) {
        return;
    }
    const uint32_t r = blockIdx.z, t = threadIdx.x;
    const uint32_t h = pb.head, split = pb.split, kv = h / (kQueryHeads / kKvHeads);
    const uint32_t position = positions[r];
    const uint32_t tokens = position + 1u;
    const uint32_t splits = row_splits(tokens, cap);
    const uint32_t chunk = (tokens + splits - 1u) / splits;
    const uint32_t begin = split * chunk;
    const bool fresh = begin <= position && position < begin + chunk;  // uniform over the block
    const float *qg = query_gate + (static_cast<size_t>(r) * kQueryHeads + h) * kQueryStride;
    float cosine = 0.0f, sine = 0.0f;
    if (t < kRopeHalf) {
        const float *row = rope_rows + static_cast<size_t>(position) * (2 * kRopeHalf);
        cosine = row[t];
        sine = row[kRopeHalf + t];
    }
    norm_rope_head(qg, q_lds, query_norm, cosine, sine, sums, head);
    if (fresh) {
        __syncthreads();  // head[] is free again
        const size_t src = (static_cast<size_t>(r) * kKvHeads + kv) * kHeadSize;
        norm_rope_head(key + src, key_lds, key_norm, cosine, sine, sums, head);
        value_lds[t] = value[src + t];
        __syncthreads();
        if (h % (kQueryHeads / kKvHeads) == 0u) {
            const size_t entry = (static_cast<size_t>(position) * kKvHeads + kv) * kHeadSize;
            rows.keys[r][entry + t] = key_lds[t];
            rows.values[r][entry + t] = value_lds[t];
        }
    }
    __syncthreads();
    float *p = partial + static_cast<size_t>(r) * kQueryHeads * grid_splits * kPartialStride;
    attention_partial_span<true>(q_lds, rows.keys[r], rows.values[r], tokens, chunk, p, h, split, grid_splits,
                                 position, key_lds, value_lds);
    wait_stores();
    __syncthreads();
    uint32_t *ticket = tickets + static_cast<size_t>(r) * kQueryHeads + h;
    if (t == 0) {
        last = coherent_add(ticket, 1u) + 1u == grid_splits ? 1u : 0u;
    }
    __syncthreads();
    if (last == 0u) {
        return;
    }
    const float gate = qg[kHeadSize + t];
    const float *ph = p + static_cast<size_t>(h) * grid_splits * kPartialStride;
    float a, d;
    if (grid_splits <= 16u) {
        combine_splits<16, true>(ph, grid_splits, t, split_max, split_den, split_factor, a, d);
    } else {
        combine_splits<kMaxSplits, true>(ph, grid_splits, t, split_max, split_den, split_factor, a, d);
    }
    attended[(static_cast<size_t>(r) * kQueryHeads + h) * kHeadSize + t] = a * (1.0f / d) * sigmoid_of(gate);
    if (t == 0) {
        coherent_store(ticket, 0u);
    }
}

// The causal convolution of 128 channels for token b of a chunk
// (src/executor.cpp:480-496) and, for the query and key groups (blocks
// 0-31), their L2 norm (497-505). The three inputs before token b are the
// chunk's earlier qkv rows or, before the chunk, the state. With `shift` (one
// token) the state shifts here; for a chunk k_conv_history does it after
// every token has read it.
__device__ __forceinline__ void linear_conv_token(const float *qkv, const uint16_t *weights,
                                                  float *state, float *convolved, uint32_t b,
                                                  bool shift) {
#pragma clang fp contract(off)
    __shared__ float partial[16];
    const uint32_t c = blockIdx.x * kLinearHead + threadIdx.x;
    float *history = state + static_cast<size_t>(c) * 3u;
    const uint2 packed = *reinterpret_cast<const uint2 *>(weights + static_cast<size_t>(c) * 4u);
    const float w0 = bf16_bits_to_float(packed.x & 0xFFFFu), w1 = bf16_bits_to_float(packed.x >> 16);
    const float w2 = bf16_bits_to_float(packed.y & 0xFFFFu), w3 = bf16_bits_to_float(packed.y >> 16);
    // input at relative time b - 3 + i: row b - 3 + i, or state slot b + i
    float earlier[3];
#pragma unroll
    for (uint32_t i = 0; i < 3; ++i) {
        earlier[i] = b + i >= 3 ? qkv[static_cast<size_t>(b + i - 3) * kChannels + c] : history[b + i];
    }
    const float h0 = earlier[0], h1 = earlier[1], h2 = earlier[2];
    const float x = qkv[static_cast<size_t>(b) * kChannels + c];
    float v = 0.0f;
    v += h0 * w0;
    v += h1 * w1;
    v += h2 * w2;
    v += x * w3;
    float y = silu_of(v);
    if (shift) {
        history[0] = h1;
        history[1] = h2;
        history[2] = x;
    }
    if (blockIdx.x < 2u * kKeyHeads) {  // uniform over the block
        const float squares = block_sum(y * y, partial);
        y *= 1.0f / sqrtf(squares + kEpsilon);
    }
    convolved[static_cast<size_t>(b) * kChannels + c] = y;
}

__global__ __launch_bounds__(kLinearHead) void k_linear_conv(const float *qkv,
                                                             const uint16_t *weights,
                                                             float *state, float *convolved) {
    linear_conv_token(qkv, weights, state, convolved, blockIdx.y, gridDim.y == 1);
}

// One decode token of each of up to kRowGroup sequences: row r convolves
// with its own state, which shifts.
__global__ __launch_bounds__(kLinearHead) void k_linear_conv_rows(const float *qkv,
                                                                  const uint16_t *weights,
                                                                  LinearRows rows,
                                                                  float *convolved) {
    const uint32_t r = blockIdx.y;
    linear_conv_token(qkv + static_cast<size_t>(r) * kChannels, weights, rows.convolution[r],
                      convolved + static_cast<size_t>(r) * kChannels, 0, true);
}

// The convolution state after a chunk of `count` tokens: the last three of
// (state, qkv rows) per channel.
__global__ __launch_bounds__(256) void k_conv_history(const float *qkv, uint32_t count,
                                                      float *state) {
    const uint32_t c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= kChannels) {
        return;
    }
    float *history = state + static_cast<size_t>(c) * 3u;
    float next[3];
#pragma unroll
    for (uint32_t i = 0; i < 3; ++i) {
        // slot i holds relative time count - 3 + i
        next[i] = count + i >= 3 ? qkv[static_cast<size_t>(count + i - 3) * kChannels + c]
                                 : history[count + i];
    }
#pragma unroll
    for (uint32_t i = 0; i < 3; ++i) {
        history[i] = next[i];
    }
}

constexpr uint32_t kDeltaTokens = 1024;  // tokens of one k_gated_delta launch, at most

// gated_delta_head (src/executor.cpp:121-155) for state rows [16 y, 16 y +
// 16) of value head x over `count` tokens in order: each wave keeps four
// rows in registers through them, a lane holding two of a row's 128 values
// (src/simd.cpp:108-127); the state is read and written once.
template <uint32_t WAVES>
__device__ __forceinline__ void gated_delta_rows_of_head(const float *convolved, const float *alpha,
                                                         const float *beta,
                                                         const uint16_t *alpha_bias,
                                                         const uint16_t *a_log, uint32_t count,
                                                         float *recurrent, float *output) {
#pragma clang fp contract(off)
    constexpr uint32_t kRows = kDeltaRows / WAVES;  // rows of a wave
    const uint32_t h = blockIdx.x;
    const uint32_t kh = h / (kValueHeads / kKeyHeads);
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t row0 = blockIdx.y * kDeltaRows + wave * kRows;
    const float bias = bf16_bits_to_float(alpha_bias[h]);
    const float rate = expf(bf16_bits_to_float(a_log[h]));
    const float output_scale = 1.0f / sqrtf(static_cast<float>(kLinearHead));
    float2 *state = reinterpret_cast<float2 *>(
        recurrent + (static_cast<size_t>(h) * kLinearHead + row0) * kLinearHead);
    float2 s[kRows];
#pragma unroll
    for (uint32_t j = 0; j < kRows; ++j) {
        s[j] = state[j * (kLinearHead / 2u) + lane];
    }
    // every token's decay and beta gate of the head, one thread a token
    // (count <= kDeltaTokens), so the rows' loop does not wait on them
    __shared__ float token_decay[kDeltaTokens], token_beta[kDeltaTokens];
    for (uint32_t b = threadIdx.x; b < count; b += blockDim.x) {
        token_beta[b] = sigmoid_of(beta[static_cast<size_t>(b) * kValueHeads + h]);
        const float biased = alpha[static_cast<size_t>(b) * kValueHeads + h] + bias;
        const float softplus = biased > 20.0f ? biased : log1pf(expf(biased));
        token_decay[b] = expf(-rate * softplus);
    }
    __syncthreads();
    // a token's inputs, loaded kAhead tokens before its update (a ring of
    // registers; a load past the last token reloads the last, unused)
    struct TokenIn {
        float2 q, k;
        float v[kRows];
    };
    const auto load_token = [&](uint32_t b, TokenIn &in) {
        const float *token = convolved + static_cast<size_t>(b) * kChannels;
        in.q = reinterpret_cast<const float2 *>(token + static_cast<size_t>(kh) * kLinearHead)[lane];
        in.k = reinterpret_cast<const float2 *>(token + kQkSize + static_cast<size_t>(kh) * kLinearHead)[lane];
        const float *v = token + 2u * kQkSize + static_cast<size_t>(h) * kLinearHead + row0;
#pragma unroll
        for (uint32_t j = 0; j < kRows; ++j) {
            in.v[j] = v[j];
        }
    };
    const auto update = [&](uint32_t b, const TokenIn &in) {
        const float beta_value = token_beta[b];
        const float decay = token_decay[b];
        // the rows' chains are independent: one block of code, one store
        float attended[kRows];
#pragma unroll
        for (uint32_t j = 0; j < kRows; ++j) {
            s[j].x *= decay;
            s[j].y *= decay;
            const float prediction = wave_sum(s[j].x * in.k.x + s[j].y * in.k.y);
            const float delta = (in.v[j] - prediction) * beta_value;
            s[j].x += in.k.x * delta;
            s[j].y += in.k.y * delta;
            attended[j] = wave_sum(s[j].x * in.q.x + s[j].y * in.q.y) * output_scale;
        }
        if (lane == 0) {
            float *dst = output + static_cast<size_t>(b) * kValueSize + static_cast<size_t>(h) * kLinearHead + row0;
            if constexpr (kRows == 4) {
                *reinterpret_cast<float4 *>(dst) = make_float4(attended[0], attended[1], attended[2], attended[3]);
            } else if constexpr (kRows == 2) {
                *reinterpret_cast<float2 *>(dst) = make_float2(attended[0], attended[1]);
            } else {
                static_assert(kRows == 1, "one, two or four rows a wave");
                dst[0] = attended[0];
            }
        }
    };
    // ring slot u holds token b0 + u; each slot is refilled (kAhead tokens
    // on) right after its token's update, in whole blocks of kAhead tokens
    // with every slot index a constant, so no register of a load in flight
    // is ever copied
    constexpr uint32_t kAhead = 8;
    TokenIn ring[kAhead];
#pragma unroll
    for (uint32_t u = 0; u < kAhead; ++u) {
        load_token(u < count ? u : count - 1u, ring[u]);
    }
    uint32_t b0 = 0;
    for (; b0 + kAhead <= count; b0 += kAhead) {
#pragma unroll
        for (uint32_t u = 0; u < kAhead; ++u) {
            update(b0 + u, ring[u]);
            const uint32_t next = b0 + u + kAhead;
            load_token(next < count ? next : count - 1u, ring[u]);
        }
    }
#pragma unroll
    for (uint32_t u = 0; u < kAhead; ++u) {
        if (b0 + u < count) {
            update(b0 + u, ring[u]);
        }
    }
#pragma unroll
    for (uint32_t j = 0; j < kRows; ++j) {
        state[j * (kLinearHead / 2u) + lane] = s[j];
    }
}

// Block (value head, row block) over the chunk's `count` tokens: sixteen
// waves of one row (four waves a SIMD, each hiding the others' reductions).
__global__ __launch_bounds__(1024) void k_gated_delta(const float *convolved, const float *alpha,
                                                     const float *beta, const uint16_t *alpha_bias,
                                                     const uint16_t *a_log, uint32_t count,
                                                     float *recurrent, float *output) {
    gated_delta_rows_of_head<16>(convolved, alpha, beta, alpha_bias, a_log, count, recurrent, output);
}

// Block (value head, row block, r): one token of sequence r with its own
// recurrent state.
__global__ __launch_bounds__(256) void k_gated_delta_rows(const float *convolved,
                                                          const float *alpha, const float *beta,
                                                          const uint16_t *alpha_bias,
                                                          const uint16_t *a_log, LinearRows rows,
                                                          float *output) {
    const uint32_t r = blockIdx.z;
    gated_delta_rows_of_head<4>(convolved + static_cast<size_t>(r) * kChannels,
                             alpha + static_cast<size_t>(r) * kValueHeads,
                             beta + static_cast<size_t>(r) * kValueHeads, alpha_bias, a_log, 1,
                             rows.recurrent[r], output + static_cast<size_t>(r) * kValueSize);
}

// The causal convolution and SiLU of channel c for one token whose three
// earlier inputs are in `history` (src/executor.cpp:480-496): the output and
// the channel's shifted state (h1, h2, x).
struct ConvChannel {
    float y, h1, h2, x;
};
__device__ __forceinline__ ConvChannel conv_channel(const float *qkv_row, const uint16_t *weights,
                                                    const float *history, uint32_t c) {
#pragma clang fp contract(off)
    const uint2 packed = *reinterpret_cast<const uint2 *>(weights + static_cast<size_t>(c) * 4u);
    const float w0 = bf16_bits_to_float(packed.x & 0xFFFFu), w1 = bf16_bits_to_float(packed.x >> 16);
    const float w2 = bf16_bits_to_float(packed.y & 0xFFFFu), w3 = bf16_bits_to_float(packed.y >> 16);
    const float h0 = history[0], h1 = history[1], h2 = history[2];
    const float x = qkv_row[c];
    float v = 0.0f;
    v += h0 * w0;
    v += h1 * w1;
    v += h2 * w2;
    v += x * w3;
    return {silu_of(v), h1, h2, x};
}

// One decode token of each of up to kRowGroup sequences through the Gated
// DeltaNet core in one launch: the convolution with the query and key L2
// norms, the delta rule and the gated RMS norm (src/executor.cpp:480-550),
// with the arithmetic of k_linear_conv_rows, k_gated_delta_rows and
// k_linear_norm_gate. Block (value head h, row block y, sequence r):
// - convolves the 128 query and 128 key channels of h's key head itself (the
//   16 blocks of a key head each do, each sum in the 128-thread block's
//   order) and its own 16 value channels, whose state only it shifts;
// - updates its 16 state rows and writes their outputs through to memory;
// - the last of the head's 8 blocks through the head's ticket reads the 128
//   outputs back and writes the head's gated norm; the last of the key
//   head's 16 blocks through its ticket shifts the query and key channels'
//   state (every one of them has read it by then).
// `tickets` holds 48 words a sequence (32 value heads, 16 key heads), zero
// between calls: the last block through each ticket clears it.
// With LANES 8 or 16 the block also computes its head's alpha and beta
// (the bf16 matmuls of the normalized row `x`, in the CPU's LANES-lane order
// as k_bf16_lds does): the row and the two weight rows staged in LDS, one
// wave's lanes 0 .. 2 LANES - 1 running the chains. With LANES 0 they come
// precomputed in alpha and beta.
constexpr uint32_t kDecayColumns = 2048;  // the widest row staged for alpha and beta
template <int LANES>
__global__ __launch_bounds__(256) void k_linear_core_rows(const float *qkv, const uint16_t *weights,
                                                          LinearRows rows, const float *x,
                                                          const uint16_t *alpha_w, const uint16_t *beta_w,
                                                          uint32_t columns, const float *alpha,
                                                          const float *beta, const uint16_t *alpha_bias,
                                                          const uint16_t *a_log, const uint16_t *norm,
                                                          const float *gate, float *recurrent_output,
                                                          float *normalized, uint32_t *tickets) {
#pragma clang fp contract(off)
    constexpr uint32_t kRows = kDeltaRows / 4u;
    constexpr uint32_t kHeadBlocks = kLinearHead / kDeltaRows;
    constexpr uint32_t kStaged = LANES > 0 ? kDecayColumns : 4u;
    __shared__ float qk[2][kLinearHead];
    __shared__ float vv[kDeltaRows];
    __shared__ float part[4];
    __shared__ float decay_in[2];
    __shared__ __align__(16) float x_lds[kStaged];
    __shared__ __align__(16) uint16_t w_lds[2][kStaged];
    __shared__ uint32_t last;
    const uint32_t h = blockIdx.x, y = blockIdx.y, r = blockIdx.z;
    const uint32_t kh = h / (kValueHeads / kKeyHeads);
    const uint32_t t = threadIdx.x, lane = t & 63u, wave = t >> 6;
    const float *row = qkv + static_cast<size_t>(r) * kChannels;
    float *history = rows.convolution[r];
    const uint32_t row0 = y * kDeltaRows + wave * kRows;
    // the state rows first, so that their loads overlap the convolution
    float2 *state = reinterpret_cast<float2 *>(rows.recurrent[r] +
                                               (static_cast<size_t>(h) * kLinearHead + row0) * kLinearHead);
    float2 s[kRows];
#pragma unroll
    for (uint32_t j = 0; j < kRows; ++j) {
        s[j] = state[j * (kLinearHead / 2u) + lane];
    }
    // the row and the head's alpha and beta weight rows (columns <= 2048, a
    // multiple of 256) into LDS: every load issued first (indexes past the
    // row clamped), then the stores
    constexpr uint32_t kX4 = LANES > 0 ? kDecayColumns / 4u / 256u : 1u;
    constexpr uint32_t kW8 = LANES > 0 ? kDecayColumns / 8u / 256u : 1u;
    float4 xv[kX4];
    uint4 av[kW8], bv[kW8];
    if constexpr (LANES > 0) {
        const float4 *xs = reinterpret_cast<const float4 *>(x + static_cast<size_t>(r) * columns);
#pragma unroll
        for (uint32_t k = 0; k < kX4; ++k) {
            xv[k] = xs[min(t + 256u * k, columns / 4u - 1u)];
        }
        const uint4 *wa = reinterpret_cast<const uint4 *>(alpha_w + static_cast<size_t>(h) * columns);
        const uint4 *wb = reinterpret_cast<const uint4 *>(beta_w + static_cast<size_t>(h) * columns);
#pragma unroll
        for (uint32_t k = 0; k < kW8; ++k) {
            av[k] = wa[min(t + 256u * k, columns / 8u - 1u)];
            bv[k] = wb[min(t + 256u * k, columns / 8u - 1u)];
        }
    }
    if constexpr (LANES > 0) {
#pragma unroll
        for (uint32_t k = 0; k < kX4; ++k) {
            if (t + 256u * k < columns / 4u) {
                reinterpret_cast<float4 *>(x_lds)[t + 256u * k] = xv[k];
            }
        }
#pragma unroll
        for (uint32_t k = 0; k < kW8; ++k) {
            if (t + 256u * k < columns / 8u) {
                reinterpret_cast<uint4 *>(w_lds[0])[t + 256u * k] = av[k];
                reinterpret_cast<uint4 *>(w_lds[1])[t + 256u * k] = bv[k];
            }
        }
    }
    // threads 0-127 the query channels, 128-255 the key channels; each L2
    // norm sums as a 128-thread block does: (0 + wave 0) + wave 1
    const uint32_t half = t >> 7;
    const uint32_t c = half * kQkSize + kh * kLinearHead + (t & (kLinearHead - 1u));
    const ConvChannel cc = conv_channel(row, weights, history + static_cast<size_t>(c) * 3u, c);
    const float sq = wave_sum(cc.y * cc.y);
    if (lane == 0) {
        part[wave] = sq;
    }
    if (t < kDeltaRows) {
        const uint32_t cv = 2u * kQkSize + h * kLinearHead + y * kDeltaRows + t;
        float *hv = history + static_cast<size_t>(cv) * 3u;
        const ConvChannel v = conv_channel(row, weights, hv, cv);
        vv[t] = v.y;
        hv[0] = v.h1;
        hv[1] = v.h2;
        hv[2] = v.x;
    }
    __syncthreads();
    float squares = 0.0f;
    squares += part[2u * half];
    squares += part[2u * half + 1u];
    qk[half][t & (kLinearHead - 1u)] = cc.y * (1.0f / sqrtf(squares + kEpsilon));
    if constexpr (LANES > 0) {
        if (wave == 3u) {
            // lanes 0 .. LANES - 1 alpha's chains, LANES .. 2 LANES - 1 beta's
            // (the lanes past them repeat those)
            const uint32_t g = (lane / LANES) & 1u;
            const float acc = router_chain<LANES>(w_lds[g], x_lds, columns, lane % LANES);
            const float a = router_lane_sum<LANES>(acc, 0u);
            const float b = router_lane_sum<LANES>(acc, 1u);
            if (lane == 0) {
                decay_in[0] = a;
                decay_in[1] = b;
            }
        }
    }
    __syncthreads();
    // the delta rule on the block's rows (gated_delta_rows_of_head, one token)
    {
        const float2 q = make_float2(qk[0][2u * lane], qk[0][2u * lane + 1u]);
        const float2 k = make_float2(qk[1][2u * lane], qk[1][2u * lane + 1u]);
        const float bias = bf16_bits_to_float(alpha_bias[h]);
        const float rate = expf(bf16_bits_to_float(a_log[h]));
        const float output_scale = 1.0f / sqrtf(static_cast<float>(kLinearHead));
        const float alpha_in = LANES > 0 ? decay_in[0] : alpha[static_cast<size_t>(r) * kValueHeads + h];
        const float beta_in = LANES > 0 ? decay_in[1] : beta[static_cast<size_t>(r) * kValueHeads + h];
        const float beta_value = sigmoid_of(beta_in);
        const float biased = alpha_in + bias;
        const float softplus = biased > 20.0f ? biased : log1pf(expf(biased));
        const float decay = expf(-rate * softplus);
        float *out = recurrent_output + static_cast<size_t>(r) * kValueSize + static_cast<size_t>(h) * kLinearHead;
        float attended[kRows];  // the rows' chains in one block of code
#pragma unroll
        for (uint32_t j = 0; j < kRows; ++j) {
            s[j].x *= decay;
            s[j].y *= decay;
            const float prediction = wave_sum(s[j].x * k.x + s[j].y * k.y);
            const float delta = (vv[wave * kRows + j] - prediction) * beta_value;
            s[j].x += k.x * delta;
            s[j].y += k.y * delta;
            attended[j] = wave_sum(s[j].x * q.x + s[j].y * q.y) * output_scale;
        }
        if (lane == 0) {
#pragma unroll
            for (uint32_t j = 0; j < kRows; ++j) {
                coherent_store(out + row0 + j, attended[j]);
            }
        }
#pragma unroll
        for (uint32_t j = 0; j < kRows; ++j) {
            state[j * (kLinearHead / 2u) + lane] = s[j];
        }
    }
    uint32_t *ticket = tickets + static_cast<size_t>(r) * (kValueHeads + kKeyHeads);
    wait_stores();
    __syncthreads();
    if (t == 0) {
        last = coherent_add(ticket + h, 1u) + 1u == kHeadBlocks ? 1u : 0u;
    }
    __syncthreads();
    if (last != 0u) {
        // the head's gated RMS norm (k_linear_norm_gate's arithmetic on
        // threads 0-127)
        const size_t i = static_cast<size_t>(r) * kValueSize + static_cast<size_t>(h) * kLinearHead + t;
        const float x = t < kLinearHead ? coherent_load(recurrent_output + i) : 0.0f;
        const float sx = wave_sum(x * x);
        if (lane == 0) {
            part[wave] = sx;
        }
        __syncthreads();
        if (t < kLinearHead) {
            float total = 0.0f;
            total += part[0];
            total += part[1];
            const float scale = 1.0f / sqrtf(total / static_cast<float>(kLinearHead) + kEpsilon);
            normalized[i] = x * scale * (0.0f + bf16_bits_to_float(norm[t])) * silu_of(gate[i]);
        }
        if (t == 0) {
            coherent_store(ticket + h, 0u);
        }
    }
    __syncthreads();
    if (t == 0) {
        last = coherent_add(ticket + kValueHeads + kh, 1u) + 1u == 2u * kHeadBlocks ? 1u : 0u;
    }
    __syncthreads();
    if (last != 0u) {
        float *hc = history + static_cast<size_t>(c) * 3u;
        hc[0] = cc.h1;
        hc[1] = cc.h2;
        hc[2] = cc.x;
        if (t == 0) {
            coherent_store(ticket + kValueHeads + kh, 0u);
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
    const size_t i = static_cast<size_t>(blockIdx.y) * kValueSize +
                     static_cast<size_t>(blockIdx.x) * kLinearHead + threadIdx.x;
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
RopeDivisors rope_divisors() {
    RopeDivisors d{};
    for (uint32_t i = 0; i < kRopeHalf; ++i) {
        d.divisor[i] = std::pow(10000000.0F, 2.0F * static_cast<float>(i) / 64.0F);
    }
    return d;
}

RopeTable rope_table(uint32_t position) {
    const RopeDivisors d = rope_divisors();
    RopeTable t{};
    for (uint32_t i = 0; i < kRopeHalf; ++i) {
        const float theta = static_cast<float>(position) / d.divisor[i];
        t.cosine[i] = std::cos(theta);
        t.sine[i] = std::sin(theta);
    }
    return t;
}

// The context's device table of rope_table(p) for p < end, grown on demand
// (the whole table is rebuilt on the host and copied when it grows).
const float *rope_rows(adi_hip_context *ctx, uint32_t end) {
    if (end > ctx->rope_positions) {
        uint32_t positions = ctx->rope_positions * 2 > 1024 ? ctx->rope_positions * 2 : 1024u;
        positions = positions > end ? positions : end;
        std::vector<float> host(size_t(positions) * 2 * kRopeHalf);
        for (uint32_t p = 0; p < positions; ++p) {
            const RopeTable t = rope_table(p);
            std::copy(t.cosine, t.cosine + kRopeHalf, host.begin() + size_t(p) * 2 * kRopeHalf);
            std::copy(t.sine, t.sine + kRopeHalf,
                      host.begin() + size_t(p) * 2 * kRopeHalf + kRopeHalf);
        }
        ctx->rope_positions = 0;
        ctx->rope_cache.ensure(host.size() * sizeof(float));  // waits for the device before a free
        check_hip(hipStreamSynchronize(ctx->stream), "rope table synchronize");
        check_hip(hipMemcpy(ctx->rope_cache.base, host.data(), host.size() * sizeof(float),
                            hipMemcpyHostToDevice),
                  "rope table upload");
        ctx->rope_positions = positions;
    }
    return static_cast<const float *>(ctx->rope_cache.base);
}

// A nested entry's status becomes this call's failure.
void forward(adi_hip_context *ctx, int status) {
    if (status != ADI_HIP_OK) {
        fail(status, ctx->last_error());
    }
}

// The query (with its gate), key and value projections of the same rows
// (three backend.ne_matmul calls, src/executor.cpp:596-613) in one NE launch
// where it takes the shapes.
void project_qkv(adi_hip_context *ctx, const adi_hip_full_attention *L, const float *inputs,
                 uint32_t count, float *query_gate, float *key, float *value, const NeNormIn *norm_in) {
    const adi_hip_ne_matrix *m[3] = {&L->query, &L->key, &L->value};
    float *out[3] = {query_gate, key, value};
    ne_matmul_group(ctx, m, 3, inputs, count, out, norm_in);
}

// The Gated DeltaNet's qkv and gate projections of the same rows (two
// backend.ne_matmul calls, src/executor.cpp:764-775) in one NE launch where
// it takes the shapes.
void project_qkv_gate(adi_hip_context *ctx, const adi_hip_linear_attention *L, const float *inputs,
                      uint32_t count, float *qkv, float *gate, const NeNormIn *norm_in) {
    const adi_hip_ne_matrix *m[2] = {&L->qkv, &L->gate};
    float *out[2] = {qkv, gate};
    ne_matmul_group(ctx, m, 2, inputs, count, out, norm_in);
}

// The decay inputs alpha and beta of the same rows (two dense bf16 matmuls,
// src/executor.cpp:776-787) in one launch where the small-batch kernel
// takes them (with the one-launch decode paths on).
void project_decay(adi_hip_context *ctx, const adi_hip_linear_attention *L, const float *x, uint32_t count,
                   float *alpha, float *beta) {
    if (!ctx->fused_moe) {
        forward(ctx, adi_hip_bf16_matmul(ctx, &L->alpha, x, count, alpha));
        forward(ctx, adi_hip_bf16_matmul(ctx, &L->beta, x, count, beta));
        return;
    }
    launch_bf16_pair(ctx, L->alpha.values, L->alpha.rows, L->beta.values, L->beta.rows, L->alpha.columns, x,
                     count, alpha, beta, ctx->isa_lanes);
}

// The output projection, then (with `tail`) the residual add and the next
// RMS norm folded into it where the one-launch NE projection takes it.
void project_output(adi_hip_context *ctx, const adi_hip_ne_matrix *m, const float *inputs, uint32_t count,
                    float *outputs, const NeNormTail *tail) {
    if (tail == nullptr) {
        forward(ctx, adi_hip_ne_matmul(ctx, m, inputs, count, outputs));
        return;
    }
    ne_matmul_group(ctx, &m, 1, inputs, count, &outputs, nullptr, tail);
}

bool ne_shaped(const adi_hip_ne_matrix &m, uint32_t rows, uint32_t columns) {
    return m.rows == rows && m.columns == columns && m.trellis != nullptr;
}

// full_attention_forward for tokens position .. position + count - 1.
void full_attention_chunk(adi_hip_context *ctx, const adi_hip_full_attention *L,
                          uint32_t position, uint32_t count, const float *inputs, float *outputs,
                          float *keys, float *values, uint32_t capacity,
                          const NeNormIn *norm_in = nullptr, const NeNormTail *norm_tail = nullptr) {
    require(L != nullptr && inputs != nullptr && outputs != nullptr && keys != nullptr &&
                values != nullptr && count > 0,
            "full attention state or input shape mismatch");
    const uint32_t hidden = L->query.columns;
    require(ne_shaped(L->query, kQueryHeads * kQueryStride, hidden) &&
                ne_shaped(L->key, kKvHeads * kHeadSize, hidden) &&
                ne_shaped(L->value, kKvHeads * kHeadSize, hidden) &&
                ne_shaped(L->output, hidden, kQueryHeads * kHeadSize) &&
                L->query_norm != nullptr && L->key_norm != nullptr && position < capacity &&
                count <= capacity - position,
            "full attention state or input shape mismatch");
    require(aligned_to(keys, 16) && aligned_to(values, 16),
            "attention caches must be 16-byte aligned");
    auto &ws = ctx->layer_workspace;
    ws.used = 0;
    // splits of the history for the chunk's last token; a chunk's many tokens
    // already give blocks enough, so they split less
    const uint32_t last = position + count;
    const uint32_t cap = kMaxSplits / count > 0 ? kMaxSplits / count : 1u;
    uint32_t splits = ceil_div(last, 32);
    splits = splits < 1 ? 1 : (splits > cap ? cap : splits);
    const uint32_t chunk = ceil_div(last, splits);
    splits = ceil_div(last, chunk);
    ws.ensure(Workspace::round(size_t(count) * kQueryHeads * kQueryStride * 4) +
              Workspace::round(size_t(count) * kQueryHeads * kHeadSize * 4) +
              Workspace::round(size_t(count) * kQueryHeads * splits * kPartialStride * 4));
    float *query_gate = ws.take<float>(size_t(count) * kQueryHeads * kQueryStride);
    float *attended = ws.take<float>(size_t(count) * kQueryHeads * kHeadSize);
    float *partial = ws.take<float>(size_t(count) * kQueryHeads * splits * kPartialStride);
    float *key = keys + static_cast<size_t>(position) * kKvHeads * kHeadSize;
    float *value = values + static_cast<size_t>(position) * kKvHeads * kHeadSize;
    project_qkv(ctx, L, inputs, count, query_gate, key, value, norm_in);
    launch(ctx, "attention_norm_rope", k_norm_rope, dim3(kQueryHeads + kKvHeads, count),
           dim3(kHeadSize), 0, query_gate, key, L->query_norm, L->key_norm,
           count == 1 ? rope_table(position) : RopeTable{},
           count == 1 ? nullptr : rope_rows(ctx, position + count), position);
    launch(ctx, "attention_partial", k_attention_partial, dim3(partial_blocks(splits), 1, count),
           dim3(256), 0, static_cast<const float *>(query_gate), static_cast<const float *>(keys),
           static_cast<const float *>(values), position, chunk, splits, partial);
    launch(ctx, "attention_combine", k_attention_combine, dim3(kQueryHeads, count),
           dim3(kHeadSize), 0, static_cast<const float *>(partial), splits,
           static_cast<const float *>(query_gate), attended);
    project_output(ctx, &L->output, attended, count, outputs, norm_tail);
}

// Whether the Gated DeltaNet core launch computes alpha and beta itself from
// the normalized rows x (8- or 16-lane order, rows of at most 2048 columns,
// a multiple of 256, 16-byte aligned).
bool core_takes_decay(const adi_hip_context *ctx, const adi_hip_linear_attention *L, const float *x) {
    const uint32_t columns = L->alpha.columns;
    return (ctx->isa_lanes == 8 || ctx->isa_lanes == 16) && columns <= kDecayColumns && columns % 256u == 0 &&
           aligned_to(x, 16) && aligned_to(L->alpha.values, 16) && aligned_to(L->beta.values, 16);
}

// The Gated DeltaNet core of one token of each of `count` (<= kRowGroup)
// sequences in one launch (k_linear_core_rows): alpha and beta from the
// normalized rows x when core_takes_decay holds, else from alpha and beta.
void launch_linear_core(adi_hip_context *ctx, const adi_hip_linear_attention *L, const float *qkv,
                        const LinearRows &table, uint32_t count, const float *x, const float *alpha,
                        const float *beta, const float *gate, float *recurrent_output, float *normalized) {
    static_assert(kRowGroup * (kValueHeads + kKeyHeads) <= kMoeSyncWords - kMoeSyncLinear,
                  "the DeltaNet tickets fit their sync lines");
    using Kernel = void (*)(const float *, const uint16_t *, LinearRows, const float *, const uint16_t *,
                            const uint16_t *, uint32_t, const float *, const float *, const uint16_t *,
                            const uint16_t *, const uint16_t *, const float *, float *, float *, uint32_t *);
    Kernel kernel = k_linear_core_rows<0>;
    if (core_takes_decay(ctx, L, x)) {
        kernel = ctx->isa_lanes == 16 ? k_linear_core_rows<16> : k_linear_core_rows<8>;
    }
    launch(ctx, "linear_core", kernel, dim3(kValueHeads, kLinearHead / kDeltaRows, count), dim3(256), 0, qkv,
           L->convolution, table, x, L->alpha.values, L->beta.values, L->alpha.columns, alpha, beta,
           L->alpha_bias, L->a_log, L->norm, gate, recurrent_output, normalized, ctx->moe_sync + kMoeSyncLinear);
}

// linear_attention_forward for `count` consecutive tokens.
void linear_attention_chunk(adi_hip_context *ctx, const adi_hip_linear_attention *L,
                            uint32_t count, const float *inputs, float *outputs,
                            float *convolution_state, float *recurrent_state,
                            const NeNormIn *norm_in = nullptr, const NeNormTail *norm_tail = nullptr) {
    require(L != nullptr && inputs != nullptr && outputs != nullptr &&
                convolution_state != nullptr && recurrent_state != nullptr && count > 0,
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
    const size_t n = count;
    ws.ensure(Workspace::round(n * kChannels * 4) * 2 + Workspace::round(n * kValueSize * 4) * 3 +
              Workspace::round(n * kValueHeads * 4) * 2);
    float *qkv = ws.take<float>(n * kChannels);
    float *convolved = ws.take<float>(n * kChannels);
    float *gate = ws.take<float>(n * kValueSize);
    float *recurrent_output = ws.take<float>(n * kValueSize);
    float *normalized = ws.take<float>(n * kValueSize);
    float *alpha = ws.take<float>(n * kValueHeads);
    float *beta = ws.take<float>(n * kValueHeads);
    project_qkv_gate(ctx, L, inputs, count, qkv, gate, norm_in);
    const float *x = norm_in != nullptr ? norm_in->out : inputs;  // the normalized rows
    if (count == 1 && ctx->fused_moe) {
        if (!core_takes_decay(ctx, L, x)) {
            project_decay(ctx, L, x, count, alpha, beta);
        }
        LinearRows table{};
        table.convolution[0] = convolution_state;
        table.recurrent[0] = recurrent_state;
        launch_linear_core(ctx, L, qkv, table, 1, x, alpha, beta, gate, recurrent_output, normalized);
        project_output(ctx, &L->output, normalized, count, outputs, norm_tail);
        return;
    }
    project_decay(ctx, L, x, count, alpha, beta);
    launch(ctx, "linear_conv", k_linear_conv, dim3(kChannels / kLinearHead, count),
           dim3(kLinearHead), 0, static_cast<const float *>(qkv), L->convolution,
           convolution_state, convolved);
    if (count > 1) {
        launch(ctx, "linear_conv_history", k_conv_history, dim3(kChannels / 256), dim3(256), 0,
               static_cast<const float *>(qkv), count, convolution_state);
    }
    // at most kDeltaTokens tokens a launch; the state carries over in order
    for (uint32_t b0 = 0; b0 < count; b0 += kDeltaTokens) {
        const uint32_t n = count - b0 < kDeltaTokens ? count - b0 : kDeltaTokens;
        launch(ctx, "gated_delta", k_gated_delta, dim3(kValueHeads, kLinearHead / kDeltaRows), dim3(1024), 0,
               static_cast<const float *>(convolved + static_cast<size_t>(b0) * kChannels),
               static_cast<const float *>(alpha + static_cast<size_t>(b0) * kValueHeads),
               static_cast<const float *>(beta + static_cast<size_t>(b0) * kValueHeads), L->alpha_bias, L->a_log,
               n, recurrent_state, recurrent_output + static_cast<size_t>(b0) * kValueSize);
    }
    launch(ctx, "linear_norm_gate", k_linear_norm_gate, dim3(kValueHeads, count),
           dim3(kLinearHead), 0, static_cast<const float *>(recurrent_output), L->norm,
           static_cast<const float *>(gate), normalized);
    project_output(ctx, &L->output, normalized, count, outputs, norm_tail);
}

// decode_layer for `count` consecutive tokens of rows `hidden`.
// The decoder layer on rows hidden[count][moe.hidden] (decode_layer,
// src/executor.cpp:1473-1529) up to its MoE block: hidden (+= pending, the
// previous layer's MoE rows, when given) is normalized, the attention's rows
// are added to it and normalized again, each add fused into its norm; the MoE
// rows go to moe_out (may be `pending`: that is read first), not yet added.
template <typename Attention>
void layer_body(adi_hip_context *ctx, const adi_hip_decoder_layer *L, uint32_t count,
                float *hidden, const float *pending, float *moe_out, Attention &&attention) {
    require(L != nullptr && hidden != nullptr && moe_out != nullptr && L->input_norm != nullptr &&
                L->post_attention_norm != nullptr && count > 0,
            "decoder layer input is null");
    const uint32_t n = L->moe.hidden;
    require(n > 0 && aligned_to(hidden, 16), "decoder hidden row must be 16-byte aligned");
    auto &ws = ctx->decoder_workspace;
    ws.used = 0;
    const size_t rows = size_t(count) * n;
    ws.ensure(Workspace::round(rows * 4) * 2);
    float *normalized = ws.take<float>(rows);
    float *branch = ws.take<float>(rows);
    // the input norm (with the residual add of the previous layer's MoE rows)
    // and the post-attention norm run inside the attention's first and last
    // projections where they can, else as norm launches around them
    const NeNormIn norm_in{hidden, pending, L->input_norm, normalized};
    const NeNormTail norm_tail{hidden, L->post_attention_norm, normalized};
    attention(static_cast<const float *>(normalized), branch, &norm_in, &norm_tail);
    forward(ctx, adi_hip_moe_forward(ctx, &L->moe, normalized, count, nullptr, moe_out, nullptr,
                                     nullptr));
}

// `count` consecutive tokens of one sequence at position .. position + count
// - 1 (pending and moe_out as layer_body's).
void decoder_chunk_body(adi_hip_context *ctx, const adi_hip_decoder_layer *L, uint32_t position,
                        uint32_t count, float *hidden, const float *pending, float *moe_out,
                        const adi_hip_layer_state *state) {
    require(state != nullptr, "decoder layer input is null");
    layer_body(ctx, L, count, hidden, pending, moe_out,
               [&](const float *in, float *out, const NeNormIn *norm_in, const NeNormTail *norm_tail) {
        if (L->full_attention != 0) {
            full_attention_chunk(ctx, &L->full, position, count, in, out, state->keys,
                                 state->values, state->capacity, norm_in, norm_tail);
        } else {
            linear_attention_chunk(ctx, &L->linear, count, in, out, state->convolution,
                                   state->recurrent, norm_in, norm_tail);
        }
    });
}

// The whole layer in place (the public layer entries): the MoE rows are
// added to hidden at the end.
void decoder_chunk(adi_hip_context *ctx, const adi_hip_decoder_layer *L, uint32_t position,
                   uint32_t count, float *hidden, const adi_hip_layer_state *state) {
    require(L != nullptr && hidden != nullptr && count > 0, "decoder layer input is null");
    auto &ws = ctx->layer_output;
    ws.used = 0;
    const size_t rows = size_t(count) * L->moe.hidden;
    ws.ensure(Workspace::round(rows * 4));
    float *moe_out = ws.take<float>(rows);
    decoder_chunk_body(ctx, L, position, count, hidden, nullptr, moe_out, state);
    launch(ctx, "residual_add", k_residual_add, dim3(ceil_div(rows, 256)), dim3(256), 0, hidden,
           static_cast<const float *>(moe_out), static_cast<uint32_t>(rows));
}

// full_attention_forward_batch (src/executor.cpp:561-731) for one decode
// token of each of `rows` sequences: row r is at positions[r] of the
// sequence whose cache is states[r]; the kernels read the positions from
// device_positions. The launches cover positions below `span` (the RoPE
// table and the grid's splits; at least every positions[r] + 1). The
// projections run batched over the rows; normalization, RoPE, the cache
// append and the attention run per sequence, kRowGroup sequences per launch.
void full_attention_rows(adi_hip_context *ctx, const adi_hip_full_attention *L, uint32_t rows,
                         const float *inputs, float *outputs,
                         const adi_hip_layer_state *const *states, const uint32_t *positions,
                         const uint32_t *device_positions, uint32_t span,
                         const NeNormIn *norm_in, const NeNormTail *norm_tail) {
    require(L != nullptr && inputs != nullptr && outputs != nullptr && states != nullptr &&
                positions != nullptr && device_positions != nullptr && rows > 0,
            "full attention batch shape mismatch");
    const uint32_t hidden = L->query.columns;
    require(ne_shaped(L->query, kQueryHeads * kQueryStride, hidden) &&
                ne_shaped(L->key, kKvHeads * kHeadSize, hidden) &&
                ne_shaped(L->value, kKvHeads * kHeadSize, hidden) &&
                ne_shaped(L->output, hidden, kQueryHeads * kHeadSize) &&
                L->query_norm != nullptr && L->key_norm != nullptr,
            "full attention batch shape mismatch");
    uint32_t last = 0;
    for (uint32_t r = 0; r < rows; ++r) {
        const adi_hip_layer_state *st = states[r];
        require(st != nullptr && st->keys != nullptr && st->values != nullptr &&
                    positions[r] < st->capacity,
                "full attention batch state mismatch");
        require(aligned_to(st->keys, 16) && aligned_to(st->values, 16),
                "attention caches must be 16-byte aligned");
        last = positions[r] + 1 > last ? positions[r] + 1 : last;
    }
    last = span > last ? span : last;
    auto &ws = ctx->layer_workspace;
    ws.used = 0;
    const uint32_t cap = kMaxSplits / rows > 0 ? kMaxSplits / rows : 1u;
    const uint32_t splits = row_splits(last, cap);
    const size_t n = rows;
    ws.ensure(Workspace::round(n * kQueryHeads * kQueryStride * 4) +
              Workspace::round(n * kKvHeads * kHeadSize * 4) * 2 +
              Workspace::round(n * kQueryHeads * kHeadSize * 4) +
              Workspace::round(n * kQueryHeads * splits * kPartialStride * 4));
    float *query_gate = ws.take<float>(n * kQueryHeads * kQueryStride);
    float *key = ws.take<float>(n * kKvHeads * kHeadSize);
    float *value = ws.take<float>(n * kKvHeads * kHeadSize);
    float *attended = ws.take<float>(n * kQueryHeads * kHeadSize);
    float *partial = ws.take<float>(n * kQueryHeads * splits * kPartialStride);
    project_qkv(ctx, L, inputs, rows, query_gate, key, value, norm_in);
    const float *rope = rope_rows(ctx, last);
    for (uint32_t first = 0; first < rows; first += kRowGroup) {
        const uint32_t count = rows - first < kRowGroup ? rows - first : kRowGroup;
        FullRows table{};
        for (uint32_t i = 0; i < count; ++i) {
            table.keys[i] = states[first + i]->keys;
            table.values[i] = states[first + i]->values;
        }
        const uint32_t *row_positions = device_positions + first;
        float *qg = query_gate + static_cast<size_t>(first) * kQueryHeads * kQueryStride;
        if (ctx->fused_moe) {
            static_assert(kRowGroup * kQueryHeads <= kMoeSyncWords - kMoeSyncAttention,
                          "the attention tickets fit their sync line");
            launch(ctx, "attention_rows_one", k_attention_rows_one, dim3(partial_blocks(splits), 1, count),
                   dim3(256), 0, static_cast<const float *>(qg),
                   static_cast<const float *>(key + static_cast<size_t>(first) * kKvHeads * kHeadSize),
                   static_cast<const float *>(value + static_cast<size_t>(first) * kKvHeads * kHeadSize),
                   L->query_norm, L->key_norm, rope, table, row_positions, cap, splits,
                   partial + static_cast<size_t>(first) * kQueryHeads * splits * kPartialStride,
                   attended + static_cast<size_t>(first) * kQueryHeads * kHeadSize,
                   ctx->moe_sync + kMoeSyncAttention);
            continue;
        }
        launch(ctx, "attention_norm_rope_rows", k_norm_rope_rows,
               dim3(kQueryHeads + 2 * kKvHeads, count), dim3(kHeadSize), 0, qg,
               static_cast<const float *>(key + static_cast<size_t>(first) * kKvHeads * kHeadSize),
               static_cast<const float *>(value + static_cast<size_t>(first) * kKvHeads * kHeadSize),
               L->query_norm, L->key_norm, rope, table, row_positions);
        launch(ctx, "attention_partial_rows", k_attention_partial_rows,
               dim3(partial_blocks(splits), 1, count), dim3(256), 0, static_cast<const float *>(qg), table,
               row_positions, cap, splits,
               partial + static_cast<size_t>(first) * kQueryHeads * splits * kPartialStride);
        launch(ctx, "attention_combine", k_attention_combine, dim3(kQueryHeads, count), dim3(kHeadSize), 0,
               static_cast<const float *>(partial + static_cast<size_t>(first) * kQueryHeads * splits * kPartialStride),
               splits, static_cast<const float *>(qg), attended + static_cast<size_t>(first) * kQueryHeads * kHeadSize);
    }
    project_output(ctx, &L->output, attended, rows, outputs, norm_tail);
}

// linear_attention_forward_batch (src/executor.cpp:733-966) for one decode
// token of each of `rows` sequences with the states states[r]: projections
// batched, convolution and recurrence per sequence.
void linear_attention_rows(adi_hip_context *ctx, const adi_hip_linear_attention *L, uint32_t rows,
                           const float *inputs, float *outputs,
                           const adi_hip_layer_state *const *states,
                           const NeNormIn *norm_in, const NeNormTail *norm_tail) {
    require(L != nullptr && inputs != nullptr && outputs != nullptr && states != nullptr &&
                rows > 0,
            "linear attention batch shape mismatch");
    const uint32_t hidden = L->qkv.columns;
    require(ne_shaped(L->qkv, kChannels, hidden) && ne_shaped(L->gate, kValueSize, hidden) &&
                ne_shaped(L->output, hidden, kValueSize),
            "linear attention batch shape mismatch");
    require(L->alpha.rows == kValueHeads && L->alpha.columns == hidden &&
                L->beta.rows == kValueHeads && L->beta.columns == hidden &&
                L->alpha.values != nullptr && L->beta.values != nullptr &&
                L->alpha_bias != nullptr && L->a_log != nullptr,
            "linear attention decay shape mismatch");
    require(L->convolution != nullptr && aligned_to(L->convolution, 8),
            "linear attention convolution shape mismatch");
    require(L->norm != nullptr, "linear attention batch shape mismatch");
    for (uint32_t r = 0; r < rows; ++r) {
        const adi_hip_layer_state *st = states[r];
        require(st != nullptr && st->convolution != nullptr && st->recurrent != nullptr,
                "linear attention recurrent state mismatch");
        require(aligned_to(st->recurrent, 8), "linear attention state must be 8-byte aligned");
    }
    auto &ws = ctx->layer_workspace;
    ws.used = 0;
    const size_t n = rows;
    ws.ensure(Workspace::round(n * kChannels * 4) * 2 + Workspace::round(n * kValueSize * 4) * 3 +
              Workspace::round(n * kValueHeads * 4) * 2);
    float *qkv = ws.take<float>(n * kChannels);
    float *convolved = ws.take<float>(n * kChannels);
    float *gate = ws.take<float>(n * kValueSize);
    float *recurrent_output = ws.take<float>(n * kValueSize);
    float *normalized = ws.take<float>(n * kValueSize);
    float *alpha = ws.take<float>(n * kValueHeads);
    float *beta = ws.take<float>(n * kValueHeads);
    project_qkv_gate(ctx, L, inputs, rows, qkv, gate, norm_in);
    const float *x = norm_in != nullptr ? norm_in->out : inputs;  // the normalized rows
    if (!ctx->fused_moe || !core_takes_decay(ctx, L, x)) {
        project_decay(ctx, L, x, rows, alpha, beta);
    }
    for (uint32_t first = 0; first < rows; first += kRowGroup) {
        const uint32_t count = rows - first < kRowGroup ? rows - first : kRowGroup;
        LinearRows table{};
        for (uint32_t i = 0; i < count; ++i) {
            table.convolution[i] = states[first + i]->convolution;
            table.recurrent[i] = states[first + i]->recurrent;
        }
        const size_t at = static_cast<size_t>(first);
        if (ctx->fused_moe) {
            launch_linear_core(ctx, L, qkv + at * kChannels, table, count, x + at * L->alpha.columns,
                               alpha + at * kValueHeads, beta + at * kValueHeads, gate + at * kValueSize,
                               recurrent_output + at * kValueSize, normalized + at * kValueSize);
            continue;
        }
        launch(ctx, "linear_conv_rows", k_linear_conv_rows, dim3(kChannels / kLinearHead, count),
               dim3(kLinearHead), 0, static_cast<const float *>(qkv + at * kChannels),
               L->convolution, table, convolved + at * kChannels);
        launch(ctx, "gated_delta_rows", k_gated_delta_rows,
               dim3(kValueHeads, kLinearHead / kDeltaRows, count), dim3(256), 0,
               static_cast<const float *>(convolved + at * kChannels),
               static_cast<const float *>(alpha + at * kValueHeads),
               static_cast<const float *>(beta + at * kValueHeads), L->alpha_bias, L->a_log, table,
               recurrent_output + at * kValueSize);
        launch(ctx, "linear_norm_gate", k_linear_norm_gate, dim3(kValueHeads, count), dim3(kLinearHead),
               0, static_cast<const float *>(recurrent_output + at * kValueSize), L->norm,
               static_cast<const float *>(gate + at * kValueSize), normalized + at * kValueSize);
    }
    project_output(ctx, &L->output, normalized, rows, outputs, norm_tail);
}

}  // namespace

void decoder_rows(adi_hip_context *ctx, const adi_hip_decoder_layer *L, uint32_t rows,
                  float *hidden, const float *pending, float *moe_out,
                  const adi_hip_layer_state *const *states, const uint32_t *positions,
                  const uint32_t *device_positions, uint32_t span) {
    require(states != nullptr && positions != nullptr, "decoder batch shape mismatch");
    layer_body(ctx, L, rows, hidden, pending, moe_out,
               [&](const float *in, float *out, const NeNormIn *norm_in, const NeNormTail *norm_tail) {
        if (L->full_attention != 0) {
            full_attention_rows(ctx, &L->full, rows, in, out, states, positions, device_positions,
                                span, norm_in, norm_tail);
        } else {
            linear_attention_rows(ctx, &L->linear, rows, in, out, states, norm_in, norm_tail);
        }
    });
}

void prefill_chunk(adi_hip_context *ctx, const adi_hip_decoder_layer *L, uint32_t position,
                   uint32_t count, float *hidden, const float *pending, float *moe_out,
                   const adi_hip_layer_state *state) {
    decoder_chunk_body(ctx, L, position, count, hidden, pending, moe_out, state);
}

}  // namespace adi_hip

using namespace adi_hip;

extern "C" {

int adi_hip_full_attention_forward(adi_hip_context *ctx, const adi_hip_full_attention *L,
                                   uint32_t position, const float *input, float *output,
                                   float *keys, float *values, uint32_t capacity) {
    return guarded(ctx, [&] {
        full_attention_chunk(ctx, L, position, 1, input, output, keys, values, capacity);
    });
}

int adi_hip_full_attention_prefill(adi_hip_context *ctx, const adi_hip_full_attention *L,
                                   uint32_t position, uint32_t count, const float *inputs,
                                   float *outputs, float *keys, float *values, uint32_t capacity) {
    return guarded(ctx, [&] {
        full_attention_chunk(ctx, L, position, count, inputs, outputs, keys, values, capacity);
    });
}

int adi_hip_linear_attention_forward(adi_hip_context *ctx, const adi_hip_linear_attention *L,
                                     const float *input, float *output, float *convolution_state,
                                     float *recurrent_state) {
    return guarded(ctx, [&] {
        linear_attention_chunk(ctx, L, 1, input, output, convolution_state, recurrent_state);
    });
}

int adi_hip_linear_attention_prefill(adi_hip_context *ctx, const adi_hip_linear_attention *L,
                                     uint32_t count, const float *inputs, float *outputs,
                                     float *convolution_state, float *recurrent_state) {
    return guarded(ctx, [&] {
        linear_attention_chunk(ctx, L, count, inputs, outputs, convolution_state, recurrent_state);
    });
}

int adi_hip_decode_layer(adi_hip_context *ctx, const adi_hip_decoder_layer *L, uint32_t position,
                         float *hidden, const adi_hip_layer_state *state) {
    return guarded(ctx, [&] { decoder_chunk(ctx, L, position, 1, hidden, state); });
}

int adi_hip_prefill_layer(adi_hip_context *ctx, const adi_hip_decoder_layer *L, uint32_t position,
                          uint32_t count, float *hidden, const adi_hip_layer_state *state) {
    return guarded(ctx, [&] { decoder_chunk(ctx, L, position, count, hidden, state); });
}

}  // extern "C"
