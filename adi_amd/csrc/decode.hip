// decode.hip -- the token side of a decode step on the device: embedding rows
// (mach_embedding_row, src/kernels.cpp:802-845) and the greedy choice of
// sample_token (src/generation.cpp:161-183), so a step's token goes from the
// head's logits to the next step's hidden state without leaving HBM.
#include "context.hpp"

#include <algorithm>
#include <cmath>

namespace adi_hip {
namespace {

constexpr uint32_t kEmbeddingThreads = 256;
constexpr uint32_t kArgmaxThreads = 1024;

// Calls f(i, v) for every logit of a row, each index once, from this thread's
// share of the block: 16-byte loads with four in flight when the row is
// 16-byte aligned, one float at a time otherwise. The order is fixed by the
// row length and the block size.
template <typename F>
__device__ __forceinline__ void for_each_logit(const float *row, uint32_t count, F &&f) {
    const uint32_t step = blockDim.x;
    if ((reinterpret_cast<uintptr_t>(row) & 15u) == 0u) {
        const uint32_t vectors = count / 4u;
        const float4 *r4 = reinterpret_cast<const float4 *>(row);
        uint32_t j = threadIdx.x;
        for (; j + 3u * step < vectors; j += 4u * step) {
            float4 a[4];
#pragma unroll
            for (uint32_t u = 0; u < 4; ++u) {
                a[u] = r4[j + u * step];
            }
#pragma unroll
            for (uint32_t u = 0; u < 4; ++u) {
                const uint32_t i = 4u * (j + u * step);
                f(i, a[u].x);
                f(i + 1u, a[u].y);
                f(i + 2u, a[u].z);
                f(i + 3u, a[u].w);
            }
        }
        for (; j < vectors; j += step) {
            const float4 a = r4[j];
            f(4u * j, a.x);
            f(4u * j + 1u, a.y);
            f(4u * j + 2u, a.z);
            f(4u * j + 3u, a.w);
        }
        for (uint32_t i = 4u * vectors + threadIdx.x; i < count; i += step) {
            f(i, row[i]);
        }
    } else {
        for (uint32_t i = threadIdx.x; i < count; i += step) {
            f(i, row[i]);
        }
    }
}

// First index of `key` in the ascending list, or `count` (lower_bound).
__device__ __forceinline__ uint32_t lower_bound_u32(const uint32_t *list, uint32_t count,
                                                    uint64_t key) {
    uint32_t lo = 0, hi = count;
    while (lo < hi) {
        const uint32_t mid = lo + ((hi - lo) >> 1);
        if (list[mid] < key) {
            lo = mid + 1;
        } else {
            hi = mid;
        }
    }
    return lo;
}

// One block per token. Thread t decodes eight consecutive columns per round
// from one 4-byte load of codes (high nibble first); one thread meanwhile
// finds the row's exceptions by lower_bound, and after a block barrier the
// block overwrites those columns.
__global__ __launch_bounds__(kEmbeddingThreads) void k_embedding_rows(adi_hip_embedding e,
                                                                      const uint32_t *tokens,
                                                                      float *out) {
#pragma clang fp contract(off)
    __shared__ uint32_t range[2];
    const uint32_t token = tokens[blockIdx.x];
    float *row = out + static_cast<size_t>(blockIdx.x) * e.columns;
    if (token >= e.rows) {
        for (uint32_t c = threadIdx.x; c < e.columns; c += blockDim.x) {
            row[c] = __builtin_nanf("");
        }
        return;  // block-uniform: the token is the block's
    }
    const uint64_t first = static_cast<uint64_t>(token) * e.columns;
    if (threadIdx.x == 0) {
        range[0] = lower_bound_u32(e.exception_indexes, e.exception_count, first);
        range[1] = lower_bound_u32(e.exception_indexes, e.exception_count, first + e.columns);
    }
    const uint8_t *codes = e.packed + first / 2;
    const uint16_t *mins = e.minimum_f16 + first / 64;
    const uint16_t *maxs = e.maximum_f16 + first / 64;
    for (uint32_t c0 = threadIdx.x * 8u; c0 < e.columns; c0 += 8u * blockDim.x) {
        const uint32_t bytes = *reinterpret_cast<const uint32_t *>(codes + c0 / 2);
        const float minimum = half_bits_to_float(mins[c0 / 64]);
        const float maximum = half_bits_to_float(maxs[c0 / 64]);
        const float span = maximum - minimum;
        const float step = (span < 1.0e-8f ? 1.0e-8f : span) / 15.0f;
        float v[8];
#pragma unroll
        for (uint32_t q = 0; q < 8; ++q) {
            const uint32_t byte = (bytes >> (8u * (q / 2))) & 0xFFu;
            const uint32_t code = (q & 1u) == 0 ? byte >> 4 : byte & 0x0Fu;
            v[q] = minimum + static_cast<float>(code) * step;
        }
        *reinterpret_cast<float4 *>(row + c0) = make_float4(v[0], v[1], v[2], v[3]);
        *reinterpret_cast<float4 *>(row + c0 + 4) = make_float4(v[4], v[5], v[6], v[7]);
    }
    __syncthreads();
    for (uint32_t i = range[0] + threadIdx.x; i < range[1]; i += blockDim.x) {
        row[e.exception_indexes[i] - first] = bf16_bits_to_float(e.exception_bf16[i]);
    }
}

// The larger of two (value, index) candidates; equal values keep the lower
// index, so the block's answer is std::max_element's first maximum.
__device__ __forceinline__ void better(float &value, uint32_t &index, float v, uint32_t i) {
    if (v > value || (v == value && i < index)) {
        value = v;
        index = i;
    }
}

// Wave and block reductions of a thread's (value, index, bad); thread 0 of
// the block returns the block's answer.
__device__ __forceinline__ void argmax_block(float &value, uint32_t &index, uint32_t &bad) {
    __shared__ float wave_value[kArgmaxThreads / kWave];
    __shared__ uint32_t wave_index[kArgmaxThreads / kWave];
    __shared__ uint32_t wave_bad[kArgmaxThreads / kWave];
#pragma unroll
    for (int offset = 32; offset > 0; offset >>= 1) {
        const float v = __shfl_xor(value, offset);
        const uint32_t i = static_cast<uint32_t>(__shfl_xor(static_cast<int>(index), offset));
        better(value, index, v, i);
        bad |= static_cast<uint32_t>(__shfl_xor(static_cast<int>(bad), offset));
    }
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    if (lane == 0) {
        wave_value[wave] = value;
        wave_index[wave] = index;
        wave_bad[wave] = bad;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (uint32_t w = 1; w < blockDim.x / kWave; ++w) {
            better(value, index, wave_value[w], wave_index[w]);
            bad |= wave_bad[w];
        }
    }
}

// One block per row: each thread scans a strided share, then wave and block
// reductions of (value, index); any non-finite logit marks the row.
__global__ __launch_bounds__(kArgmaxThreads) void k_argmax_rows(const float *logits,
                                                                uint32_t count,
                                                                uint32_t *tokens) {
    const float *row = logits + static_cast<size_t>(blockIdx.x) * count;
    float value = -__builtin_huge_valf();
    uint32_t index = 0xFFFFFFFFu;
    uint32_t bad = 0;
    for_each_logit(row, count, [&](uint32_t i, float v) {
        bad |= __builtin_isfinite(v) ? 0u : 1u;
        better(value, index, v, i);
    });
    argmax_block(value, index, bad);
    if (threadIdx.x == 0) {
        tokens[blockIdx.x] = bad != 0u ? 0xFFFFFFFFu : index;
    }
}

// A long row splits into `gridDim.x` spans of `span` logits (a multiple of 4,
// so an aligned row keeps its spans aligned); block (p, r) reduces span p of
// row r into partial p of that row. The answer does not depend on the split:
// better() keeps the larger value and, among equal values, the lower index.
constexpr uint32_t kArgmaxPartThreads = 256;
constexpr uint32_t kArgmaxMaxParts = 64;
constexpr uint32_t kArgmaxSplitCount = 32768;  // shorter rows take one block

__global__ __launch_bounds__(kArgmaxPartThreads) void k_argmax_parts(
    const float *logits, uint32_t count, uint32_t span, float *part_value,
    uint32_t *part_index, uint32_t *zero, uint32_t zero_words, uint32_t zero_stride) {
    if (zero != nullptr) {
        // the sampler's per-row bins and state (the first zero_words of each
        // row's zero_stride), cleared for the launches after
        const uint32_t share = (zero_words + gridDim.x - 1u) / gridDim.x;
        uint32_t *words = zero + static_cast<size_t>(blockIdx.y) * zero_stride;
        const uint32_t w0 = blockIdx.x * share, w1 = w0 + share < zero_words ? w0 + share : zero_words;
        for (uint32_t w = w0 + threadIdx.x; w < w1; w += blockDim.x) {
            words[w] = 0u;
        }
    }
    const uint32_t begin = blockIdx.x * span;
    const uint32_t end = begin + span < count ? begin + span : count;
    const float *row = logits + static_cast<size_t>(blockIdx.y) * count + begin;
    float value = -__builtin_huge_valf();
    uint32_t index = 0xFFFFFFFFu;
    uint32_t bad = 0;
    for_each_logit(row, end - begin, [&](uint32_t i, float v) {
        bad |= __builtin_isfinite(v) ? 0u : 1u;
        better(value, index, v, begin + i);
    });
    argmax_block(value, index, bad);
    if (threadIdx.x == 0) {
        const size_t slot = static_cast<size_t>(blockIdx.y) * gridDim.x + blockIdx.x;
        part_value[slot] = value;
        part_index[slot] = bad != 0u ? 0xFFFFFFFFu : index;
    }
}

// One wave per row folds that row's `parts` partials; a partial index of
// 0xFFFFFFFF marks a span that held a non-finite logit (every span holds at
// least one logit, so no finite span reports that index).
__global__ __launch_bounds__(kWave) void k_argmax_finish(const float *part_value,
                                                         const uint32_t *part_index,
                                                         uint32_t parts, uint32_t *tokens) {
    const size_t base = static_cast<size_t>(blockIdx.x) * parts;
    float value = -__builtin_huge_valf();
    uint32_t index = 0xFFFFFFFFu;
    uint32_t bad = 0;
    for (uint32_t p = threadIdx.x; p < parts; p += kWave) {
        const uint32_t i = part_index[base + p];
        bad |= i == 0xFFFFFFFFu ? 1u : 0u;
        better(value, index, part_value[base + p], i);
    }
#pragma unroll
    for (int offset = 32; offset > 0; offset >>= 1) {
        const float v = __shfl_xor(value, offset);
        const uint32_t i = static_cast<uint32_t>(__shfl_xor(static_cast<int>(index), offset));
        better(value, index, v, i);
        bad |= static_cast<uint32_t>(__shfl_xor(static_cast<int>(bad), offset));
    }
    if (threadIdx.x == 0) {
        tokens[blockIdx.x] = bad != 0u ? 0xFFFFFFFFu : index;
    }
}

// Greedy choice of every row: rows of at least kArgmaxSplitCount logits split
// over up to kArgmaxMaxParts blocks each (a 248,320-logit row is one block's
// worth of latency otherwise), shorter rows take one block.
void launch_argmax(adi_hip_context *ctx, const float *logits, uint32_t rows, uint32_t count,
                   uint32_t *tokens) {
    if (count < kArgmaxSplitCount || rows > 65535u) {
        launch(ctx, "argmax", k_argmax_rows, dim3(rows), dim3(kArgmaxThreads), 0, logits, count,
               tokens);
        return;
    }
    const uint32_t wanted = std::min<uint32_t>(kArgmaxMaxParts, ceil_div(count, 4096));
    const uint32_t span = (ceil_div(count, wanted) + 3u) & ~3u;
    const uint32_t parts = ceil_div(count, span);
    auto &ws = ctx->workspace;
    ws.used = 0;
    ws.ensure(Workspace::round(size_t(rows) * parts * 4) * 2);
    float *part_value = ws.take<float>(size_t(rows) * parts);
    uint32_t *part_index = ws.take<uint32_t>(size_t(rows) * parts);
    launch(ctx, "argmax_parts", k_argmax_parts, dim3(parts, rows), dim3(kArgmaxPartThreads), 0,
           logits, count, span, part_value, part_index, static_cast<uint32_t *>(nullptr), 0u, 0u);
    launch(ctx, "argmax_finish", k_argmax_finish, dim3(rows), dim3(kWave), 0,
           static_cast<const float *>(part_value), static_cast<const uint32_t *>(part_index),
           parts, tokens);
}

// ---- top-p sampling ----------------------------------------------------------

constexpr uint32_t kSampleThreads = 1024;
constexpr uint32_t kSampleWaves = kSampleThreads / kWave;
constexpr uint32_t kWindow = 4096;  // candidates sorted and walked at a time

// The sampler's words of a long row (after the span maxima and sums): token
// counts and float masses p of 4096 bins of the descending key's top 12 bits,
// the state of the short walk, then up to kWindow candidates (key, index).
constexpr uint32_t kTopBins = 4096, kTopShift = 20;
constexpr uint32_t kTopState = 2 * kTopBins;      // appended, expected, decided
constexpr uint32_t kTopCand = kTopState + 8;      // 8-byte aligned
constexpr uint32_t kTopRowWords = kTopCand + 2 * kWindow;
constexpr uint32_t kTopZeroWords = kTopState + 4;  // cleared before a call

// Ascending order of this key is descending logit order, with -0 folded into
// +0 (src/generation.cpp:36-47); ties keep ascending token order.
__device__ __forceinline__ uint32_t descending_key(float v) {
    const uint32_t bits = v == 0.0f ? 0u : __float_as_uint(v);
    const uint32_t ascending = (bits & 0x80000000u) != 0u ? ~bits : bits ^ 0x80000000u;
    return ~ascending;
}

// The split denominator of a long row: block (p, r) folds row r's span maxima
// (k_argmax_parts: the maximum is the same in any order) and sums
// exp((v - max) / t) in double over span p, each thread in index order, then
// a fixed tree; k_sample_rows adds the spans' sums in span order. A row with
// a non-finite logit (a span index of 0xFFFFFFFF) gets sums of 0: the
// sampler rejects it.
__global__ __launch_bounds__(kArgmaxPartThreads) void k_expsum_parts(
    const float *logits, uint32_t count, uint32_t span, const float *part_value,
    const uint32_t *part_index, float temperature, double *part_sum, uint32_t *top) {
    __shared__ double wave_sum[kArgmaxPartThreads / kWave];
    // with `top`: the span's bin counts and masses, added into the row's
    __shared__ uint32_t bin_count[kTopBins];
    __shared__ float bin_mass[kTopBins];
    const size_t base = static_cast<size_t>(blockIdx.y) * gridDim.x;
    float m = -__builtin_huge_valf();
    uint32_t bad = 0;
    for (uint32_t p = 0; p < gridDim.x; ++p) {
        const float v = part_value[base + p];
        m = v > m ? v : m;
        bad |= part_index[base + p] == 0xFFFFFFFFu ? 1u : 0u;
    }
    if (bad != 0u) {
        if (threadIdx.x == 0) {
            part_sum[base + blockIdx.x] = 0.0;
        }
        return;
    }
    const double maximum = static_cast<double>(m);
    const double t = static_cast<double>(temperature);
    const uint32_t begin = blockIdx.x * span;
    const uint32_t end = begin + span < count ? begin + span : count;
    const float *row = logits + static_cast<size_t>(blockIdx.y) * count + begin;
    if (top != nullptr) {
        for (uint32_t b = threadIdx.x; b < kTopBins; b += blockDim.x) {
            bin_count[b] = 0u;
            bin_mass[b] = 0.0f;
        }
        __syncthreads();
    }
    double part = 0.0;
    for_each_logit(row, end - begin, [&](uint32_t, float v) {
        const double p = exp((static_cast<double>(v) - maximum) / t);
        part += p;
        if (top != nullptr) {
            const uint32_t bin = descending_key(v) >> kTopShift;
            atomicAdd(&bin_count[bin], 1u);
            atomicAdd(&bin_mass[bin], static_cast<float>(p));
        }
    });
    if (top != nullptr) {
        __syncthreads();
        uint32_t *counts = top + static_cast<size_t>(blockIdx.y) * kTopRowWords;
        float *masses = reinterpret_cast<float *>(counts + kTopBins);
        for (uint32_t b = threadIdx.x; b < kTopBins; b += blockDim.x) {
            if (bin_count[b] != 0u) {
                atomicAdd(&counts[b], bin_count[b]);
                atomicAdd(&masses[b], bin_mass[b]);
            }
        }
    }
#pragma unroll
    for (int offset = 32; offset > 0; offset >>= 1) {
        part += __shfl_xor(part, offset);
    }
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    if (lane == 0) {
        wave_sum[wave] = part;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        double sum = 0.0;
        for (uint32_t w = 0; w < kArgmaxPartThreads / kWave; ++w) {
            sum += wave_sum[w];
        }
        part_sum[base + blockIdx.x] = sum;
    }
}

// The block's state between the phases of a row (in LDS).
struct SampleState {
    uint64_t floor;     // (key << 32 | index) of the last walked candidate
    uint32_t has_floor;
    uint32_t count;     // candidates in the window
    uint32_t select;    // radix select: chosen prefix
    uint32_t want;      // rank still wanted within the prefix
    uint32_t all;       // fewer than kWindow eligible: take them all
    uint32_t ties;      // eligible candidates with the selected key
    uint32_t done;
    uint32_t token;
    double walk[2];     // running sums carried across windows
};

__device__ __forceinline__ bool eligible(const SampleState &s, uint32_t key, uint32_t index) {
    const uint64_t packed = (static_cast<uint64_t>(key) << 32) | index;
    return s.has_floor == 0u || packed > s.floor;
}

// Radix select over 32-bit values v(i) of the eligible tokens passing
// `filter`: the value of the s.want-th smallest (MSB first, 8 bits a pass),
// with s.want left as the rank within it; s.all when fewer are eligible.
template <typename Value, typename Filter>
__device__ void radix_select(const float *row, uint32_t count, SampleState &s, uint32_t *hist,
                             Value value, Filter filter) {
    uint32_t prefix = 0, mask = 0;
    for (int shift = 24; shift >= 0; shift -= 8) {
        for (uint32_t b = threadIdx.x; b < 256u; b += blockDim.x) {
            hist[b] = 0u;
        }
        __syncthreads();
        for_each_logit(row, count, [&](uint32_t i, float logit) {
            const uint32_t key = descending_key(logit);
            const uint32_t v = value(key, i);
            if (eligible(s, key, i) && filter(key, i) && (v & mask) == prefix) {
                atomicAdd(&hist[(v >> shift) & 0xFFu], 1u);
            }
        });
        __syncthreads();
        if (threadIdx.x == 0) {
            uint32_t b = 0, w = s.want;
            while (b < 256u && w > hist[b]) {
                w -= hist[b];
                ++b;
            }
            if (b == 256u) {
                s.all = 1u;
            } else {
                s.select = prefix | (b << shift);
                s.want = w;
                s.ties = hist[b];
            }
        }
        __syncthreads();
        if (s.all != 0u) {
            return;
        }
        prefix = s.select;
        mask |= 0xFFu << shift;
    }
}

// The next kWindow tokens after s.floor in (key, index) order, sorted into
// cand, with their p in prob.
__device__ void gather_window(const float *row, uint32_t count, double maximum, double temperature,
                              SampleState &s, uint64_t *cand, double *prob, uint32_t *hist) {
    if (threadIdx.x == 0) {
        s.want = kWindow;
        s.all = 0u;
        s.count = 0u;
    }
    __syncthreads();
    radix_select(row, count, s, hist, [](uint32_t key, uint32_t) { return key; },
                 [](uint32_t, uint32_t) { return true; });
    const uint32_t take_all = s.all;
    const uint32_t key_th = s.select;
    uint32_t index_th = 0xFFFFFFFFu;
    if (take_all == 0u && s.ties != s.want) {
        // only the first `want` of the tokens tied at key_th, by index
        radix_select(row, count, s, hist, [](uint32_t, uint32_t i) { return i; },
                     [key_th](uint32_t key, uint32_t) { return key == key_th; });
        index_th = s.select;
    }
    __syncthreads();
    for_each_logit(row, count, [&](uint32_t i, float logit) {
        const uint32_t key = descending_key(logit);
        if (eligible(s, key, i) &&
            (take_all != 0u || key < key_th || (key == key_th && i <= index_th))) {
            const uint32_t at = atomicAdd(&s.count, 1u);
            if (at < kWindow) {  // the select admits exactly min(kWindow, eligible)
                cand[at] = (static_cast<uint64_t>(key) << 32) | i;
            }
        }
    });
    __syncthreads();
    const uint32_t n = s.count < kWindow ? s.count : kWindow;
    for (uint32_t k = n + threadIdx.x; k < kWindow; k += blockDim.x) {
        cand[k] = ~0ull;
    }
    // bitonic sort, ascending
    for (uint32_t size = 2; size <= kWindow; size <<= 1) {
        for (uint32_t stride = size >> 1; stride > 0; stride >>= 1) {
            __syncthreads();
            for (uint32_t i = threadIdx.x; i < kWindow; i += blockDim.x) {
                const uint32_t j = i ^ stride;
                if (j > i) {
                    const uint64_t a = cand[i], b = cand[j];
                    const bool up = (i & size) == 0u;
                    if ((a > b) == up) {
                        cand[i] = b;
                        cand[j] = a;
                    }
                }
            }
        }
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        s.count = n;
    }
    for (uint32_t k = threadIdx.x; k < n; k += blockDim.x) {
        const float logit = row[static_cast<uint32_t>(cand[k])];
        prob[k] = exp((static_cast<double>(logit) - maximum) / temperature);
    }
    __syncthreads();
}

// One block per row (src/generation.cpp:161-225): the maximum, the sum of p
// over all tokens (a fixed tree order), then windows of the sorted order
// walked on one thread exactly as the reference walks its sorted vector:
// first the cumulative p / sum up to top_p (summing the kept p on the way),
// then the running p up to the target.
__global__ __launch_bounds__(kSampleThreads) void k_sample_rows(const float *logits, uint32_t count,
                                                                float temperature, float top_p,
                                                                const uint64_t *words,
                                                                uint32_t *tokens, uint32_t parts,
                                                                const float *part_value,
                                                                const uint32_t *part_index,
                                                                const double *part_sum,
                                                                const uint32_t *top) {
    if (top != nullptr && top[static_cast<size_t>(blockIdx.x) * kTopRowWords + kTopState + 2] != 0u) {
        return;  // the short walk chose this row's token
    }
    __shared__ uint64_t cand[kWindow];
    __shared__ double prob[kWindow];
    __shared__ uint32_t hist[256];
    __shared__ double wave_sum[kSampleWaves];
    __shared__ float wave_max[kSampleWaves];
    __shared__ uint32_t wave_bad[kSampleWaves];
    __shared__ SampleState s;
    const float *row = logits + static_cast<size_t>(blockIdx.x) * count;
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    // the maximum; any non-finite logit rejects the row
    float m = -__builtin_huge_valf();
    uint32_t bad = 0;
    if (parts != 0u) {
        // split rows: the spans' maxima and flags, read by every thread
        const size_t base = static_cast<size_t>(blockIdx.x) * parts;
        for (uint32_t p = 0; p < parts; ++p) {
            const float v = part_value[base + p];
            m = v > m ? v : m;
            bad |= part_index[base + p] == 0xFFFFFFFFu ? 1u : 0u;
        }
    } else {
        for_each_logit(row, count, [&](uint32_t, float v) {
            bad |= __builtin_isfinite(v) ? 0u : 1u;
            m = v > m ? v : m;
        });
    }
#pragma unroll
    for (int offset = 32; offset > 0; offset >>= 1) {
        const float o = __shfl_xor(m, offset);
        m = o > m ? o : m;
        bad |= static_cast<uint32_t>(__shfl_xor(static_cast<int>(bad), offset));
    }
    if (lane == 0) {
        wave_max[wave] = m;
        wave_bad[wave] = bad;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (uint32_t w = 1; w < kSampleWaves; ++w) {
            m = wave_max[w] > m ? wave_max[w] : m;
            bad |= wave_bad[w];
        }
        wave_max[0] = m;
        s.done = bad;
        s.has_floor = 0u;
        s.walk[0] = 0.0;
        s.walk[1] = 0.0;
    }
    __syncthreads();
    if (s.done != 0u) {
        if (threadIdx.x == 0) {
            tokens[blockIdx.x] = 0xFFFFFFFFu;
        }
        return;
    }
    const double maximum = static_cast<double>(wave_max[0]);
    const double t = static_cast<double>(temperature);
    // sum of p over the row: each thread in index order, then a fixed tree
    // (split rows: the spans' sums in span order)
    double denominator = 0.0;
    if (parts != 0u) {
        const size_t base = static_cast<size_t>(blockIdx.x) * parts;
        for (uint32_t p = 0; p < parts; ++p) {
            denominator += part_sum[base + p];
        }
    } else {
        double part = 0.0;
        for_each_logit(row, count, [&](uint32_t, float v) {
            part += exp((static_cast<double>(v) - maximum) / t);
        });
#pragma unroll
        for (int offset = 32; offset > 0; offset >>= 1) {
            part += __shfl_xor(part, offset);
        }
        if (lane == 0) {
            wave_sum[wave] = part;
        }
        __syncthreads();
        for (uint32_t w = 0; w < kSampleWaves; ++w) {
            denominator += wave_sum[w];
        }
    }
    // phase 1: the kept prefix and the sum of its p
    uint64_t last = 0;
    uint32_t window = 0;
    while (true) {
        gather_window(row, count, maximum, t, s, cand, prob, hist);
        if (threadIdx.x == 0) {
            double cumulative = s.walk[0], kept = s.walk[1];
            const uint32_t n = s.count;
            uint32_t k = 0;
            for (; k < n; ++k) {
                cumulative += prob[k] / denominator;
                kept += prob[k];
                if (cumulative >= static_cast<double>(top_p)) {
                    break;
                }
            }
            s.walk[0] = cumulative;
            s.walk[1] = kept;
            if (k < n || n < kWindow) {
                // crossed, or every token is walked: the kept set ends here
                // (an empty window leaves the previous window's last token)
                s.done = 1u;
                if (n > 0) {
                    s.floor = cand[k < n ? k : n - 1];
                }
            } else {
                s.floor = cand[n - 1];
                s.has_floor = 1u;
            }
        }
        __syncthreads();
        if (s.done != 0u) {
            break;
        }
        ++window;
    }
    last = s.floor;  // the last kept token
    // the draw (std::uniform_real_distribution<double>(0, kept) over
    // generate_canonical<double, 53> of a 64-bit engine)
    double u = static_cast<double>(words[blockIdx.x]) * 0x1p-64;
    if (u >= 1.0) {
        u = 0x1.fffffffffffffp-1;
    }
    const double target = u * s.walk[1];
    // phase 2: the running p from the first token until it reaches target
    __syncthreads();
    if (threadIdx.x == 0) {
        s.done = 0u;
        s.walk[0] = 0.0;
        s.token = static_cast<uint32_t>(last);
    }
    __syncthreads();
    uint32_t current = window;  // the window in LDS
    if (current != 0u) {
        if (threadIdx.x == 0) {
            s.has_floor = 0u;
        }
        __syncthreads();
    }
    while (true) {
        if (current != 0u) {
            gather_window(row, count, maximum, t, s, cand, prob, hist);
        }
        current = 1u;  // later windows are gathered after the floor
        if (threadIdx.x == 0) {
            double running = s.walk[0];
            const uint32_t n = s.count;
            for (uint32_t k = 0; k < n && s.done == 0u; ++k) {
                running += prob[k];
                if (target <= running) {
                    s.done = 1u;
                    s.token = static_cast<uint32_t>(cand[k]);
                } else if (cand[k] == last) {
                    s.done = 1u;  // past the kept set: the last kept token
                }
            }
            s.walk[0] = running;
            if (s.done == 0u && n == 0u) {
                s.done = 1u;  // not reached: the last kept token stands
            } else if (s.done == 0u) {
                s.floor = cand[n - 1];
                s.has_floor = 1u;
            }
        }
        __syncthreads();
        if (s.done != 0u) {
            break;
        }
    }
    if (threadIdx.x == 0) {
        tokens[blockIdx.x] = s.token;
    }
}

// The short walk of a long row, first step: the prefix of the sorted order
// (ascending key: descending logit, then ascending index) up to the first
// bin whose inclusive mass reaches top_p of the row's sum, by a 0.1% margin
// over the bins' float masses, when it holds at most kWindow tokens. Every
// block (p, r) finds the same cut from the row's bins and appends its span's
// tokens before it; block (0, r) records how many the prefix holds. A row
// with a non-finite logit, or whose cut is out of reach, is left to the
// full sampler.
__global__ __launch_bounds__(kArgmaxPartThreads) void k_top_collect(const float *logits, uint32_t count,
                                                                    uint32_t span, const uint32_t *part_index,
                                                                    const double *part_sum, float top_p,
                                                                    uint32_t *top) {
    constexpr uint32_t kPer = kTopBins / kArgmaxPartThreads;
    __shared__ uint32_t scan_count[kArgmaxPartThreads];
    __shared__ double scan_mass[kArgmaxPartThreads];
    __shared__ uint32_t cut, cut_count;
    const uint32_t t = threadIdx.x;
    const size_t base = static_cast<size_t>(blockIdx.y) * gridDim.x;
    uint32_t bad = 0;
    double denominator = 0.0;
    for (uint32_t p = 0; p < gridDim.x; ++p) {
        bad |= part_index[base + p] == 0xFFFFFFFFu ? 1u : 0u;
        denominator += part_sum[base + p];
    }
    if (bad != 0u) {
        return;
    }
    uint32_t *words = top + static_cast<size_t>(blockIdx.y) * kTopRowWords;
    const float *masses = reinterpret_cast<const float *>(words + kTopBins);
    uint32_t c[kPer], own_count = 0;
    double mass[kPer], own_mass = 0.0;
#pragma unroll
    for (uint32_t j = 0; j < kPer; ++j) {
        c[j] = words[kPer * t + j];
        mass[j] = static_cast<double>(masses[kPer * t + j]);
        own_count += c[j];
        own_mass += mass[j];
    }
    scan_count[t] = own_count;
    scan_mass[t] = own_mass;
    if (t == 0) {
        cut = 0xFFFFFFFFu;
    }
    __syncthreads();
    for (uint32_t d = 1; d < kArgmaxPartThreads; d <<= 1) {
        const uint32_t a = t >= d ? scan_count[t - d] : 0u;
        const double m = t >= d ? scan_mass[t - d] : 0.0;
        __syncthreads();
        scan_count[t] += a;
        scan_mass[t] += m;
        __syncthreads();
    }
    const double target = static_cast<double>(top_p) * denominator * 1.001;
    double reached = scan_mass[t] - own_mass;
    for (uint32_t j = 0; j < kPer; ++j) {
        reached += mass[j];
        if (reached >= target) {
            atomicMin(&cut, kPer * t + j);
            break;
        }
    }
    __syncthreads();
    const uint32_t b_cut = cut;
    if (b_cut / kPer == t) {
        uint32_t inclusive = scan_count[t] - own_count;
        for (uint32_t j = 0; j <= b_cut % kPer; ++j) {
            inclusive += c[j];
        }
        cut_count = inclusive;
    }
    __syncthreads();
    if (b_cut == 0xFFFFFFFFu || cut_count > kWindow) {
        return;
    }
    if (blockIdx.x == 0 && t == 0) {
        words[kTopState + 1] = cut_count;
    }
    uint64_t *cand = reinterpret_cast<uint64_t *>(words + kTopCand);
    const uint32_t begin = blockIdx.x * span;
    const uint32_t end = begin + span < count ? begin + span : count;
    const float *row = logits + static_cast<size_t>(blockIdx.y) * count + begin;
    for_each_logit(row, end - begin, [&](uint32_t i, float v) {
        const uint32_t key = descending_key(v);
        if ((key >> kTopShift) <= b_cut) {
            const uint32_t at = atomicAdd(&words[kTopState], 1u);
            cand[at] = (static_cast<uint64_t>(key) << 32) | (begin + i);
        }
    });
}

// The short walk, second step (one block per row, src/generation.cpp:
// 184-225): the prefix sorted, its p, and the reference's two walks over it
// on one thread, as k_sample_rows walks its first window. When the kept set
// ends inside the prefix the row's token is chosen here; otherwise the row
// is left to the full sampler.
__global__ __launch_bounds__(kArgmaxPartThreads) void k_top_walk(const float *logits, uint32_t count,
                                                                 float temperature, float top_p,
                                                                 const uint64_t *words, uint32_t *tokens,
                                                                 uint32_t parts, const float *part_value,
                                                                 const double *part_sum, uint32_t *top) {
    __shared__ uint64_t cand[kWindow];
    __shared__ double prob[kWindow];
    uint32_t *state = top + static_cast<size_t>(blockIdx.x) * kTopRowWords;
    const uint32_t n = state[kTopState + 1];
    if (n == 0u) {
        return;
    }
    const float *row = logits + static_cast<size_t>(blockIdx.x) * count;
    const size_t base = static_cast<size_t>(blockIdx.x) * parts;
    float m = -__builtin_huge_valf();
    double denominator = 0.0;
    for (uint32_t p = 0; p < parts; ++p) {
        const float v = part_value[base + p];
        m = v > m ? v : m;
        denominator += part_sum[base + p];
    }
    const double maximum = static_cast<double>(m);
    const double t = static_cast<double>(temperature);
    uint32_t size = 1;
    while (size < n) {
        size <<= 1;
    }
    const uint64_t *src = reinterpret_cast<const uint64_t *>(state + kTopCand);
    for (uint32_t k = threadIdx.x; k < size; k += blockDim.x) {
        cand[k] = k < n ? src[k] : ~0ull;
    }
    // bitonic sort, ascending
    for (uint32_t width = 2; width <= size; width <<= 1) {
        for (uint32_t stride = width >> 1; stride > 0; stride >>= 1) {
            __syncthreads();
            for (uint32_t i = threadIdx.x; i < size; i += blockDim.x) {
                const uint32_t j = i ^ stride;
                if (j > i) {
                    const uint64_t a = cand[i], b = cand[j];
                    const bool up = (i & width) == 0u;
                    if ((a > b) == up) {
                        cand[i] = b;
                        cand[j] = a;
                    }
                }
            }
        }
    }
    __syncthreads();
    for (uint32_t k = threadIdx.x; k < n; k += blockDim.x) {
        const float logit = row[static_cast<uint32_t>(cand[k])];
        prob[k] = exp((static_cast<double>(logit) - maximum) / t);
    }
    __syncthreads();
    if (threadIdx.x != 0) {
        return;
    }
    // phase 1: the kept prefix and the sum of its p
    double cumulative = 0.0, kept = 0.0;
    uint32_t k = 0;
    for (; k < n; ++k) {
        cumulative += prob[k] / denominator;
        kept += prob[k];
        if (cumulative >= static_cast<double>(top_p)) {
            break;
        }
    }
    if (k == n) {
        return;  // the kept set reaches past the prefix
    }
    const uint64_t last = cand[k];
    // the draw, as k_sample_rows takes it
    double u = static_cast<double>(words[blockIdx.x]) * 0x1p-64;
    if (u >= 1.0) {
        u = 0x1.fffffffffffffp-1;
    }
    const double target = u * kept;
    // phase 2: the running p from the first token until it reaches target
    double running = 0.0;
    uint32_t token = static_cast<uint32_t>(last);
    for (uint32_t j = 0; j <= k; ++j) {
        running += prob[j];
        if (target <= running) {
            token = static_cast<uint32_t>(cand[j]);
            break;
        }
        if (cand[j] == last) {
            break;
        }
    }
    tokens[blockIdx.x] = token;
    state[kTopState + 2] = 1u;
}

}  // namespace
}  // namespace adi_hip

using namespace adi_hip;

extern "C" {

int adi_hip_embedding_rows(adi_hip_context *ctx, const adi_hip_embedding *e,
                           const uint32_t *tokens, uint32_t count, float *outputs) {
    return guarded(ctx, [&] {
        require(e != nullptr, "Mach embedding is null");
        require(e->rows > 0 && e->columns > 0 && e->columns % 64 == 0 &&
                    static_cast<uint64_t>(e->rows) * e->columns <= 0xFFFFFFFFull,
                "Mach embedding shape mismatch");
        require(e->packed != nullptr && e->minimum_f16 != nullptr && e->maximum_f16 != nullptr &&
                    (e->exception_count == 0 ||
                     (e->exception_indexes != nullptr && e->exception_bf16 != nullptr)),
                "Mach embedding scale or exception shape mismatch");
        require(count == 0 || (tokens != nullptr && outputs != nullptr),
                "Mach embedding vector is null");
        require(aligned_to(e->packed, 4) && aligned_to(outputs, 16),
                "embedding codes must be 4-byte and outputs 16-byte aligned");
        if (count == 0) {
            return;
        }
        launch(ctx, "embedding", k_embedding_rows, dim3(count), dim3(kEmbeddingThreads), 0, *e,
               tokens, outputs);
    });
}

int adi_hip_argmax_rows(adi_hip_context *ctx, const float *logits, uint32_t rows,
                        uint32_t count, uint32_t *tokens) {
    return guarded(ctx, [&] {
        require(count > 0, "invalid sampling parameters");
        require(rows == 0 || (logits != nullptr && tokens != nullptr), "sampling vector is null");
        if (rows == 0) {
            return;
        }
        launch_argmax(ctx, logits, rows, count, tokens);
    });
}

int adi_hip_sample_rows(adi_hip_context *ctx, const float *logits, uint32_t rows,
                        uint32_t count, float temperature, float top_p,
                        const uint64_t *words, uint32_t *tokens) {
    return guarded(ctx, [&] {
        // the reference's parameter checks (src/generation.cpp:167-176)
        require(count > 0 && std::isfinite(temperature) && std::isfinite(top_p) &&
                    temperature >= 0.0f && !(temperature > 0.0f && temperature < 1.0e-4f) &&
                    temperature <= 2.0f && top_p > 0.0f && top_p <= 1.0f,
                "invalid sampling parameters");
        require(rows == 0 || (logits != nullptr && tokens != nullptr), "sampling vector is null");
        require(temperature == 0.0f || rows == 0 || words != nullptr,
                "sampling needs one random word per row");
        if (rows == 0) {
            return;
        }
        if (temperature == 0.0f) {
            launch_argmax(ctx, logits, rows, count, tokens);
            return;
        }
        if (count < kArgmaxSplitCount || rows > 65535u) {
            launch(ctx, "sample", k_sample_rows, dim3(rows), dim3(kSampleThreads), 0, logits,
                   count, temperature, top_p, words, tokens, 0u,
                   static_cast<const float *>(nullptr), static_cast<const uint32_t *>(nullptr),
                   static_cast<const double *>(nullptr), static_cast<const uint32_t *>(nullptr));
            return;
        }
        // long rows: the maximum and the denominator over up to 64 blocks a row
        const uint32_t wanted = std::min<uint32_t>(kArgmaxMaxParts, ceil_div(count, 4096));
        const uint32_t span = (ceil_div(count, wanted) + 3u) & ~3u;
        const uint32_t parts = ceil_div(count, span);
        auto &ws = ctx->workspace;
        ws.used = 0;
        ws.ensure(Workspace::round(size_t(rows) * parts * 4) * 2 +
                  Workspace::round(size_t(rows) * parts * 8) + Workspace::round(size_t(rows) * kTopRowWords * 4));
        float *part_value = ws.take<float>(size_t(rows) * parts);
        uint32_t *part_index = ws.take<uint32_t>(size_t(rows) * parts);
        double *part_sum = ws.take<double>(size_t(rows) * parts);
        uint32_t *top = ws.take<uint32_t>(size_t(rows) * kTopRowWords);
        launch(ctx, "argmax_parts", k_argmax_parts, dim3(parts, rows), dim3(kArgmaxPartThreads), 0,
               logits, count, span, part_value, part_index, top, kTopZeroWords, kTopRowWords);
        launch(ctx, "expsum_parts", k_expsum_parts, dim3(parts, rows), dim3(kArgmaxPartThreads), 0,
               logits, count, span, static_cast<const float *>(part_value),
               static_cast<const uint32_t *>(part_index), temperature, part_sum, top);
        // the short walk: the kept set of most rows ends in a short prefix of
        // the sorted order; the full sampler then only runs for the rest
        launch(ctx, "top_collect", k_top_collect, dim3(parts, rows), dim3(kArgmaxPartThreads), 0, logits,
               count, span, static_cast<const uint32_t *>(part_index), static_cast<const double *>(part_sum),
               top_p, top);
        launch(ctx, "top_walk", k_top_walk, dim3(rows), dim3(kArgmaxPartThreads), 0, logits, count, temperature,
               top_p, words, tokens, parts, static_cast<const float *>(part_value),
               static_cast<const double *>(part_sum), top);
        launch(ctx, "sample", k_sample_rows, dim3(rows), dim3(kSampleThreads), 0, logits, count,
               temperature, top_p, words, tokens, parts, static_cast<const float *>(part_value),
               static_cast<const uint32_t *>(part_index), static_cast<const double *>(part_sum),
               static_cast<const uint32_t *>(top));
    });
}

}  // extern "C"
