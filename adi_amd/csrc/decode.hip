// decode.hip -- the token side of a decode step on the device: embedding rows
// (mach_embedding_row, src/kernels.cpp:802-845) and the greedy choice of
// sample_token (src/generation.cpp:161-183), so a step's token goes from the
// head's logits to the next step's hidden state without leaving HBM.
#include "context.hpp"

#include <cmath>

namespace adi_hip {
namespace {

constexpr uint32_t kEmbeddingThreads = 256;
constexpr uint32_t kArgmaxThreads = 256;

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

// One block per row: each thread scans a strided share, then wave and block
// reductions of (value, index); any non-finite logit marks the row.
__global__ __launch_bounds__(kArgmaxThreads) void k_argmax_rows(const float *logits,
                                                                uint32_t count,
                                                                uint32_t *tokens) {
    __shared__ float wave_value[kArgmaxThreads / kWave];
    __shared__ uint32_t wave_index[kArgmaxThreads / kWave];
    __shared__ uint32_t wave_bad[kArgmaxThreads / kWave];
    const float *row = logits + static_cast<size_t>(blockIdx.x) * count;
    float value = -__builtin_huge_valf();
    uint32_t index = 0xFFFFFFFFu;
    uint32_t bad = 0;
    for (uint32_t i = threadIdx.x; i < count; i += blockDim.x) {
        const float v = row[i];
        bad |= __builtin_isfinite(v) ? 0u : 1u;
        better(value, index, v, i);
    }
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
        tokens[blockIdx.x] = bad != 0u ? 0xFFFFFFFFu : index;
    }
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
        launch(ctx, "argmax", k_argmax_rows, dim3(rows), dim3(kArgmaxThreads), 0, logits, count,
               tokens);
    });
}

}  // extern "C"
