// common.hpp -- shared host/device definitions of the gfx950 hot path.
#pragma once

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstring>
#include <string>
#include <vector>

#include "adi_hip.h"

namespace adi_hip {

constexpr uint32_t kTile = 16;
constexpr uint32_t kExpertWords = 24;  // 384-bit stream per expert tile
constexpr uint32_t kNeWords = 64;      // 1024-bit stream per NE tile
constexpr uint32_t kExpertRows = 16384; // reachable expert codebook rows
constexpr uint32_t kWave = 64;

// A failed precondition: the message becomes adi_hip_last_error().
struct Failure {
    int status;
    std::string message;
};

[[noreturn]] inline void fail(int status, std::string message) {
    throw Failure{status, std::move(message)};
}

inline void require(bool condition, const char *message) {
    if (!condition) {
        fail(ADI_HIP_INVALID_ARGUMENT, message);
    }
}

inline void check_hip(hipError_t error, const char *what) {
    if (error != hipSuccess) {
        fail(error == hipErrorOutOfMemory ? ADI_HIP_OUT_OF_MEMORY : ADI_HIP_DEVICE_ERROR,
             std::string(what) + ": " + hipGetErrorString(error));
    }
}

inline bool is_power_of_two(uint32_t v) { return v != 0 && (v & (v - 1)) == 0; }

// 1/sqrt(n) exactly as the reference computes it on the host
// (src/simd.cpp:59): a correctly rounded sqrt and a correctly rounded divide.
inline float hadamard_scale(uint32_t n) {
    return 1.0f / std::sqrt(static_cast<float>(n));
}

// ---- device helpers -------------------------------------------------------

// f16 bits -> f32 (exact for every value; the tables and scale surfaces are
// validated finite by the loader).
__device__ __forceinline__ float half_bits_to_float(uint32_t bits) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(bits)));
}

// Both f16 halves of a dword as f32: (low, high).
__device__ __forceinline__ float2 half2_bits_to_float2(uint32_t bits) {
    return make_float2(half_bits_to_float(bits & 0xFFFFu), half_bits_to_float(bits >> 16));
}

__device__ __forceinline__ float bf16_bits_to_float(uint32_t bits) {
    return __uint_as_float(bits << 16);
}

// u16 word k of a stream held as little-endian dwords (word 2j = low half).
template <int K, int N>
__device__ __forceinline__ uint32_t stream_word(const uint32_t (&d)[N]) {
    return (K & 1) ? (d[K >> 1] >> 16) : (d[K >> 1] & 0xFFFFu);
}

// The 16-bit window at bit B of a local stream whose u16 words are read
// most-significant bit first (src/expert_trellis.hpp:81-105,
// src/ne_trellis.hpp:177-204).
template <int B, int N>
__device__ __forceinline__ uint32_t stream_window(const uint32_t (&d)[N]) {
    constexpr int w = B / 16;
    constexpr int o = B % 16;
    if constexpr (o == 0) {
        return stream_word<w>(d);
    } else {
        const uint32_t pair = (stream_word<w>(d) << 16) | stream_word<w + 1>(d);
        return (pair >> (16 - o)) & 0xFFFFu;
    }
}

// Expert state hash (src/codec_cache.cpp:17-25): p = s(s+1) mod 2^16. The
// TLUT row is p & 0x7FFF, which is always even, so the 16384 reachable rows
// are indexed by (p >> 1) & 0x3FFF; bit 15 negates component 0.
__device__ __forceinline__ uint32_t state_product(uint32_t s) {
    return __umul24(s, s + 1u) & 0xFFFFu;
}

// Wave-gamma slot of tile (tr, tc) in an R_t x C_t grid: the closed form of
// build_wave_indexes (src/codec_cache.cpp:117-147). Slot R_t-1 is never used.
__device__ __forceinline__ uint32_t wave_slot(uint32_t tr, uint32_t tc,
                                              uint32_t tile_rows,
                                              uint32_t tile_columns) {
    const uint32_t d = tr + tc;
    return d <= tile_columns - 1 ? tile_rows + tile_columns - 1 - d
                                 : tile_rows + tile_columns - 2 - d;
}

// In-place normalised FWHT of n values in LDS by `threads` threads, the
// butterflies applied with strides 1, 2, 4, ... exactly as the reference's
// scalar loop (src/simd.cpp:48-63), so every element sees the same sequence of
// additions and the result is bit-identical. Ends with a barrier.
__device__ __forceinline__ void block_hadamard(float *v, uint32_t n, float scale) {
#pragma clang fp contract(off)
    const uint32_t half = n >> 1;
    for (uint32_t stride = 1; stride < n; stride <<= 1) {
        __syncthreads();
        for (uint32_t k = threadIdx.x; k < half; k += blockDim.x) {
            const uint32_t lo = ((k & ~(stride - 1)) << 1) | (k & (stride - 1));
            const float a = v[lo];
            const float b = v[lo + stride];
            v[lo] = a + b;
            v[lo + stride] = a - b;
        }
    }
    __syncthreads();
    for (uint32_t k = threadIdx.x; k < n; k += blockDim.x) {
        v[k] = v[k] * scale;
    }
    __syncthreads();
}

// Value of lane (lane ^ MASK) for MASK < 32, without the LDS crossbar for
// masks 1, 2, 4 and 8 (DPP: quad permutes, half-row mirror, row rotate by 8;
// every pattern used is its own inverse, so the DPP shift direction does not
// matter) and with a swizzle for 16.
template <int MASK>
__device__ __forceinline__ float lane_xor(float v) {
    const int bits = __float_as_int(v);
    if constexpr (MASK == 1) {
        return __int_as_float(__builtin_amdgcn_mov_dpp(bits, 0xB1, 0xF, 0xF, true));
    } else if constexpr (MASK == 2) {
        return __int_as_float(__builtin_amdgcn_mov_dpp(bits, 0x4E, 0xF, 0xF, true));
    } else if constexpr (MASK == 4) {
        // lane i of a half-row takes lane 7-i after a [3,2,1,0] quad permute
        const int q = __builtin_amdgcn_mov_dpp(bits, 0x1B, 0xF, 0xF, true);
        return __int_as_float(__builtin_amdgcn_mov_dpp(q, 0x141, 0xF, 0xF, true));
    } else if constexpr (MASK == 8) {
        return __int_as_float(__builtin_amdgcn_mov_dpp(bits, 0x128, 0xF, 0xF, true));
    } else if constexpr (MASK == 16) {
        // bitmask swizzle: and 0x1F, or 0, xor 0x10 within 32 lanes
        return __int_as_float(__builtin_amdgcn_ds_swizzle(bits, 0x401F));
    } else {
        return __shfl_xor(v, MASK);
    }
}

// Normalised FWHT of n = 64*VPL values held by one wave, element e in lane
// e % 64, register e / 64 (consecutive lanes hold consecutive elements, so
// loads and stores coalesce and LDS staging is conflict-free). Strides 1..32
// pair lanes l and l ^ stride; strides 64, 128, ... pair registers. Strides
// run 1, 2, 4, ... and each pair becomes (lo + hi, lo - hi): the reference's
// exact sequence (src/simd.cpp:48-63), so the result is bit-identical to it.
// Every lane of the wave must call this.
template <int VPL>
__device__ __forceinline__ void wave_hadamard(float (&v)[VPL], float scale, uint32_t lane) {
#pragma clang fp contract(off)
    // All exchanges of a stage are issued before any is consumed so the
    // LDS-routed ones (masks 16 and 32) pipeline instead of waiting in turn.
#define ADI_XOR_STAGE(MASK)                                              \
    {                                                                    \
        const bool upper = (lane & static_cast<uint32_t>(MASK)) != 0;    \
        float other[VPL];                                                \
        _Pragma("unroll") for (int i = 0; i < VPL; ++i) {                \
            other[i] = lane_xor<MASK>(v[i]);                             \
        }                                                                \
        _Pragma("unroll") for (int i = 0; i < VPL; ++i) {                \
            v[i] = upper ? other[i] - v[i] : v[i] + other[i];            \
        }                                                                \
    }
    ADI_XOR_STAGE(1) ADI_XOR_STAGE(2) ADI_XOR_STAGE(4) ADI_XOR_STAGE(8)
    ADI_XOR_STAGE(16) ADI_XOR_STAGE(32)
#undef ADI_XOR_STAGE
#pragma unroll
    for (int stride = 1; stride < VPL; stride <<= 1) {
#pragma unroll
        for (int i = 0; i < VPL; ++i) {
            if ((i & stride) == 0) {
                const float a = v[i];
                const float b = v[i + stride];
                v[i] = a + b;
                v[i + stride] = a - b;
            }
        }
    }
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
        v[i] = v[i] * scale;
    }
}

}  // namespace adi_hip
