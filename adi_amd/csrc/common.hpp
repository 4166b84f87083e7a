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

// log2 of a power of two.
inline uint32_t log2_of(uint32_t v) {
    uint32_t s = 0;
    while ((1u << s) < v) {
        ++s;
    }
    return s;
}

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

// Value of lane (lane ^ MASK) for MASK in {1, 2, 4, 8, 16, 32}, without the
// LDS crossbar: DPP quad permutes, half-row mirror and row rotate by 8 for
// masks up to 8 (every pattern used is its own inverse, so the DPP shift
// direction does not matter), and gfx950's row swaps for 16 and 32.
template <int MASK>
__device__ __forceinline__ uint32_t lane_xor_bits(uint32_t v) {
    const int bits = static_cast<int>(v);
    if constexpr (MASK == 1) {
        return static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(bits, 0xB1, 0xF, 0xF, true));
    } else if constexpr (MASK == 2) {
        return static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(bits, 0x4E, 0xF, 0xF, true));
    } else if constexpr (MASK == 4) {
        // lane i of a half-row takes lane 7-i after a [3,2,1,0] quad permute
        const int q = __builtin_amdgcn_mov_dpp(bits, 0x1B, 0xF, 0xF, true);
        return static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(q, 0x141, 0xF, 0xF, true));
    } else if constexpr (MASK == 8) {
        return static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(bits, 0x128, 0xF, 0xF, true));
    } else if constexpr (MASK == 16) {
        // v_permlane16_swap(v, v): the first result holds each even 16-lane
        // row twice, the second each odd row twice
        const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
        return (__lane_id() & 16u) ? r[0] : r[1];
    } else {
        static_assert(MASK == 32, "lane_xor: unsupported mask");
        // v_permlane32_swap(v, v): the first result holds lanes 0-31 twice,
        // the second lanes 32-63 twice
        const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
        return (__lane_id() & 32u) ? r[0] : r[1];
    }
}

template <int MASK>
__device__ __forceinline__ float lane_xor(float v) {
    return __uint_as_float(lane_xor_bits<MASK>(__float_as_uint(v)));
}

// Value of the next lane of the lane's quad (lane 3 of a quad reads lane 0):
// a DPP quad permute [1, 2, 3, 0].
__device__ __forceinline__ uint32_t quad_next(uint32_t v) {
    return static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(v), 0x39, 0xF, 0xF, true));
}

// Sums v over the lanes that differ only in lane bits 2.. of `span` (a power
// of two up to 16): the four lanes of a quad position across `span` quads.
__device__ __forceinline__ float sum_over_quads(float v, uint32_t span) {
    if (span > 1) {
        v += lane_xor<4>(v);
    }
    if (span > 2) {
        v += lane_xor<8>(v);
    }
    if (span > 4) {
        v += lane_xor<16>(v);
    }
    if (span > 8) {
        v += lane_xor<32>(v);
    }
    return v;
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

// v[i] = sum over slices s < splits of src[s * stride + i * 64 + lane], added
// in slice order; two slices are loaded per round so the loads overlap (one
// for the widest vectors, whose registers would not hold two).
template <int VPL>
__device__ __forceinline__ void sum_slices(const float *src, size_t stride, uint32_t splits,
                                           uint32_t lane, float (&v)[VPL]) {
#pragma clang fp contract(off)
    src += lane;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
        v[i] = 0.0f;
    }
    constexpr uint32_t kRound = VPL > 32 ? 1u : 2u;
    for (uint32_t s = 0; s < splits; s += kRound) {
        const bool second = kRound == 2 && s + 1 < splits;
        float a[VPL], b[VPL];
#pragma unroll
        for (int i = 0; i < VPL; ++i) {
            a[i] = src[s * stride + i * 64];
            b[i] = second ? src[(s + 1) * stride + i * 64] : 0.0f;
        }
#pragma unroll
        for (int i = 0; i < VPL; ++i) {
            v[i] = v[i] + a[i];
            v[i] = v[i] + b[i];
        }
    }
}

// Destination of a Hadamard-transformed input vector x_hat:
//   planes 0: fp32 [vectors][n] (decode-GEMV);
//   planes 1: f16 hi/lo pairs [vectors][n] (MFMA GEMM of an NE matrix);
//   planes 2: f16 hi/lo pairs split by expert codebook plane,
//             [2][vectors][n/2] (MFMA GEMM of an expert matrix).
// hi = f16(x_hat), lo = f16(x_hat - hi), so hi + lo carries x_hat to about
// 2^-22 relative. In the plane order, column c of tile column t = c/16 with
// in-tile column q = c%16 goes to plane (q/4)%2 at position t*8 + (q/8)*4 +
// q%4: the eight columns a codebook plane covers in each tile, contiguous.
struct XhatOut {
    float *f32;
    uint16_t *hi;
    uint16_t *lo;
    uint32_t planes;
    uint32_t vectors;  // vectors in the destination (plane stride)
};

__device__ __forceinline__ uint32_t f16_bits_rne(float v) {
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(v));
}

template <int VPL>
__device__ __forceinline__ void store_xhat(const XhatOut &out, uint32_t vector, uint32_t lane,
                                           const float (&v)[VPL]) {
#pragma clang fp contract(off)
    constexpr uint32_t n = 64u * VPL;
    if (out.planes == 0) {
        float *dst = out.f32 + static_cast<size_t>(vector) * n + lane;
#pragma unroll
        for (int i = 0; i < VPL; ++i) {
            dst[i * 64] = v[i];
        }
        return;
    }
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
        const uint32_t hi = f16_bits_rne(v[i]);
        const uint32_t lo = f16_bits_rne(v[i] - half_bits_to_float(hi));
        const uint32_t c = static_cast<uint32_t>(i) * 64u + lane;
        size_t at;
        if (out.planes == 1) {
            at = static_cast<size_t>(vector) * n + c;
        } else {
            const uint32_t q = c & 15u;
            at = static_cast<size_t>((q >> 2) & 1u) * out.vectors * (n / 2) +
                 static_cast<size_t>(vector) * (n / 2) + (c >> 4) * 8u + (q >> 3) * 4u + (q & 3u);
        }
        out.hi[at] = static_cast<uint16_t>(hi);
        out.lo[at] = static_cast<uint16_t>(lo);
    }
}

}  // namespace adi_hip
