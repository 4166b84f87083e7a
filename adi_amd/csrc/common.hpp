// common.hpp -- shared host/device definitions of the gfx950 hot path.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>

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

// A failed runtime call also leaves its error as the thread's last error,
// which the launch checks read: consume it here, so that a failed call (an
// allocation beyond the device's memory) does not fail the next launch.
inline void check_hip(hipError_t error, const char *what) {
    if (error != hipSuccess) {
        (void)hipGetLastError();
        fail(error == hipErrorOutOfMemory ? ADI_HIP_OUT_OF_MEMORY : ADI_HIP_DEVICE_ERROR,
             std::string(what) + ": " + hipGetErrorString(error));
    }
}

inline bool is_power_of_two(uint32_t v) { return v != 0 && (v & (v - 1)) == 0; }

// The wave-per-vector kernels move vectors of 512 or more elements with
// 16-byte accesses (f32 vectors, 16-byte aligned), f16 scale rows with 8-byte
// and +-1 sign rows with 4-byte accesses.
inline bool aligned_to(const void *p, uintptr_t bytes) {
    return (reinterpret_cast<uintptr_t>(p) & (bytes - 1)) == 0;
}

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

// One router logit per LANES-lane group in the CPU's order (dense.hip): lane
// j of the group adds columns j, j + LANES, ... of its row (fused multiply-add
// for the 16-lane order, multiply then add for the 8-lane order), then the
// group's lane sums are added in lane order from 0. w (bf16) and x in LDS.
template <int LANES>
__device__ __forceinline__ float router_chain(const uint16_t *w, const float *x, uint32_t columns,
                                              uint32_t j) {
#pragma clang fp contract(off)
    constexpr uint32_t kBatch = 16;  // LDS reads of 16 steps issued before their adds
    float acc = 0.0f;
    for (uint32_t base = 0; base < columns; base += kBatch * LANES) {
        float wk[kBatch], xk[kBatch];
#pragma unroll
        for (uint32_t u = 0; u < kBatch; ++u) {
            const uint32_t k = base + u * LANES + j;
            wk[u] = bf16_bits_to_float(w[k]);
            xk[u] = x[k];
        }
#pragma unroll
        for (uint32_t u = 0; u < kBatch; ++u) {
            if constexpr (LANES == 16) {
                acc = fmaf(wk[u], xk[u], acc);
            } else {
                acc = acc + wk[u] * xk[u];
            }
        }
    }
    return acc;
}

// The lane sums of lanes group * LANES .. + LANES - 1, added in lane order
// from 0 (every lane gets the sum).
template <int LANES>
__device__ __forceinline__ float router_lane_sum(float acc, uint32_t group) {
#pragma clang fp contract(off)
    float sum = 0.0f;
#pragma unroll
    for (uint32_t j = 0; j < LANES; ++j) {
        sum = sum + __uint_as_float(static_cast<uint32_t>(
                        __builtin_amdgcn_readlane(static_cast<int>(__float_as_uint(acc)),
                                                  static_cast<int>(group * LANES + j))));
    }
    return sum;
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

// rms_norm of one row of up to 2048 values (src/kernels.cpp:1052-1073) by
// threads tid 0..255 of a block; threads from 256 take part in the two block
// barriers only. Thread t holds values t + 256 k (k < 8): value(i) gives them
// (the row, or the row plus a residual), keep(i, v) sees each once (to write
// the sum back), and the sum of squares runs in k order, then over the lanes
// (xor 1 .. 32) and the four waves ((0 + 1) + (2 + 3)); dst[i] = v * scale *
// (offset + w[i]). wave_sums (4 floats) and scale_shared are LDS. The same
// values as the rms_norm launch.
// block_rms_norm from the values a thread already holds: v[k] and the weights
// w[k] (as floats) of indexes tid + 256 k, so that a caller can issue the
// loads early. keep(i, v) sees each value once, first.
template <typename Keep>
__device__ __forceinline__ void block_rms_norm_held(const float (&v)[8], const float (&w)[8], Keep &&keep,
                                                    uint32_t count, float offset, float epsilon, float *dst,
                                                    float *wave_sums, float *scale_shared, uint32_t tid) {
#pragma clang fp contract(off)
    constexpr uint32_t kHeld = 8, kThreads = 256;
    float squares = 0.0f;
    if (tid < kThreads) {
#pragma unroll
        for (uint32_t k = 0; k < kHeld; ++k) {
            const uint32_t i = tid + k * kThreads;
            if (i < count) {
                keep(i, v[k]);
            }
        }
#pragma unroll
        for (uint32_t k = 0; k < kHeld; ++k) {
            if (tid + k * kThreads < count) {
                squares += v[k] * v[k];
            }
        }
        squares += lane_xor<1>(squares);
        squares += lane_xor<2>(squares);
        squares += lane_xor<4>(squares);
        squares += lane_xor<8>(squares);
        squares += lane_xor<16>(squares);
        squares += lane_xor<32>(squares);
        if ((tid & 63u) == 0) {
            wave_sums[tid >> 6] = squares;
        }
    }
    __syncthreads();
    if (tid == 0) {
        const float total = (wave_sums[0] + wave_sums[1]) + (wave_sums[2] + wave_sums[3]);
        *scale_shared = 1.0f / sqrtf(total / static_cast<float>(count) + epsilon);
    }
    __syncthreads();
    if (tid < kThreads) {
        const float scale = *scale_shared;
#pragma unroll
        for (uint32_t k = 0; k < kHeld; ++k) {
            const uint32_t i = tid + k * kThreads;
            if (i < count) {
                dst[i] = v[k] * scale * (offset + w[k]);
            }
        }
    }
}

template <typename Value, typename Keep>
__device__ __forceinline__ void block_rms_norm(Value &&value, Keep &&keep, const uint16_t *weight, uint32_t count,
                                               float offset, float epsilon, float *dst, float *wave_sums,
                                               float *scale_shared, uint32_t tid) {
    constexpr uint32_t kHeld = 8, kThreads = 256;
    float v[kHeld], w[kHeld];
    if (tid < kThreads) {
        // every load issued with its index clamped into the row (count >= 1),
        // the values past the row zeroed after: a branch around each load
        // would make the compiler wait for each before issuing the next
#pragma unroll
        for (uint32_t k = 0; k < kHeld; ++k) {
            const uint32_t i = min(tid + k * kThreads, count - 1u);
            v[k] = value(i);
            w[k] = bf16_bits_to_float(weight[i]);
        }
#pragma unroll
        for (uint32_t k = 0; k < kHeld; ++k) {
            if (tid + k * kThreads >= count) {
                v[k] = 0.0f;
                w[k] = 0.0f;
            }
        }
    }
    block_rms_norm_held(v, w, keep, count, offset, epsilon, dst, wave_sums, scale_shared, tid);
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

// Normalised FWHT of n = 64*VPL values held by one wave in the wave layout
// (tiled_group_base: the tiled layout from VPL 8, element e in lane e % 64,
// register e / 64 below). Each index bit's stride pairs either two registers
// of a lane or lanes l and l ^ mask. Strides run 1, 2, 4, ... and each pair
// becomes (lo + hi, lo - hi): the reference's exact sequence
// (src/simd.cpp:48-63), so the result is bit-identical to it. Every lane of
// the wave must call this.
template <int VPL>
__device__ __forceinline__ void wave_hadamard(float (&v)[VPL], float scale, uint32_t lane) {
#pragma clang fp contract(off)
    // One butterfly stage per index bit b, lower element of each pair a + b,
    // upper a - b. The stages run in index-bit order (strides 1, 2, 4, ...),
    // so the rounding is that of the in-place transform in that order. All
    // exchanges of a lane stage are issued before any is consumed so the
    // LDS-routed ones (masks 16 and 32) pipeline instead of waiting in turn.
    // A lane stage gives the lower lane v + other and the upper other - v,
    // both as fma(+-1, v, other): the product is exact, so the fma rounds
    // the same sum once (x - x and -0 + -0 give the same zeros).
#define ADI_LANE_STAGE(MASK)                                             \
    {                                                                    \
        const float sign = (lane & static_cast<uint32_t>(MASK)) != 0 ? -1.0f : 1.0f; \
        float other[VPL];                                                \
        _Pragma("unroll") for (int i = 0; i < VPL; ++i) {                \
            other[i] = lane_xor<MASK>(v[i]);                             \
        }                                                                \
        _Pragma("unroll") for (int i = 0; i < VPL; ++i) {                \
            v[i] = __builtin_fmaf(sign, v[i], other[i]);                 \
        }                                                                \
    }
#define ADI_REG_STAGE(STRIDE)                                            \
    {                                                                    \
        _Pragma("unroll") for (int i = 0; i < VPL; ++i) {                \
            if ((i & (STRIDE)) == 0) {                                   \
                const float a = v[i];                                    \
                const float b = v[i + (STRIDE)];                         \
                v[i] = a + b;                                            \
                v[i + (STRIDE)] = a - b;                                 \
            }                                                            \
        }                                                                \
    }
    if constexpr (VPL >= 8) {
        // tiled layout: index bits 0, 1, 3 = register bits 0, 1, 2; bit 2 =
        // register bit 3 (VPL >= 16) or lane bit 5; bits 4.. = lane bits, then
        // register bits 4..
        ADI_REG_STAGE(1) ADI_REG_STAGE(2)
        if constexpr (VPL >= 16) {
            ADI_REG_STAGE(8)
        } else {
            ADI_LANE_STAGE(32)
        }
        ADI_REG_STAGE(4)
        ADI_LANE_STAGE(1) ADI_LANE_STAGE(2) ADI_LANE_STAGE(4) ADI_LANE_STAGE(8) ADI_LANE_STAGE(16)
        if constexpr (VPL >= 16) {
            ADI_LANE_STAGE(32)
        }
#pragma unroll
        for (int stride = 16; stride < VPL; stride <<= 1) {
            ADI_REG_STAGE(stride)
        }
    } else {
        // c = 64 i + lane: the lane bits first, then the register bits
        ADI_LANE_STAGE(1) ADI_LANE_STAGE(2) ADI_LANE_STAGE(4) ADI_LANE_STAGE(8)
        ADI_LANE_STAGE(16) ADI_LANE_STAGE(32)
#pragma unroll
        for (int stride = 1; stride < VPL; stride <<= 1) {
            ADI_REG_STAGE(stride)
        }
    }
#undef ADI_LANE_STAGE
#undef ADI_REG_STAGE
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
        v[i] = v[i] * scale;
    }
}


// Tiled wave layout of an n = 64 * VPL vector (VPL >= 8) for the
// wave-per-vector kernels. Register i of lane l holds element c(i, l) with
//   c bits 0, 1 = i bits 0, 1;  c bit 3 = i bit 2;
//   c bit 2     = i bit 3 (VPL >= 16) or l bit 5 (VPL == 8);
//   c bits 4..  = the remaining lane bits, then the remaining register bits.
// Registers 4g .. 4g + 3 are then four consecutive elements (one 16-byte
// load or store) and registers 8k .. 8k + 7 are the eight columns that one
// codebook plane covers in one 16-column tile, in plane order (one 16-byte
// f16 store). Below VPL 8 the layout is c = 64 i + l.
template <int VPL>
__device__ __forceinline__ uint32_t tiled_group_base(uint32_t g, uint32_t lane) {
    static_assert(VPL >= 8, "tiled layout needs 512 or more elements");
    if constexpr (VPL >= 16) {
        return ((g & 1u) << 3) | (((g >> 1) & 1u) << 2) | (lane << 4) | ((g >> 2) << 10);
    } else {
        return ((g & 1u) << 3) | ((lane >> 5) << 2) | ((lane & 31u) << 4);
    }
}

// ---- data handed between blocks of one launch ------------------------------
//
// The L2 of each XCD is not coherent with the others', and the device-scope
// release and acquire fences (an L2 writeback and an L2 invalidate) cost about
// 0.3 us per block on this part, serialised. Data a block passes to another
// block of the same launch therefore moves through device-coherent accesses:
// relaxed device-scope atomics, which compile to sc1 stores (written through
// to memory) and sc1 loads (not served from a line another XCD may hold
// stale). The producer waits for its own stores (wait_stores: vmcnt(0)) before
// the relaxed atomic that signals them; the consumer polls the signal with
// coherent loads. Bulk data it then reads for the first time in the launch
// may come through ordinary loads (no cache can hold an older copy of lines
// the launch has not touched before), which are several times faster than
// 4-byte coherent loads.
__device__ __forceinline__ float coherent_load(const float *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t coherent_load(const uint32_t *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void coherent_store(float *p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void coherent_store(uint32_t *p, uint32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t coherent_add(uint32_t *p, uint32_t v) {
    return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Waits until every memory access the wave issued has completed.
__device__ __forceinline__ void wait_stores() { __builtin_amdgcn_s_waitcnt(0); }
// s_waitcnt operand that waits for the wave's LDS (and scalar) accesses only:
// lgkmcnt 0 (bits 11:8) with vmcnt (bits 15:14, 3:0) and expcnt (bits 6:4)
// at their maxima, so outstanding global loads stay in flight.
constexpr uint16_t kWaitLds = 0xC07F;

// float4 at p (16-byte aligned), through coherent loads when COHERENT.
template <bool COHERENT>
__device__ __forceinline__ float4 load4(const float *p) {
    if constexpr (COHERENT) {
        return make_float4(coherent_load(p), coherent_load(p + 1), coherent_load(p + 2),
                           coherent_load(p + 3));
    } else {
        return *reinterpret_cast<const float4 *>(p);
    }
}

template <bool COHERENT>
__device__ __forceinline__ void store4(float *p, float4 v) {
    if constexpr (COHERENT) {
        coherent_store(p, v.x);
        coherent_store(p + 1, v.y);
        coherent_store(p + 2, v.z);
        coherent_store(p + 3, v.w);
    } else {
        *reinterpret_cast<float4 *>(p) = v;
    }
}

// dst = v from the wave layout (VPL >= 8, dst wave-uniform and 16-byte
// aligned) through 16-byte stores written through to memory (buffer stores
// with the sc1 bit): the coherent form of store_wave for hand-over data.
template <int VPL>
__device__ __forceinline__ void store_wave_through(float *dst, uint32_t lane, const float (&v)[VPL]) {
    static_assert(VPL >= 8, "16-byte groups need the tiled layout");
    typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc(dst, 0, static_cast<int>(64u * VPL * sizeof(float)), 0x00020000);
#pragma unroll
    for (int g = 0; g < VPL / 4; ++g) {
        const u32x4_t q = {__float_as_uint(v[4 * g]), __float_as_uint(v[4 * g + 1]),
                           __float_as_uint(v[4 * g + 2]), __float_as_uint(v[4 * g + 3])};
        __builtin_amdgcn_raw_buffer_store_b128(q, rs, tiled_group_base<VPL>(g, lane) * 4u, 0, 16 /* sc1 */);
    }
}

// v = src in the wave layout (src 16-byte aligned when tiled).
template <int VPL, bool COHERENT = false>
__device__ __forceinline__ void load_wave(const float *src, uint32_t lane, float (&v)[VPL]) {
    if constexpr (VPL >= 8) {
#pragma unroll
        for (int g = 0; g < VPL / 4; ++g) {
            const float4 q = load4<COHERENT>(src + tiled_group_base<VPL>(g, lane));
            v[4 * g] = q.x;
            v[4 * g + 1] = q.y;
            v[4 * g + 2] = q.z;
            v[4 * g + 3] = q.w;
        }
    } else {
#pragma unroll
        for (int i = 0; i < VPL; ++i) {
            v[i] = COHERENT ? coherent_load(src + i * 64 + lane) : src[i * 64 + lane];
        }
    }
}

// v = f16 src in the wave layout, widened (src 8-byte aligned when tiled).
template <int VPL>
__device__ __forceinline__ void load_wave_f16(const uint16_t *src, uint32_t lane, float (&v)[VPL]) {
    if constexpr (VPL >= 8) {
#pragma unroll
        for (int g = 0; g < VPL / 4; ++g) {
            const uint2 q = *reinterpret_cast<const uint2 *>(src + tiled_group_base<VPL>(g, lane));
            v[4 * g] = half_bits_to_float(static_cast<uint16_t>(q.x));
            v[4 * g + 1] = half_bits_to_float(static_cast<uint16_t>(q.x >> 16));
            v[4 * g + 2] = half_bits_to_float(static_cast<uint16_t>(q.y));
            v[4 * g + 3] = half_bits_to_float(static_cast<uint16_t>(q.y >> 16));
        }
    } else {
#pragma unroll
        for (int i = 0; i < VPL; ++i) {
            v[i] = half_bits_to_float(src[i * 64 + lane]);
        }
    }
}

// v = +-1 signs src in the wave layout (src 4-byte aligned when tiled).
template <int VPL>
__device__ __forceinline__ void load_wave_sign(const int8_t *src, uint32_t lane, float (&v)[VPL]) {
    if constexpr (VPL >= 8) {
#pragma unroll
        for (int g = 0; g < VPL / 4; ++g) {
            const uint32_t q = *reinterpret_cast<const uint32_t *>(src + tiled_group_base<VPL>(g, lane));
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                v[4 * g + e] = static_cast<float>(static_cast<int8_t>(q >> (8 * e)));
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < VPL; ++i) {
            v[i] = static_cast<float>(src[i * 64 + lane]);
        }
    }
}

// dst = v from the wave layout.
template <int VPL, bool COHERENT = false>
__device__ __forceinline__ void store_wave(float *dst, uint32_t lane, const float (&v)[VPL]) {
    if constexpr (VPL >= 8) {
#pragma unroll
        for (int g = 0; g < VPL / 4; ++g) {
            store4<COHERENT>(dst + tiled_group_base<VPL>(g, lane),
                             make_float4(v[4 * g], v[4 * g + 1], v[4 * g + 2], v[4 * g + 3]));
        }
    } else {
#pragma unroll
        for (int i = 0; i < VPL; ++i) {
            if constexpr (COHERENT) {
                coherent_store(dst + i * 64 + lane, v[i]);
            } else {
                dst[i * 64 + lane] = v[i];
            }
        }
    }
}

// Up to four slices of a vector of at most 512 elements, loaded at once
// (slices past `splits` reload the last one and are not added).
template <int VPL>
struct SliceLoads {
    float a[4][VPL];
};

template <int VPL, bool COHERENT = false>
__device__ __forceinline__ void load_slices(const float *src, size_t stride, uint32_t splits,
                                            uint32_t lane, SliceLoads<VPL> &l) {
    static_assert(VPL <= 8, "load_slices: vectors of at most 512 elements");
#pragma unroll
    for (uint32_t s = 0; s < 4; ++s) {
        load_wave<VPL, COHERENT>(src + (s < splits ? s : splits - 1u) * stride, lane, l.a[s]);
    }
}

// v = ((0 + slice 0) + slice 1) + ..., the order of sum_slices.
template <int VPL>
__device__ __forceinline__ void add_slices(const SliceLoads<VPL> &l, uint32_t splits,
                                           float (&v)[VPL]) {
#pragma clang fp contract(off)
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
        v[i] = 0.0f + l.a[0][i];
    }
#pragma unroll
    for (uint32_t s = 1; s < 4; ++s) {
#pragma unroll
        for (int i = 0; i < VPL; ++i) {
            v[i] = s < splits ? v[i] + l.a[s][i] : v[i];
        }
    }
}

// v = sum over slices s < splits of src[s * stride ..] in the wave layout,
// added in slice order; two slices are loaded per round so the loads overlap
// (one for the widest vectors, whose registers would not hold two).
template <int VPL, bool COHERENT = false>
__device__ __forceinline__ void sum_slices(const float *src, size_t stride, uint32_t splits,
                                           uint32_t lane, float (&v)[VPL]) {
#pragma clang fp contract(off)
    if constexpr (VPL <= 8) {
        if (splits >= 1 && splits <= 4) {
            SliceLoads<VPL> l;
            load_slices<VPL, COHERENT>(src, stride, splits, lane, l);
            add_slices<VPL>(l, splits, v);
            return;
        }
    }
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
        v[i] = 0.0f;
    }
    // slices loaded per round: four for short vectors (the registers of the
    // at-once path above), two up to 2048 elements, one beyond
    constexpr uint32_t kRound = VPL > 32 ? 1u : (VPL <= 8 ? 4u : 2u);
    for (uint32_t s = 0; s < splits; s += kRound) {
        // a missing later slice reloads the round's first and adds nothing
        float a[kRound][VPL];
#pragma unroll
        for (uint32_t q = 0; q < kRound; ++q) {
            load_wave<VPL, COHERENT>(src + (s + q < splits ? s + q : s) * stride, lane, a[q]);
        }
#pragma unroll
        for (uint32_t q = 0; q < kRound; ++q) {
#pragma unroll
            for (int i = 0; i < VPL; ++i) {
                v[i] = s + q < splits ? v[i] + a[q][i] : v[i];
            }
        }
    }
}

// sum_slices with up to `G` slices of loads in flight per round, G * VPL
// at most 256 registers (for kernels that may hold that many): the same
// slice-order sum, fewer dependent rounds of memory latency.
template <int VPL>
__device__ __forceinline__ void sum_slices_deep(const float *src, size_t stride, uint32_t splits,
                                                uint32_t lane, float (&v)[VPL]) {
#pragma clang fp contract(off)
    constexpr uint32_t G = VPL >= 64 ? 4u : 8u;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
        v[i] = 0.0f;
    }
    for (uint32_t s0 = 0; s0 < splits; s0 += G) {
        float a[G][VPL];
#pragma unroll
        for (uint32_t g = 0; g < G; ++g) {
            // a slice past the end reloads the last one and is not added
            const uint32_t s = s0 + g < splits ? s0 + g : splits - 1u;
            load_wave<VPL>(src + s * stride, lane, a[g]);
        }
#pragma unroll
        for (uint32_t g = 0; g < G; ++g) {
#pragma unroll
            for (int i = 0; i < VPL; ++i) {
                v[i] = s0 + g < splits ? v[i] + a[g][i] : v[i];
            }
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
        store_wave<VPL>(out.f32 + static_cast<size_t>(vector) * n, lane, v);
        return;
    }
    if constexpr (VPL >= 8) {
        uint32_t hi[VPL], lo[VPL];
#pragma unroll
        for (int i = 0; i < VPL; ++i) {
            hi[i] = f16_bits_rne(v[i]);
            lo[i] = f16_bits_rne(v[i] - half_bits_to_float(hi[i]));
        }
        if (out.planes == 1) {
            // four consecutive columns per register group: 8-byte stores
            uint16_t *dh = out.hi + static_cast<size_t>(vector) * n;
            uint16_t *dl = out.lo + static_cast<size_t>(vector) * n;
#pragma unroll
            for (int g = 0; g < VPL / 4; ++g) {
                const uint32_t c = tiled_group_base<VPL>(g, lane);
                *reinterpret_cast<uint2 *>(dh + c) =
                    make_uint2(hi[4 * g] | hi[4 * g + 1] << 16, hi[4 * g + 2] | hi[4 * g + 3] << 16);
                *reinterpret_cast<uint2 *>(dl + c) =
                    make_uint2(lo[4 * g] | lo[4 * g + 1] << 16, lo[4 * g + 2] | lo[4 * g + 3] << 16);
            }
        } else {
            // registers 8k .. 8k + 7: one plane's columns of one tile, in
            // plane order: 16-byte stores
#pragma unroll
            for (int k = 0; k < VPL / 8; ++k) {
                const uint32_t c = tiled_group_base<VPL>(2 * k, lane);  // first column of the eight
                const uint32_t plane = (c >> 2) & 1u, tile = c >> 4;
                const size_t at = static_cast<size_t>(plane) * out.vectors * (n / 2) +
                                  static_cast<size_t>(vector) * (n / 2) + tile * 8u;
                const uint32_t *h = hi + 8 * k, *l = lo + 8 * k;
                *reinterpret_cast<uint4 *>(out.hi + at) =
                    make_uint4(h[0] | h[1] << 16, h[2] | h[3] << 16, h[4] | h[5] << 16, h[6] | h[7] << 16);
                *reinterpret_cast<uint4 *>(out.lo + at) =
                    make_uint4(l[0] | l[1] << 16, l[2] | l[3] << 16, l[4] | l[5] << 16, l[6] | l[7] << 16);
            }
        }
    } else {
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
}

}  // namespace adi_hip
