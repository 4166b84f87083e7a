// head.hip -- int5_g64 output head (src/kernels.cpp:847-979,
// src/simd.cpp:65-86) and the certified greedy arg-max over its logits.
//
// Logits. Each row is columns/8 five-byte blocks, i.e. a little-endian bit
// stream of 5-bit codes u; the weight is (u - 16) * scale of its 64-column
// group. A lane owns 32 consecutive columns ("quad" of 4 blocks, 20 bytes,
// half a scale group) of a row: it loads its 20 bytes as 5 dwords (the lanes
// of a wave cover contiguous bytes), keeps its 32 x values per token in
// registers, and computes scale * (sum u*x - 16 * sum x) with the 32-column x
// sums precomputed per token. Lanes sharing a row add their parts with wave
// shuffles. Waves walk the rows grid-stride.
//
// Certified arg-max. GPU and CPU sum the same exact products w_k*x_k (w_k is
// exact in fp32: a 5-bit integer times an f16) in different orders, so each
// is within (n + 80) * 2^-24 * sum|w_k x_k| of the exact sum, and
// sum|w_k x_k| <= sum_k 16*scale*|x_k| =: A (computed per row alongside the
// logit). A row can be the CPU's first maximum only if its GPU logit plus
// its bound reaches the top GPU logit minus that row's bound; those
// candidates are re-evaluated in the CPU order (ISA lanes, fused or not, as
// the bf16 dot) and the first maximum among them is the CPU's greedy token
// (std::max_element, src/generation.cpp:177-180).
#include "context.hpp"
#include "dense.hpp"

#include <algorithm>

namespace adi_hip {
namespace {

constexpr uint32_t kQuadColumns = 32;

// x sums per 32-column quad: sum x and sum |x|.
__global__ __launch_bounds__(256) void k_head_sums(const float *__restrict__ x, uint32_t columns,
                                                   float *__restrict__ sums,
                                                   float *__restrict__ abs_sums) {
#pragma clang fp contract(off)
    const uint32_t quads = columns / kQuadColumns;
    const uint32_t b = blockIdx.x;
    for (uint32_t q = threadIdx.x; q < quads; q += blockDim.x) {
        const float *src = x + static_cast<size_t>(b) * columns + q * kQuadColumns;
        float s = 0.0f, a = 0.0f;
        for (uint32_t k = 0; k < kQuadColumns; ++k) {
            s += src[k];
            a += fabsf(src[k]);
        }
        sums[static_cast<size_t>(b) * quads + q] = s;
        abs_sums[static_cast<size_t>(b) * quads + q] = a;
    }
}

template <int K>
__device__ __forceinline__ float code_at(const uint32_t (&d)[6]) {
    constexpr int bit = 5 * K;
    constexpr int w = bit / 32;
    constexpr int s = bit % 32;
    if constexpr (s <= 27) {
        return static_cast<float>(__builtin_amdgcn_ubfe(d[w], s, 5));
    } else {
        return static_cast<float>(__builtin_amdgcn_alignbit(d[w + 1], d[w], s) & 31u);
    }
}

// quads = columns/32 must be a power of two <= 64 (columns 64..2048).
template <int NT>
__global__ __launch_bounds__(256) void k_head_gemv(
    const uint8_t *__restrict__ packed, const uint16_t *__restrict__ scales, uint32_t rows,
    uint32_t columns, const float *__restrict__ x, const float *__restrict__ sums,
    const float *__restrict__ abs_sums, uint32_t batch, float *__restrict__ logits,
    float *__restrict__ bounds) {
    const uint32_t quads = columns / kQuadColumns;
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t quad = lane % quads;
    const uint32_t rows_per_wave = 64u / quads;
    const uint32_t wave_global = blockIdx.x * (blockDim.x / 64u) + (threadIdx.x >> 6);
    const uint32_t wave_count = gridDim.x * (blockDim.x / 64u);
    const uint32_t groups = columns / 64u;

    for (uint32_t t0 = 0; t0 < batch; t0 += NT) {
        float xv[NT][kQuadColumns];
        float sx[NT], sa[NT];
#pragma unroll
        for (int j = 0; j < NT; ++j) {
            const bool ok = t0 + j < batch;
            const float4 *src = reinterpret_cast<const float4 *>(
                x + static_cast<size_t>(ok ? t0 + j : t0) * columns + quad * kQuadColumns);
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                const float4 v = src[q];
                xv[j][4 * q] = v.x;
                xv[j][4 * q + 1] = v.y;
                xv[j][4 * q + 2] = v.z;
                xv[j][4 * q + 3] = v.w;
            }
            const size_t si = static_cast<size_t>(ok ? t0 + j : t0) * quads + quad;
            sx[j] = sums[si];
            sa[j] = abs_sums[si];
        }
        for (uint32_t row0 = wave_global * rows_per_wave; row0 < rows;
             row0 += wave_count * rows_per_wave) {
            const uint32_t row = row0 + lane / quads;
            const bool ok = row < rows;
            uint32_t d[6] = {0u, 0u, 0u, 0u, 0u, 0u};
            float scale = 0.0f;
            if (ok) {
                const uint32_t *src = reinterpret_cast<const uint32_t *>(packed) +
                                      (static_cast<size_t>(row) * quads + quad) * 5u;
#pragma unroll
                for (int i = 0; i < 5; ++i) {
                    d[i] = __builtin_nontemporal_load(src + i);
                }
                scale = half_bits_to_float(scales[static_cast<size_t>(row) * groups + quad / 2u]);
            }
            float u[kQuadColumns];
#define ADI_CODE(K) u[K] = code_at<K>(d);
            ADI_CODE(0) ADI_CODE(1) ADI_CODE(2) ADI_CODE(3) ADI_CODE(4) ADI_CODE(5) ADI_CODE(6)
            ADI_CODE(7) ADI_CODE(8) ADI_CODE(9) ADI_CODE(10) ADI_CODE(11) ADI_CODE(12)
            ADI_CODE(13) ADI_CODE(14) ADI_CODE(15) ADI_CODE(16) ADI_CODE(17) ADI_CODE(18)
            ADI_CODE(19) ADI_CODE(20) ADI_CODE(21) ADI_CODE(22) ADI_CODE(23) ADI_CODE(24)
            ADI_CODE(25) ADI_CODE(26) ADI_CODE(27) ADI_CODE(28) ADI_CODE(29) ADI_CODE(30)
            ADI_CODE(31)
#undef ADI_CODE
            float val[NT], bnd[NT];
#pragma unroll
            for (int j = 0; j < NT; ++j) {
                float acc0 = 0.0f, acc1 = 0.0f;
#pragma unroll
                for (int k = 0; k < 32; k += 2) {
                    acc0 = fmaf(u[k], xv[j][k], acc0);
                    acc1 = fmaf(u[k + 1], xv[j][k + 1], acc1);
                }
                val[j] = scale * ((acc0 + acc1) - 16.0f * sx[j]);
                bnd[j] = 16.0f * scale * sa[j];
            }
            for (uint32_t off = 1; off < quads; off <<= 1) {
#pragma unroll
                for (int j = 0; j < NT; ++j) {
                    val[j] += __shfl_xor(val[j], static_cast<int>(off));
                    bnd[j] += __shfl_xor(bnd[j], static_cast<int>(off));
                }
            }
            if (ok && quad == 0) {
#pragma unroll
                for (int j = 0; j < NT; ++j) {
                    if (t0 + j < batch) {
                        logits[static_cast<size_t>(t0 + j) * rows + row] = val[j];
                        if (bounds != nullptr) {
                            bounds[static_cast<size_t>(t0 + j) * rows + row] = bnd[j];
                        }
                    }
                }
            }
        }
    }
}

// Sums V per-lane values over the 64 lanes of a wave by halving exchanges:
// at offset 1 a lane keeps one half of its values and sends the other, then
// at offset 2 half of the rest, until one value is left, which the remaining
// offsets sum over all lanes. `which` says which value the lane ends with;
// lanes 0..V-1 hold all V. Every value is summed over the same pair tree as
// a full xor butterfly with offsets 1, 2, ..., 32, so the sums are
// bit-identical to it.
__device__ __forceinline__ bool first_max_before(float a, uint32_t ia, float b, uint32_t ib) {
    return a == b ? ia < ib : a > b;
}

// Per-wave summaries the 2048-column GEMV leaves for the certified arg-max,
// [batch][waves] each: the wave's first maximum logit and its row
// (0xFFFFFFFF for a wave with no rows), and the largest
// fmaf(factor, bound, logit) over the wave's rows.
struct HeadWaveBest {
    float factor;
    float *value;
    uint32_t *index;
    float *upper;
};

template <int V>
__device__ __forceinline__ float reduce_scatter64(float (&v)[V], uint32_t lane,
                                                  uint32_t &which) {
#pragma clang fp contract(off)
    uint32_t off = 1;
    which = 0;
#pragma unroll
    for (int h = V / 2; h >= 1; h /= 2) {
        const bool hi = (lane & off) != 0u;
#pragma unroll
        for (int i = 0; i < h; ++i) {
            const float send = hi ? v[i] : v[i + h];
            const float keep = hi ? v[i + h] : v[i];
            v[i] = keep + __shfl_xor(send, static_cast<int>(off));
        }
        which += hi ? static_cast<uint32_t>(h) : 0u;
        off <<= 1;
    }
    for (; off < 64u; off <<= 1) {
        v[0] += __shfl_xor(v[0], static_cast<int>(off));
    }
    return v[0];
}

// k_head_gemv for 2048 columns (64 quads: one row per wave per pass), with
// the x sums of a lane's quad computed in place, the next row's codes loaded
// while this row is summed, the lane sums
// reduce-scattered, and the bound sums only when they are wanted.
template <int NT, bool BOUNDS>
__global__ __launch_bounds__(256) void k_head_gemv_2048(
    const uint8_t *__restrict__ packed, const uint16_t *__restrict__ scales, uint32_t rows,
    const float *__restrict__ x, uint32_t batch, float *__restrict__ logits,
    float *__restrict__ bounds, HeadWaveBest best) {
    // no contraction: a lane's logit stays a rounded product in every variant
    // (with the bounds or without), so both variants give the same bits
#pragma clang fp contract(off)
    constexpr uint32_t columns = 2048u, quads = 64u, groups = 32u;
    constexpr int V = BOUNDS ? 2 * NT : NT;
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave_global = blockIdx.x * (blockDim.x / 64u) + (threadIdx.x >> 6);
    const uint32_t wave_count = gridDim.x * (blockDim.x / 64u);
    const uint32_t *codes = reinterpret_cast<const uint32_t *>(packed);

    for (uint32_t t0 = 0; t0 < batch; t0 += NT) {
        float xv[NT][kQuadColumns];
        float sx[NT], sa[NT];
#pragma unroll
        for (int j = 0; j < NT; ++j) {
            const uint32_t t = t0 + j < batch ? t0 + j : t0;
            const float4 *src = reinterpret_cast<const float4 *>(
                x + static_cast<size_t>(t) * columns + lane * kQuadColumns);
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                const float4 v = src[q];
                xv[j][4 * q] = v.x;
                xv[j][4 * q + 1] = v.y;
                xv[j][4 * q + 2] = v.z;
                xv[j][4 * q + 3] = v.w;
            }
            // the quad's sums of x and |x|, in k_head_sums' order
            float s = 0.0f, a = 0.0f;
#pragma unroll
            for (int k = 0; k < 32; ++k) {
                s += xv[j][k];
                a += fabsf(xv[j][k]);
            }
            sx[j] = s;
            sa[j] = a;
        }
        // with the bounds, even lanes end a row with a logit and their odd
        // partners with its bound (the first halving exchange is at offset 1)
        float best_v = -INFINITY, upper = -INFINITY;
        uint32_t best_i = 0xFFFFFFFFu;
        uint32_t row = wave_global;
        uint32_t dn[5] = {0u, 0u, 0u, 0u, 0u};
        uint16_t sn = 0;
        if (row < rows) {
            const uint32_t *src = codes + (static_cast<size_t>(row) * quads + lane) * 5u;
#pragma unroll
            for (int i = 0; i < 5; ++i) {
                dn[i] = __builtin_nontemporal_load(src + i);
            }
            sn = scales[static_cast<size_t>(row) * groups + lane / 2u];
        }
        for (; row < rows; row += wave_count) {
            uint32_t d[6] = {dn[0], dn[1], dn[2], dn[3], dn[4], 0u};
            const float scale = half_bits_to_float(sn);
            const uint32_t next = row + wave_count;
            if (next < rows) {
                const uint32_t *src = codes + (static_cast<size_t>(next) * quads + lane) * 5u;
#pragma unroll
                for (int i = 0; i < 5; ++i) {
                    dn[i] = __builtin_nontemporal_load(src + i);
                }
                sn = scales[static_cast<size_t>(next) * groups + lane / 2u];
            }
            float u[kQuadColumns];
#define ADI_CODE(K) u[K] = code_at<K>(d);
            ADI_CODE(0) ADI_CODE(1) ADI_CODE(2) ADI_CODE(3) ADI_CODE(4) ADI_CODE(5) ADI_CODE(6)
            ADI_CODE(7) ADI_CODE(8) ADI_CODE(9) ADI_CODE(10) ADI_CODE(11) ADI_CODE(12)
            ADI_CODE(13) ADI_CODE(14) ADI_CODE(15) ADI_CODE(16) ADI_CODE(17) ADI_CODE(18)
            ADI_CODE(19) ADI_CODE(20) ADI_CODE(21) ADI_CODE(22) ADI_CODE(23) ADI_CODE(24)
            ADI_CODE(25) ADI_CODE(26) ADI_CODE(27) ADI_CODE(28) ADI_CODE(29) ADI_CODE(30)
            ADI_CODE(31)
#undef ADI_CODE
            float v[V];
#pragma unroll
            for (int j = 0; j < NT; ++j) {
                float acc0 = 0.0f, acc1 = 0.0f;
#pragma unroll
                for (int k = 0; k < 32; k += 2) {
                    acc0 = fmaf(u[k], xv[j][k], acc0);
                    acc1 = fmaf(u[k + 1], xv[j][k + 1], acc1);
                }
                v[j] = scale * ((acc0 + acc1) - 16.0f * sx[j]);
                if constexpr (BOUNDS) {
                    v[NT + j] = 16.0f * scale * sa[j];
                }
            }
            uint32_t k;
            const float total = reduce_scatter64<V>(v, lane, k);
            if (lane < static_cast<uint32_t>(V)) {
                const uint32_t j = k % NT;
                if (t0 + j < batch) {
                    float *dst = BOUNDS && k >= NT ? bounds : logits;
                    dst[static_cast<size_t>(t0 + j) * rows + row] = total;
                }
            }
            if constexpr (BOUNDS) {
                const float bound = __shfl_xor(total, 1);
                const float up = fmaf(best.factor, bound, total);
                upper = up > upper ? up : upper;
                if (best_i == 0xFFFFFFFFu || first_max_before(total, row, best_v, best_i)) {
                    best_v = total;
                    best_i = row;
                }
            }
        }
        if constexpr (BOUNDS) {
            uint32_t j = 0;  // the token of an even lane below V (as reduce_scatter64)
            for (uint32_t off = 1, h = V / 2; h >= 1u; h /= 2u, off <<= 1) {
                j += (lane & off) != 0u ? h : 0u;
            }
            if (best.value != nullptr && (lane & 1u) == 0u && lane < static_cast<uint32_t>(V) &&
                t0 + j < batch) {
                const size_t at = static_cast<size_t>(t0 + j) * wave_count + wave_global;
                best.value[at] = best_v;
                best.index[at] = best_i;
                best.upper[at] = upper;
            }
        }
    }
}

// A row's dot in the CPU order: weights of lane j are columns j, j+LANES,
// ...; lane sums added 0..LANES-1 from 0; then the tail (columns % LANES).
// `weight(k)` supplies w_k. Runs on one wave; the result is valid on lane 0.
template <int LANES, bool FUSED, typename Weight>
__device__ float ordered_row_dot(uint32_t columns, const float *__restrict__ x, Weight weight) {
#pragma clang fp contract(off)
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t full = columns / LANES * LANES;
    float acc = 0.0f;
    if (lane < LANES) {
        // unrolled so that the loads of many steps are in flight at once;
        // the sum still runs in k order
#pragma unroll 16
        for (uint32_t base = 0; base < full; base += LANES) {
            const uint32_t k = base + lane;
            if constexpr (FUSED) {
                acc = fmaf(weight(k), x[k], acc);
            } else {
                acc = acc + weight(k) * x[k];
            }
        }
    }
    float sum = 0.0f;
    for (int j = 0; j < LANES; ++j) {
        sum = sum + __shfl(acc, j);
    }
    for (uint32_t k = full; k < columns; ++k) {
        if constexpr (FUSED) {
            sum = fmaf(weight(k), x[k], sum);
        } else {
            sum = sum + weight(k) * x[k];
        }
    }
    return sum;
}

struct HeadView {
    const uint8_t *packed;
    const uint16_t *scales;
    const uint32_t *protected_rows;
    const uint16_t *protected_bf16;
    uint32_t protected_count;
    uint32_t rows;
    uint32_t columns;
};

template <int LANES, bool FUSED>
__device__ float exact_logit(const HeadView &h, uint32_t row, const float *x) {
    for (uint32_t p = 0; p < h.protected_count; ++p) {
        if (h.protected_rows[p] == row) {
            const uint16_t *w = h.protected_bf16 + static_cast<size_t>(p) * h.columns;
            return ordered_row_dot<LANES, FUSED>(
                h.columns, x, [&](uint32_t k) { return bf16_bits_to_float(w[k]); });
        }
    }
    const uint8_t *rb = h.packed + static_cast<size_t>(row) * (h.columns / 8u * 5u);
    const uint16_t *rs = h.scales + static_cast<size_t>(row) * (h.columns / 64u);
    return ordered_row_dot<LANES, FUSED>(h.columns, x, [&](uint32_t k) {
        const uint32_t block = k >> 3, index = k & 7u;
        const uint8_t *bytes = rb + block * 5u;
        uint64_t word = 0;
        for (int i = 0; i < 5; ++i) {
            word |= static_cast<uint64_t>(bytes[i]) << (8 * i);
        }
        const int code = static_cast<int>((word >> (5u * index)) & 31u) - 16;
        return static_cast<float>(code) * half_bits_to_float(rs[k >> 6]);
    });
}

// Protected rows: their logits are the bf16 dot in CPU order, exactly.
template <int LANES, bool FUSED>
__global__ __launch_bounds__(64) void k_head_protected(HeadView h, const float *__restrict__ x,
                                                       float *__restrict__ logits,
                                                       float *__restrict__ bounds) {
    const uint32_t p = blockIdx.x, b = blockIdx.y;
    const uint16_t *w = h.protected_bf16 + static_cast<size_t>(p) * h.columns;
    const float v = ordered_row_dot<LANES, FUSED>(
        h.columns, x + static_cast<size_t>(b) * h.columns,
        [&](uint32_t k) { return bf16_bits_to_float(w[k]); });
    const uint32_t row = h.protected_rows[p];
    if (threadIdx.x == 0 && row < h.rows) {  // rows out of range are ignored
        const size_t at = static_cast<size_t>(b) * h.rows + row;
        logits[at] = v;
        if (bounds != nullptr) {
            bounds[at] = 0.0f;
        }
    }
}

// Every row in CPU order (fallback for widths the fast kernel does not tile).
template <int LANES, bool FUSED>
__global__ __launch_bounds__(64) void k_head_exact_rows(HeadView h, const float *__restrict__ x,
                                                        float *__restrict__ logits,
                                                        float *__restrict__ bounds) {
    const uint32_t row = blockIdx.x, b = blockIdx.y;
    const float v = exact_logit<LANES, FUSED>(h, row, x + static_cast<size_t>(b) * h.columns);
    if (threadIdx.x == 0) {
        logits[static_cast<size_t>(b) * h.rows + row] = v;
        if (bounds != nullptr) {
            bounds[static_cast<size_t>(b) * h.rows + row] = 0.0f;
        }
    }
}

constexpr uint32_t kArgmaxThreads = 1024;
constexpr uint32_t kCandidateCap = 2048;
constexpr uint32_t kWaveListCap = 1024;

__device__ __forceinline__ uint32_t ceil_div_device(uint32_t a, uint32_t b) {
    return (a + b - 1u) / b;
}

// Calls f(r, logit, bound) for every row r of this thread's share of the
// block, each row once: 16-byte loads (four of the logits in flight, or two
// of each array with the bounds) when the arrays are 16-byte aligned, one
// float at a time otherwise. `bound` is 0 when BOUND is false.
template <bool BOUND, typename F>
__device__ __forceinline__ void for_each_head_row(const float *__restrict__ a,
                                                  const float *__restrict__ b, uint32_t count,
                                                  F &&f) {
    constexpr uint32_t kUnroll = BOUND ? 2u : 4u;
    const uint32_t step = blockDim.x;
    const uintptr_t bits =
        reinterpret_cast<uintptr_t>(a) | (BOUND ? reinterpret_cast<uintptr_t>(b) : uintptr_t(0));
    if ((bits & 15u) == 0u) {
        const uint32_t vectors = count / 4u;
        const float4 *a4 = reinterpret_cast<const float4 *>(a);
        const float4 *b4 = reinterpret_cast<const float4 *>(b);
        uint32_t j = threadIdx.x;
        for (; j + (kUnroll - 1u) * step < vectors; j += kUnroll * step) {
            float4 va[kUnroll], vb[kUnroll];
#pragma unroll
            for (uint32_t u = 0; u < kUnroll; ++u) {
                va[u] = a4[j + u * step];
                vb[u] = BOUND ? b4[j + u * step] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            }
#pragma unroll
            for (uint32_t u = 0; u < kUnroll; ++u) {
                const uint32_t i = 4u * (j + u * step);
                f(i, va[u].x, vb[u].x);
                f(i + 1u, va[u].y, vb[u].y);
                f(i + 2u, va[u].z, vb[u].z);
                f(i + 3u, va[u].w, vb[u].w);
            }
        }
        for (; j < vectors; j += step) {
            const float4 va = a4[j];
            const float4 vb = BOUND ? b4[j] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            f(4u * j, va.x, vb.x);
            f(4u * j + 1u, va.y, vb.y);
            f(4u * j + 2u, va.z, vb.z);
            f(4u * j + 3u, va.w, vb.w);
        }
        for (uint32_t i = 4u * vectors + threadIdx.x; i < count; i += step) {
            f(i, a[i], BOUND ? b[i] : 0.0f);
        }
    } else {
        for (uint32_t i = threadIdx.x; i < count; i += step) {
            f(i, a[i], BOUND ? b[i] : 0.0f);
        }
    }
}

// One block per row of logits: top GPU logit, candidate rows, exact
// re-evaluation, first maximum.
//
// With WAVES the GEMV's per-wave summaries stand in for the scans: the top
// logit is the first maximum of the waves' maxima, and only the rows of
// waves whose largest fmaf(factor, bound, logit) reaches the threshold are
// tested (a wave of `wave_count` covers rows w, w + wave_count, ...). The
// candidate set is the same as the full scan's.
template <int LANES, bool FUSED, bool WAVES>
__global__ __launch_bounds__(kArgmaxThreads) void k_head_argmax(
    HeadView h, const float *__restrict__ x, const float *__restrict__ logits,
    const float *__restrict__ bounds, float factor, const float *__restrict__ wave_value,
    const uint32_t *__restrict__ wave_index, const float *__restrict__ wave_upper,
    uint32_t wave_count, uint32_t *__restrict__ argmax) {
    __shared__ float best_value[kArgmaxThreads / 64];
    __shared__ uint32_t best_index[kArgmaxThreads / 64];
    __shared__ uint32_t candidates[kCandidateCap];
    __shared__ uint32_t candidate_count;
    __shared__ float threshold;
    __shared__ uint32_t wave_list[WAVES ? kWaveListCap : 1];
    __shared__ __align__(16) float weights[WAVES ? kArgmaxThreads / 64 : 1][WAVES ? 2048 : 4];
    __shared__ uint32_t wave_list_count;
    const uint32_t b = blockIdx.x;
    const float *row_logits = logits + static_cast<size_t>(b) * h.rows;
    const float *row_bounds = bounds + static_cast<size_t>(b) * h.rows;
    const float *xb = x + static_cast<size_t>(b) * h.columns;
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t waves = kArgmaxThreads / 64;

    // 1. first maximum of the GPU logits
    float v = -INFINITY;
    uint32_t vi = 0xFFFFFFFFu;
    if constexpr (WAVES) {
        const size_t base = static_cast<size_t>(b) * wave_count;
        for (uint32_t w = threadIdx.x; w < wave_count; w += kArgmaxThreads) {
            const uint32_t r = wave_index[base + w];
            const float c = wave_value[base + w];
            if (r != 0xFFFFFFFFu && (vi == 0xFFFFFFFFu || first_max_before(c, r, v, vi))) {
                v = c;
                vi = r;
            }
        }
    } else {
        for_each_head_row<false>(row_logits, nullptr, h.rows, [&](uint32_t r, float c, float) {
            if (vi == 0xFFFFFFFFu || first_max_before(c, r, v, vi)) {
                v = c;
                vi = r;
            }
        });
    }
    for (int off = 32; off >= 1; off >>= 1) {
        const float ov = __shfl_xor(v, off);
        const uint32_t oi = static_cast<uint32_t>(__shfl_xor(static_cast<int>(vi), off));
        if (oi != 0xFFFFFFFFu && (vi == 0xFFFFFFFFu || first_max_before(ov, oi, v, vi))) {
            v = ov;
            vi = oi;
        }
    }
    if (lane == 0) {
        best_value[wave] = v;
        best_index[wave] = vi;
    }
    if (threadIdx.x == 0) {
        candidate_count = 0;
        wave_list_count = 0;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float bv = best_value[0];
        uint32_t bi = best_index[0];
        for (uint32_t w = 1; w < waves; ++w) {
            if (best_index[w] != 0xFFFFFFFFu && first_max_before(best_value[w], best_index[w], bv, bi)) {
                bv = best_value[w];
                bi = best_index[w];
            }
        }
        threshold = bv - factor * row_bounds[bi];
    }
    __syncthreads();
    // 2. candidates: rows whose bound interval reaches the threshold
    const float t = threshold;
    const auto consider = [&](uint32_t r, float c, float bd) {
        if (fmaf(factor, bd, c) >= t) {
            const uint32_t slot = atomicAdd(&candidate_count, 1u);
            if (slot < kCandidateCap) {
                candidates[slot] = r;
            }
        }
    };
    if constexpr (WAVES) {
        // the waves that reach the threshold, then their rows over the block
        // (every row of a wave once); too many such waves: the full scan
        const size_t base = static_cast<size_t>(b) * wave_count;
        for (uint32_t w = threadIdx.x; w < wave_count; w += kArgmaxThreads) {
            if (wave_upper[base + w] >= t) {
                const uint32_t slot = atomicAdd(&wave_list_count, 1u);
                if (slot < kWaveListCap) {
                    wave_list[slot] = w;
                }
            }
        }
        __syncthreads();
        const uint32_t listed = wave_list_count;
        if (listed <= kWaveListCap) {
            const uint32_t passes = ceil_div_device(h.rows, wave_count);
            for (uint32_t k = threadIdx.x; k < listed * passes; k += kArgmaxThreads) {
                const uint32_t r = wave_list[k / passes] + (k % passes) * wave_count;
                if (r < h.rows) {
                    consider(r, row_logits[r], row_bounds[r]);
                }
            }
        } else {
            for_each_head_row<true>(row_logits, row_bounds, h.rows, consider);
        }
    } else {
        for_each_head_row<true>(row_logits, row_bounds, h.rows, consider);
    }
    __syncthreads();
    const uint32_t count = candidate_count;
    const bool overflow = count > kCandidateCap;
    const uint32_t work = overflow ? h.rows : count;
    // 3. exact re-evaluation, one wave per candidate
    float wv = -INFINITY;
    uint32_t wi = 0xFFFFFFFFu;
    for (uint32_t c = wave; c < work; c += waves) {
        const uint32_t r = overflow ? c : candidates[c];
        float e;
        if constexpr (WAVES) {
            // 2048 columns, no protected rows: the wave decodes the row into
            // LDS with the GEMV's coalesced loads (lane l: columns 32l..32l+31,
            // the same float (u - 16) * scale as exact_logit), then runs the
            // CPU-order dot over it
            float *w = weights[wave];
            const uint32_t *src = reinterpret_cast<const uint32_t *>(h.packed) +
                                  (static_cast<size_t>(r) * 64u + lane) * 5u;
            uint32_t d[6] = {src[0], src[1], src[2], src[3], src[4], 0u};
            const float scale = half_bits_to_float(h.scales[static_cast<size_t>(r) * 32u + lane / 2u]);
            float u[kQuadColumns];
#define ADI_CODE(K) u[K] = code_at<K>(d);
            ADI_CODE(0) ADI_CODE(1) ADI_CODE(2) ADI_CODE(3) ADI_CODE(4) ADI_CODE(5) ADI_CODE(6)
            ADI_CODE(7) ADI_CODE(8) ADI_CODE(9) ADI_CODE(10) ADI_CODE(11) ADI_CODE(12)
            ADI_CODE(13) ADI_CODE(14) ADI_CODE(15) ADI_CODE(16) ADI_CODE(17) ADI_CODE(18)
            ADI_CODE(19) ADI_CODE(20) ADI_CODE(21) ADI_CODE(22) ADI_CODE(23) ADI_CODE(24)
            ADI_CODE(25) ADI_CODE(26) ADI_CODE(27) ADI_CODE(28) ADI_CODE(29) ADI_CODE(30)
            ADI_CODE(31)
#undef ADI_CODE
            float4 *w4 = reinterpret_cast<float4 *>(w + lane * kQuadColumns);
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                w4[q] = make_float4(static_cast<float>(static_cast<int>(u[4 * q]) - 16) * scale,
                                    static_cast<float>(static_cast<int>(u[4 * q + 1]) - 16) * scale,
                                    static_cast<float>(static_cast<int>(u[4 * q + 2]) - 16) * scale,
                                    static_cast<float>(static_cast<int>(u[4 * q + 3]) - 16) * scale);
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            e = ordered_row_dot<LANES, FUSED>(2048u, xb, [&](uint32_t k) { return w[k]; });
            // every lane's reads of w end before the next row is written
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        } else {
            e = exact_logit<LANES, FUSED>(h, r, xb);
        }
        if (wi == 0xFFFFFFFFu || first_max_before(e, r, wv, wi)) {
            wv = e;
            wi = r;
        }
    }
    __syncthreads();
    if (lane == 0) {
        best_value[wave] = wv;
        best_index[wave] = wi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float bv = best_value[0];
        uint32_t bi = best_index[0];
        for (uint32_t w = 1; w < waves; ++w) {
            if (best_index[w] != 0xFFFFFFFFu &&
                (bi == 0xFFFFFFFFu || first_max_before(best_value[w], best_index[w], bv, bi))) {
                bv = best_value[w];
                bi = best_index[w];
            }
        }
        argmax[b] = bi;
    }
}

void validate_head(const adi_hip_head_chunk *h) {
    require(h != nullptr, "Mach output head is null");
    require(h->rows > 0 && h->columns > 0 && h->columns % 64u == 0,
            "Mach output head shape mismatch");
    require(h->packed != nullptr && h->group_scale_f16 != nullptr,
            "Mach output head tensor is null");
    require(h->protected_count == 0 ||
                (h->protected_rows != nullptr && h->protected_bf16 != nullptr),
            "Mach protected output row shape mismatch");
}

bool fast_width(uint32_t columns) {
    const uint32_t quads = columns / kQuadColumns;
    return columns % 64u == 0 && is_power_of_two(quads) && quads <= 64u;
}

HeadView view_of(const adi_hip_head_chunk *h) {
    return HeadView{h->packed,         h->group_scale_f16, h->protected_rows,
                    h->protected_bf16, h->protected_count, h->rows,
                    h->columns};
}

template <int LANES, bool FUSED>
void launch_exact_parts(adi_hip_context *ctx, const HeadView &v, const float *x, uint32_t batch,
                        float *logits, float *bounds, bool all_rows) {
    if (all_rows) {
        launch(ctx, "head_exact", k_head_exact_rows<LANES, FUSED>, dim3(v.rows, batch), dim3(64),
               0, v, x, logits, bounds);
    } else if (v.protected_count > 0) {
        launch(ctx, "head_protected", k_head_protected<LANES, FUSED>,
               dim3(v.protected_count, batch), dim3(64), 0, v, x, logits, bounds);
    }
}

// Blocks of the 2048-column GEMV: one row per wave per pass, enough waves
// for four passes each.
uint32_t head_wide_blocks(const adi_hip_context *ctx, uint32_t rows) {
    return std::min<uint32_t>(ceil_div(rows, 4u * 4u), static_cast<uint32_t>(ctx->cu_count) * 8u);
}

// Whether head_logits can leave per-wave summaries (2048 columns, no
// protected rows: those are rewritten after the GEMV).
bool head_wave_best(const adi_hip_head_chunk *h) {
    return h->columns == 2048u && h->protected_count == 0;
}

void head_logits(adi_hip_context *ctx, const adi_hip_head_chunk *h, const float *x,
                 uint32_t batch, float *logits, float *bounds,
                 HeadWaveBest best = HeadWaveBest{0.0f, nullptr, nullptr, nullptr}) {
    const HeadView v = view_of(h);
    const bool fast = fast_width(h->columns);
    if (fast) {
        const uint32_t quads = h->columns / kQuadColumns;
        auto &ws = ctx->workspace;
        float *sums = ws.take<float>(size_t(batch) * quads);
        float *abs_sums = ws.take<float>(size_t(batch) * quads);
        if (quads != 64u) {
            launch(ctx, "head_sums", k_head_sums, dim3(batch), dim3(256), 0, x, h->columns, sums,
                   abs_sums);
        }
        const uint32_t rows_per_block = 4u * (64u / quads);
        const uint32_t blocks = std::min<uint32_t>(ceil_div(h->rows, rows_per_block),
                                                   static_cast<uint32_t>(ctx->cu_count) * 8u);
        if (quads == 64u) {
            const uint32_t wide = head_wide_blocks(ctx, h->rows);
            const bool with = bounds != nullptr;
            const auto kernel = batch == 1 ? (with ? k_head_gemv_2048<1, true>
                                                   : k_head_gemv_2048<1, false>)
                                           : (with ? k_head_gemv_2048<4, true>
                                                   : k_head_gemv_2048<4, false>);
            launch(ctx, "head_gemv", kernel, dim3(wide), dim3(256), 0, h->packed,
                   h->group_scale_f16, h->rows, x, batch, logits, bounds, best);
        } else if (batch == 1) {
            launch(ctx, "head_gemv", k_head_gemv<1>, dim3(blocks), dim3(256), 0, h->packed,
                   h->group_scale_f16, h->rows, h->columns, x, static_cast<const float *>(sums),
                   static_cast<const float *>(abs_sums), batch, logits, bounds);
        } else {
            launch(ctx, "head_gemv", k_head_gemv<4>, dim3(blocks), dim3(256), 0, h->packed,
                   h->group_scale_f16, h->rows, h->columns, x, static_cast<const float *>(sums),
                   static_cast<const float *>(abs_sums), batch, logits, bounds);
        }
    }
    switch (ctx->isa_lanes) {
    case 1:
        launch_exact_parts<1, false>(ctx, v, x, batch, logits, bounds, !fast);
        break;
    case 8:
        launch_exact_parts<8, false>(ctx, v, x, batch, logits, bounds, !fast);
        break;
    default:
        launch_exact_parts<16, true>(ctx, v, x, batch, logits, bounds, !fast);
        break;
    }
}

size_t head_workspace(const adi_hip_context *ctx, const adi_hip_head_chunk *h, uint32_t batch,
                      bool with_logits, bool with_bounds) {
    const size_t quads = h->columns / kQuadColumns;
    const size_t waves = static_cast<size_t>(head_wide_blocks(ctx, h->rows)) * 4u;
    return Workspace::round(batch * quads * 4) * 2 +
           (with_bounds && head_wave_best(h) ? Workspace::round(batch * waves * 4) * 3 : 0) +
           (with_logits ? Workspace::round(size_t(batch) * h->rows * 4) : 0) +
           (with_bounds ? Workspace::round(size_t(batch) * h->rows * 4) : 0);
}

}  // namespace
}  // namespace adi_hip

using namespace adi_hip;

extern "C" {

int adi_hip_head_matmul(adi_hip_context *ctx, const adi_hip_head_chunk *h, const float *inputs,
                        uint32_t batch, float *outputs) {
    return guarded(ctx, [&] {
        validate_head(h);
        require(batch > 0 && inputs != nullptr && outputs != nullptr,
                "Mach output head batch shape mismatch");
        auto &ws = ctx->workspace;
        ws.used = 0;
        ws.ensure(head_workspace(ctx, h, batch, false, false));
        head_logits(ctx, h, inputs, batch, outputs, nullptr);
    });
}

int adi_hip_head_matvec(adi_hip_context *ctx, const adi_hip_head_chunk *h, const float *input,
                        float *output) {
    return adi_hip_head_matmul(ctx, h, input, 1, output);
}

int adi_hip_head_argmax(adi_hip_context *ctx, const adi_hip_head_chunk *h, const float *inputs,
                        uint32_t batch, float *logits, uint32_t *argmax) {
    return guarded(ctx, [&] {
        validate_head(h);
        require(batch > 0 && inputs != nullptr && argmax != nullptr,
                "Mach output head batch shape mismatch");
        auto &ws = ctx->workspace;
        ws.used = 0;
        ws.ensure(head_workspace(ctx, h, batch, logits == nullptr, true));
        float *out = logits != nullptr ? logits : ws.take<float>(size_t(batch) * h->rows);
        float *bounds = ws.take<float>(size_t(batch) * h->rows);
        // Both orders are within (n + 80) * 2^-24 * A of the exact sum; the
        // 1.25 margin also covers the rounding of A itself.
        const float factor = 2.5f * static_cast<float>(h->columns + 80u) * 5.9604645e-8f;
        HeadWaveBest best{factor, nullptr, nullptr, nullptr};
        const bool waves = head_wave_best(h);
        const uint32_t wave_count = head_wide_blocks(ctx, h->rows) * 4u;
        if (waves) {
            best.value = ws.take<float>(size_t(batch) * wave_count);
            best.index = ws.take<uint32_t>(size_t(batch) * wave_count);
            best.upper = ws.take<float>(size_t(batch) * wave_count);
        }
        head_logits(ctx, h, inputs, batch, out, bounds, best);
        const HeadView v = view_of(h);
        const auto run = [&](auto kernel) {
            launch(ctx, "head_argmax", kernel, dim3(batch), dim3(kArgmaxThreads), 0, v, inputs,
                   static_cast<const float *>(out), static_cast<const float *>(bounds), factor,
                   static_cast<const float *>(best.value),
                   static_cast<const uint32_t *>(best.index),
                   static_cast<const float *>(best.upper), wave_count, argmax);
        };
        switch (ctx->isa_lanes) {
        case 1:
            waves ? run(k_head_argmax<1, false, true>) : run(k_head_argmax<1, false, false>);
            break;
        case 8:
            waves ? run(k_head_argmax<8, false, true>) : run(k_head_argmax<8, false, false>);
            break;
        default:
            waves ? run(k_head_argmax<16, true, true>) : run(k_head_argmax<16, true, false>);
            break;
        }
    });
}

}  // extern "C"
