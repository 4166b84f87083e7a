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

__device__ __forceinline__ bool first_max_before(float a, uint32_t ia, float b, uint32_t ib) {
    return a == b ? ia < ib : a > b;
}

// Per-wave summaries the 2048-column MFMA head leaves for the certified arg-max,
// [batch][waves] each: the wave's first maximum logit and its row
// (0xFFFFFFFF for a wave with no rows), and the largest
// fmaf(factor, bound, logit) over the wave's rows.
struct HeadWaveBest {
    float factor;
    float *value;
    uint32_t *index;
    float *upper;
};

// ---- the 2048-column head on the bf16 MFMA ----------------------------------
//
// logit[t][r] = sum over the 32 groups g of 64 columns of scale[r][g] *
// sum_{k in g} (u[r][k] - 16) x[t][k]. A wave takes 16-row tiles; per group a
// tile is two v_mfma_f32_16x16x32_bf16 whose operands are exact:
//   A[r][slot] = 1 + u * delta, bf16 0x3F80 | u << 2 (delta 1/32, the low
//                half of a dword) or 0x3F80 | u << 1 (delta 1/64, the high half)
//   B[slot][4t + p] = piece p of x[t][k] / delta, three bf16 pieces (p 0-2)
//                that sum to it exactly (8 + 8 + 8 significant bits)
// so column 4t + p accumulates sum_k a_k b_k = sum_k b_k + sum_k u_k x_k in
// fp32 over exact products. The accumulator starts at -K[g][4t + p] with K =
// sum_k b_k (1 + 16 delta_k), so the pieces' sum is sum_k (u_k - 16) x_k;
// column 4t + 3 has B = 0 and K = -16 sum_k |x_k|, and accumulates the row's
// bound sum 16 sum_g scale sum|x| of the certified arg-max. The group sums
// are scaled and added per row in fp32; the pieces of a row add in the order
// (0 + 1) + 2. Each rounding is relative to sums of |u x|, |x| / delta, well
// inside the arg-max bound's (n + 80) 2^-24 16 scale sum|x| (x 2.5).
//
// A lane holds 16 codes of its row per group (columns 16q .. 16q + 15, q =
// lane / 16): its three aligned dwords, shifted by 16 bits for odd q, hold
// code c at bits 5c; pairs (c, c + 3) and (13, 14) each take one funnel shift
// and one and-or into the two bf16 mantissas of an A dword. The B fragments,
// K and each tile's scales live in LDS; the B fragments are built by every
// block from x while its first tile's codes load.
constexpr uint32_t kHmWaves = 8;
constexpr uint32_t kHmThreads = 64 * kHmWaves;
constexpr uint32_t kHmGroups = 32;
constexpr uint32_t kHmTile = 16;    // rows per tile
constexpr uint32_t kHmTokens = 4;   // tokens per pass: 4 columns each
constexpr uint32_t kHmChunk = 8;    // groups per load chunk (a quarter tile)

typedef __bf16 hm_bf16x8 __attribute__((ext_vector_type(8)));
typedef float hm_f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t hm_u32x4 __attribute__((ext_vector_type(4)));

// A quarter tile (8 groups of 16 rows: 16 row pieces of 320 bytes) as the
// wave stages it: rows kHmStagePitch bytes apart.
constexpr uint32_t kHmPieceBytes = kHmChunk * 40u;          // 320
constexpr uint32_t kHmStagePitch = kHmPieceBytes + 16u;      // 336: rows start on other banks
constexpr uint32_t kHmRawLoads = kHmTile * kHmPieceBytes / (16u * 64u);  // 5 16-byte loads a lane

struct HeadMfmaLds {
    hm_u32x4 b[kHmGroups][2][4][16];  // B fragment of (group, MFMA, lane / 16, column)
    float c[kHmGroups][16];           // -K of (group, column), the accumulator's start
    union {
        float part[kHmGroups][16][8];               // K's partial sums while the tables build
        uint16_t scale[kHmWaves][kHmGroups][kHmTile];  // each wave's tile scales (f16 bits)
    } u;
    // each wave's staging of the quarter tile it sums (the coalesced loads'
    // bytes, read back in the A layout)
    uint32_t stage[kHmWaves][kHmTile * kHmStagePitch / 4];
};

// The two codes of each A dword, by MFMA and dword: (low half, high half).
__device__ __forceinline__ uint32_t hm_code(uint32_t i, uint32_t d, uint32_t h) {
    // MFMA 0: (0,3) (1,4) (2,5) (6,9); MFMA 1: (7,10) (8,11) (12,15) (13,14)
    constexpr uint8_t lo[8] = {0, 1, 2, 6, 7, 8, 12, 13};
    constexpr uint8_t hi[8] = {3, 4, 5, 9, 10, 11, 15, 14};
    return h == 0 ? lo[4 * i + d] : hi[4 * i + d];
}

// bf16 bits of piece p of v (p < 3): v = hi + mid + lo exactly, each the
// leading 8 significant bits of what is left.
__device__ __forceinline__ uint32_t hm_piece(float v, uint32_t p) {
    const uint32_t bits = __float_as_uint(v);
    const float hi = __uint_as_float(bits & 0xFFFF0000u);
    const float r1 = v - hi;
    const float mid = __uint_as_float(__float_as_uint(r1) & 0xFFFF0000u);
    const float r2 = r1 - mid;
    const float pick = p == 0 ? hi : (p == 1 ? mid : r2);
    return __float_as_uint(pick) >> 16;
}

// The 16 codes of (row, group g, quarter q) as the 8 A dwords of the
// group's two MFMAs, from the lane's three dwords w (already shifted so
// that code c sits at bits 5c).
__device__ __forceinline__ void hm_decode(uint32_t w0, uint32_t w1, uint32_t w2, hm_u32x4 &a0,
                                          hm_u32x4 &a1) {
    constexpr uint32_t M = 0x003E007Cu, ONE = 0x3F803F80u;
    const auto and_or = [](uint32_t v, uint32_t m, uint32_t o) { return (v & m) | o; };
    a0.x = and_or(w0 << 2, M, ONE);
    a0.y = and_or(w0 >> 3, M, ONE);
    a0.z = and_or(w0 >> 8, M, ONE);
    a0.w = and_or(__builtin_amdgcn_alignbit(w1, w0, 28), M, ONE);
    a1.x = and_or(w1 >> 1, M, ONE);
    a1.y = and_or(w1 >> 6, M, ONE);
    a1.z = and_or(__builtin_amdgcn_alignbit(w2, w1, 26), M, ONE);
    const uint32_t high = and_or(__builtin_amdgcn_alignbit(w2, w1, 21), 0x003E0000u, ONE);
    a1.w = and_or(__builtin_amdgcn_alignbit(w2, w1, 31), 0x7Cu, high);
}

// LDS reads at a byte address the compiler keeps in one VGPR per array,
// the per-group part an immediate offset (all under 64 KiB past the base).
typedef __attribute__((address_space(3))) const hm_u32x4 *hm_lds_u32x4;
typedef __attribute__((address_space(3))) const hm_f32x4 *hm_lds_f32x4;
__device__ __forceinline__ hm_u32x4 hm_lds_u(uint32_t address) {
    return *reinterpret_cast<hm_lds_u32x4>(static_cast<size_t>(address));
}
__device__ __forceinline__ float hm_lds_f1(uint32_t address) {
    return *reinterpret_cast<__attribute__((address_space(3))) const float *>(static_cast<size_t>(address));
}
typedef uint32_t hm_u32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ hm_u32x2 hm_lds_u2(uint32_t address) {
    return *reinterpret_cast<__attribute__((address_space(3))) const hm_u32x2 *>(static_cast<size_t>(address));
}
__device__ __forceinline__ hm_f32x4 hm_lds_f(uint32_t address) {
    return *reinterpret_cast<hm_lds_f32x4>(static_cast<size_t>(address));
}
__device__ __forceinline__ uint32_t hm_opaque(uint32_t v) {
    asm volatile("" : "+v"(v));
    return v;
}

__device__ __forceinline__ hm_f32x4 hm_mfma(hm_u32x4 a, hm_u32x4 b, hm_f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(hm_bf16x8, a),
                                                    __builtin_bit_cast(hm_bf16x8, b), c, 0, 0, 0);
}

// The B fragments and accumulator starts of tokens t0 .. t0 + 3 (zero past
// `batch`) into LDS; ends with a block barrier.
__device__ void hm_build_tables(HeadMfmaLds &L, const float *__restrict__ x, uint32_t t0,
                                uint32_t batch) {
#pragma clang fp contract(off)
    // thread (group, quarter, token): per MFMA the fragments of its three
    // pieces and the bound column, and their four partial sums of K
    for (uint32_t e = threadIdx.x; e < kHmGroups * 4 * kHmTokens; e += kHmThreads) {
        const uint32_t t = e % kHmTokens, q = (e / kHmTokens) % 4, g = e / 16;
        const bool live = t0 + t < batch;
        const float *xt = x + static_cast<size_t>(live ? t0 + t : 0) * 2048u + 64u * g + 16u * q;
#pragma unroll
        for (uint32_t i = 0; i < 2; ++i) {
            hm_u32x4 frag[3];
            float sum[3] = {0.0f, 0.0f, 0.0f}, bound = 0.0f;
#pragma unroll
            for (uint32_t d = 0; d < 4; ++d) {
                uint32_t half[3][2];
#pragma unroll
                for (uint32_t h = 0; h < 2; ++h) {
                    const float xv = live ? xt[hm_code(i, d, h)] : 0.0f;
                    const float v = xv * (h == 0 ? 32.0f : 64.0f);  // exact
                    const float f = h == 0 ? 1.5f : 1.25f;           // 1 + 16 delta
#pragma unroll
                    for (uint32_t p = 0; p < 3; ++p) {
                        half[p][h] = hm_piece(v, p);
                        sum[p] += __uint_as_float(half[p][h] << 16) * f;
                    }
                    bound += fabsf(xv);
                }
#pragma unroll
                for (uint32_t p = 0; p < 3; ++p) {
                    frag[p][d] = half[p][0] | (half[p][1] << 16);
                }
            }
#pragma unroll
            for (uint32_t p = 0; p < 3; ++p) {
                L.b[g][i][q][4 * t + p] = frag[p];
                L.u.part[g][4 * t + p][4 * i + q] = sum[p];
            }
            L.b[g][i][q][4 * t + 3] = hm_u32x4{0u, 0u, 0u, 0u};
            L.u.part[g][4 * t + 3][4 * i + q] = -16.0f * bound;
        }
    }
    __syncthreads();
    for (uint32_t e = threadIdx.x; e < kHmGroups * 16; e += kHmThreads) {
        const uint32_t g = e / 16, n = e % 16;
        float k = 0.0f;
#pragma unroll
        for (uint32_t j = 0; j < 8; ++j) {
            k += L.u.part[g][n][j];
        }
        L.c[g][n] = -k;
    }
    __syncthreads();
}

// The lane's three dwords of (row, group g) for its quarter q: aligned, from
// the 10-byte stretch's start (even q) or two bytes before it (odd q).
__device__ __forceinline__ void hm_load(const uint8_t *__restrict__ row_codes, uint32_t g,
                                        uint32_t q, uint32_t (&w)[3]) {
    const uint32_t *src = reinterpret_cast<const uint32_t *>(
        row_codes + 40u * g + 10u * q - 2u * (q & 1u));
    // plain loads: the four quarters of a row's 40 bytes and the next
    // groups' share cache lines, which nontemporal loads would fetch again
    // (2048-column head, loads alone: 75.6 us nontemporal, 47.0 us plain)
#pragma unroll
    for (uint32_t i = 0; i < 3; ++i) {
        w[i] = src[i];
    }
}

// Wave w takes tiles w, w + waves, ...; per pass of four tokens it leaves
// the logits and, with BOUNDS, the bounds and its per-token summary
// (HeadWaveBest) for the arg-max. With COALESCED (16-byte aligned codes) a
// quarter tile is loaded as 16-byte pieces in row order, each load
// instruction of the wave covering about 1 KiB of consecutive bytes, and
// staged in the wave's LDS before its lanes read their three dwords of each
// group; otherwise each lane loads its three dwords of every group itself
// (16 rows' 40-byte groups a load instruction). Both give the same bits.
template <bool BOUNDS, bool COALESCED>
__global__ __launch_bounds__(kHmThreads) void k_head_mfma(
    const uint8_t *__restrict__ packed, const uint16_t *__restrict__ scales, uint32_t rows,
    const float *__restrict__ x, uint32_t batch, float *__restrict__ logits,
    float *__restrict__ bounds, HeadWaveBest best) {
#pragma clang fp contract(off)
    extern __shared__ __align__(16) unsigned char hm_raw[];
    HeadMfmaLds &L = *reinterpret_cast<HeadMfmaLds *>(hm_raw);
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t wave_global = blockIdx.x * kHmWaves + wave;
    const uint32_t wave_count = gridDim.x * kHmWaves;
    const uint32_t tiles = (rows + kHmTile - 1u) / kHmTile;
    const uint32_t q = lane / 16u, i_row = lane % 16u;
    const uint32_t n = lane % 16u, p = lane % 4u, t_lane = n / 4u;
    const uint32_t shift = 16u * (q & 1u);
    uint16_t *sc = &L.u.scale[wave][0][0];
    // LDS byte addresses of this lane's B fragment, accumulator start and
    // scales for group 0; group g adds g * 2048, g * 256, g * 64
    const uint32_t lds0 = static_cast<uint32_t>(
        (uintptr_t)(__attribute__((address_space(3))) unsigned char *)hm_raw);
    const uint32_t b_at = hm_opaque(lds0 + static_cast<uint32_t>(offsetof(HeadMfmaLds, b)) +
                                    q * 256u + n * 16u);
    const uint32_t c_at = hm_opaque(lds0 + static_cast<uint32_t>(offsetof(HeadMfmaLds, c)) + n * 4u);
    const uint32_t s_at = hm_opaque(lds0 + static_cast<uint32_t>(offsetof(HeadMfmaLds, u)) +
                                    (wave * kHmGroups * kHmTile + 4u * q) * 2u);

    for (uint32_t t0 = 0; t0 < batch; t0 += kHmTokens) {
        float best_v = -INFINITY, upper = -INFINITY;
        uint32_t best_i = 0xFFFFFFFFu;
        // a ring of the four quarter-tile chunks: after a chunk is summed its
        // slot loads the same chunk of the wave's next tile, three chunks of
        // codes (18 KiB a wave) in flight while one is summed
        uint32_t w[COALESCED ? 1 : 4][kHmChunk][3];
        hm_u32x4 raw[COALESCED ? 4 : 1][kHmRawLoads];
        hm_u32x4 sreg = hm_u32x4{0u, 0u, 0u, 0u};
        uint32_t tile = wave_global;
        // the first tile's codes and scales load while the tables build
        const auto row_of = [&](uint32_t t, uint32_t r) {
            const uint32_t row = t < tiles ? t * kHmTile + r : rows;
            return row < rows ? row : rows - 1u;
        };
        const auto load_chunk = [&](uint32_t t, uint32_t part, uint32_t (&dst)[kHmChunk][3]) {
            const uint8_t *rc = packed + static_cast<size_t>(row_of(t, i_row)) * 1280u;
#pragma unroll
            for (uint32_t g = 0; g < kHmChunk; ++g) {
                hm_load(rc, kHmChunk * part + g, q, dst[g]);
            }
        };
        // load k of a lane: piece e = 64 k + lane of the quarter tile, row
        // e / 20, bytes 16 (e % 20) .. + 15 of that row's 320
        const auto load_raw = [&](uint32_t t, uint32_t part, hm_u32x4 (&dst)[kHmRawLoads]) {
#pragma unroll
            for (uint32_t k = 0; k < kHmRawLoads; ++k) {
                const uint32_t e = 64u * k + lane;
                const uint32_t r = e / 20u, piece = e % 20u;
                dst[k] = *reinterpret_cast<const hm_u32x4 *>(
                    packed + static_cast<size_t>(row_of(t, r)) * 1280u + kHmPieceBytes * part + 16u * piece);
            }
        };
        uint32_t *stage = &L.stage[wave][0];
        // the staged quarter tile back as the lane's three dwords of each of
        // its eight groups (the bytes hm_load reads from memory)
        const auto unstage = [&](const hm_u32x4 (&src)[kHmRawLoads], uint32_t (&dst)[kHmChunk][3]) {
#pragma unroll
            for (uint32_t k = 0; k < kHmRawLoads; ++k) {
                const uint32_t e = 64u * k + lane;
                const uint32_t r = e / 20u, piece = e % 20u;
                *reinterpret_cast<hm_u32x4 *>(stage + (r * kHmStagePitch + 16u * piece) / 4u) = src[k];
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            const uint32_t *row = stage + (i_row * kHmStagePitch) / 4u;
#pragma unroll
            for (uint32_t g = 0; g < kHmChunk; ++g) {
                const uint32_t *at = row + (40u * g + 10u * q - 2u * (q & 1u)) / 4u;
#pragma unroll
                for (uint32_t i = 0; i < 3; ++i) {
                    dst[g][i] = at[i];
                }
            }
            // every lane's reads end before the next quarter is staged
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        };
        const auto load_scales = [&](uint32_t t) {
            // lane l: row l / 4, groups 8 (l % 4) .. + 7
            const hm_u32x4 *src = reinterpret_cast<const hm_u32x4 *>(
                scales + static_cast<size_t>(row_of(t, lane / 4u)) * kHmGroups + 8u * (lane % 4u));
            sreg = *src;
        };
        // issued in the order the tile loop issues them (first quarter,
        // scales, the other quarters), so that the loop's counted waits hold
        // on entry as on every later tile; in another order the compiler can
        // only wait for every load at the top of each tile
        if (tile < tiles) {
            if constexpr (COALESCED) {
                load_raw(tile, 0, raw[0]);
                load_scales(tile);
                __builtin_amdgcn_sched_barrier(0);
                load_raw(tile, 1, raw[1]);
                __builtin_amdgcn_sched_barrier(0);
                load_raw(tile, 2, raw[2]);
                __builtin_amdgcn_sched_barrier(0);
                load_raw(tile, 3, raw[3]);
            } else {
                load_chunk(tile, 0, w[0]);
                load_scales(tile);
                __builtin_amdgcn_sched_barrier(0);
                load_chunk(tile, 1, w[1]);
                __builtin_amdgcn_sched_barrier(0);
                load_chunk(tile, 2, w[2]);
                __builtin_amdgcn_sched_barrier(0);
                load_chunk(tile, 3, w[3]);
            }
        }
        if (t0 > 0) {
            __syncthreads();  // the previous pass's readers are done with the tables
        }
        hm_build_tables(L, x, t0, batch);
        for (; tile < tiles; tile += wave_count) {
            // this tile's scales, transposed: sc[g][row] as f16 bits
#pragma unroll
            for (uint32_t e = 0; e < 8; ++e) {
                const uint32_t bits = sreg[e / 2] >> (16u * (e % 2u));
                sc[(8u * (lane % 4u) + e) * kHmTile + lane / 4u] = static_cast<uint16_t>(bits & 0xFFFFu);
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            hm_f32x4 out = hm_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            const auto run_chunk = [&](uint32_t part, const uint32_t (&src)[kHmChunk][3]) {
#pragma unroll
                for (uint32_t j = 0; j < kHmChunk; ++j) {
                    const uint32_t g = kHmChunk * part + j;
                    const uint32_t w0 = __builtin_amdgcn_alignbit(src[j][1], src[j][0], shift);
                    const uint32_t w1 = __builtin_amdgcn_alignbit(src[j][2], src[j][1], shift);
                    const uint32_t w2 = src[j][2] >> shift;
                    hm_u32x4 a0, a1;
                    hm_decode(w0, w1, w2, a0, a1);
                    // the group's accumulator start is one float per column
                    // (the same for the four rows a lane holds)
                    const float c0 = hm_lds_f1(c_at + g * 64u);
                    hm_f32x4 acc = hm_mfma(a0, hm_lds_u(b_at + g * 2048u), hm_f32x4{c0, c0, c0, c0});
                    acc = hm_mfma(a1, hm_lds_u(b_at + g * 2048u + 1024u), acc);
                    const hm_u32x2 sb = hm_lds_u2(s_at + g * 32u);
                    const hm_f32x4 s = hm_f32x4{half_bits_to_float(sb.x & 0xFFFFu), half_bits_to_float(sb.x >> 16),
                                                half_bits_to_float(sb.y & 0xFFFFu), half_bits_to_float(sb.y >> 16)};
                    out.x = fmaf(s.x, acc.x, out.x);
                    out.y = fmaf(s.y, acc.y, out.y);
                    out.z = fmaf(s.z, acc.z, out.z);
                    out.w = fmaf(s.w, acc.w, out.w);
                    // the sums complete here, group by group: left to the
                    // compiler, they sink past the next loads and every
                    // group's accumulator and scales stay live (and spill)
                    asm volatile("" : "+v"(out.x), "+v"(out.y), "+v"(out.z), "+v"(out.w));
                }
            };
            // past the last tile the loads read the last row again (row_of
            // clamps), unused: no branch breaks the in-order load counts
            const uint32_t next = tile + wave_count;
            if constexpr (COALESCED) {
                // each quarter staged and read back, its registers then
                // reloaded with the next tile's quarter
                unstage(raw[0], w[0]);
                load_raw(next, 0, raw[0]);
                load_scales(next);
                run_chunk(0, w[0]);
                unstage(raw[1], w[0]);
                load_raw(next, 1, raw[1]);
                run_chunk(1, w[0]);
                unstage(raw[2], w[0]);
                load_raw(next, 2, raw[2]);
                run_chunk(2, w[0]);
                unstage(raw[3], w[0]);
                load_raw(next, 3, raw[3]);
                run_chunk(3, w[0]);
            } else {
                run_chunk(0, w[0]);
                load_chunk(next, 0, w[0]);
                load_scales(next);
                run_chunk(1, w[1]);
                load_chunk(next, 1, w[1]);
                run_chunk(2, w[2]);
                load_chunk(next, 2, w[2]);
                run_chunk(3, w[3]);
                load_chunk(next, 3, w[3]);
            }
            // every lane's reads of this tile's scales end before the next
            // tile's are written
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            // lane p = 0 of a quad: logit (piece 0 + piece 1) + piece 2, bound piece 3
            for (uint32_t j = 0; j < 4; ++j) {
                const float v = out[j];
                const float v1 = __uint_as_float(static_cast<uint32_t>(
                    __builtin_amdgcn_mov_dpp(static_cast<int>(__float_as_uint(v)), 0x39, 0xF, 0xF, true)));
                const float v2 = __uint_as_float(static_cast<uint32_t>(
                    __builtin_amdgcn_mov_dpp(static_cast<int>(__float_as_uint(v)), 0x4E, 0xF, 0xF, true)));
                const float v3 = __uint_as_float(static_cast<uint32_t>(
                    __builtin_amdgcn_mov_dpp(static_cast<int>(__float_as_uint(v)), 0x93, 0xF, 0xF, true)));
                const float total = (v + v1) + v2;
                const uint32_t row = tile * kHmTile + 4u * q + j;
                const uint32_t t = t0 + t_lane;
                if (p == 0 && row < rows && t < batch) {
                    logits[static_cast<size_t>(t) * rows + row] = total;
                    if constexpr (BOUNDS) {
                        bounds[static_cast<size_t>(t) * rows + row] = v3;
                        const float up = fmaf(best.factor, v3, total);
                        upper = up > upper ? up : upper;
                        if (best_i == 0xFFFFFFFFu || first_max_before(total, row, best_v, best_i)) {
                            best_v = total;
                            best_i = row;
                        }
                    }
                }
            }
        }
        if constexpr (BOUNDS) {
            // the wave's summary per token: over the four quarters' lanes of
            // column 4t (lanes 4t + 16 k)
#pragma unroll
            for (int off = 16; off <= 32; off <<= 1) {
                const float ov = __shfl_xor(best_v, off);
                const uint32_t oi = static_cast<uint32_t>(__shfl_xor(static_cast<int>(best_i), off));
                const float ou = __shfl_xor(upper, off);
                upper = ou > upper ? ou : upper;
                if (oi != 0xFFFFFFFFu && (best_i == 0xFFFFFFFFu || first_max_before(ov, oi, best_v, best_i))) {
                    best_v = ov;
                    best_i = oi;
                }
            }
            const uint32_t t = t0 + t_lane;
            if (best.value != nullptr && lane < 16u && p == 0 && t < batch) {
                const size_t at = static_cast<size_t>(t) * wave_count + wave_global;
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
            // wave w's rows: 16-row tiles w, w + wave_count, ...
            const uint32_t span = ceil_div_device(ceil_div_device(h.rows, kHmTile), wave_count) * kHmTile;
            for (uint32_t k = threadIdx.x; k < listed * span; k += kArgmaxThreads) {
                const uint32_t at = k % span;
                const uint32_t r = (wave_list[k / span] + (at / kHmTile) * wave_count) * kHmTile +
                                   at % kHmTile;
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

// Blocks of the 2048-column MFMA head: one per CU (its LDS tables), fewer
// when the tiles do not need them.
uint32_t head_wide_blocks(const adi_hip_context *ctx, uint32_t rows) {
    return std::min<uint32_t>(ceil_div(ceil_div(rows, kHmTile), kHmWaves),
                              static_cast<uint32_t>(ctx->cu_count));
}

// Waves of that launch: the per-wave arg-max summaries are [batch][waves].
uint32_t head_wave_count(const adi_hip_context *ctx, uint32_t rows) {
    return head_wide_blocks(ctx, rows) * kHmWaves;
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
            // 16-byte aligned codes (every row is 1280 bytes) take the
            // coalesced loads
            const bool coalesced = aligned_to(h->packed, 16);
            const auto kernel = bounds != nullptr
                                    ? (coalesced ? k_head_mfma<true, true> : k_head_mfma<true, false>)
                                    : (coalesced ? k_head_mfma<false, true> : k_head_mfma<false, false>);
            static const bool ready =
                set_lds_limit(reinterpret_cast<const void *>(&k_head_mfma<true, true>), sizeof(HeadMfmaLds)) &&
                set_lds_limit(reinterpret_cast<const void *>(&k_head_mfma<false, true>), sizeof(HeadMfmaLds)) &&
                set_lds_limit(reinterpret_cast<const void *>(&k_head_mfma<true, false>), sizeof(HeadMfmaLds)) &&
                set_lds_limit(reinterpret_cast<const void *>(&k_head_mfma<false, false>), sizeof(HeadMfmaLds));
            (void)ready;
            launch(ctx, "head_mfma", kernel, dim3(wide), dim3(kHmThreads), sizeof(HeadMfmaLds),
                   h->packed, h->group_scale_f16, h->rows, x, batch, logits, bounds, best);
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
    const size_t waves = head_wave_count(ctx, h->rows);
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
        const uint32_t wave_count = head_wave_count(ctx, h->rows);
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
