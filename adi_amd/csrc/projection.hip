// projection.hip -- decode-GEMV kernels for the expert (K=1.5/V=8) and
// non-expert (K=4/V=2) trellis codecs, the Hadamard prologue/epilogue around
// them, and the Backend entry points expert_matvec/matmul and
// ne_matvec/matmul.
//
// Data flow of one projection y = W x (src/kernels.cpp:385-800):
//   prologue  x_hat = H_C(su * x)                 one block per vector, LDS
//   gemv      Z[r] = sum_tiles decoded(tile) . x_hat   codes read once, decoded
//                                                  in registers
//   epilogue  y = sv * H_R(sum_splits Z)           one block per vector, LDS
//
// GEMV work split: a 256-thread block owns 64 consecutive tiles of a matrix
// (tile-row-major order), a wave 16 of them, and each tile is shared by four
// lanes that own four of its sixteen rows ("quads"). A lane loads its quad's
// slice of the packed stream with one coalesced vector load, decodes the
// states of its four rows in registers, and multiplies them with the x_hat
// values of the tile column. Rows are summed over the tiles of a tile row
// with wave shuffles and, across waves, through LDS. With more than 64 tile
// columns each block writes its own partial (split); the epilogue adds them.
#include "projection.hpp"

namespace adi_hip {
namespace {

// ---- shared decode of one quad (four rows of a tile) ------------------------

// Expert: four rows = 8 states = bits [96q, 96q + 112) of the tile's 384-bit
// stream, i.e. words 6q..6q+5 of this lane plus word 0 of the next quad
// (taken from the neighbouring lane; quad 3 wraps to word 0 of the tile,
// src/expert_trellis.hpp:79-80). All four lanes of a tile must call this.
__device__ __forceinline__ void load_expert_quad(const uint16_t *trellis, uint32_t tile,
                                                 uint32_t quad, bool valid, uint32_t lane,
                                                 uint32_t (&d)[4]) {
    d[0] = d[1] = d[2] = 0u;
    if (valid) {
        const uint32_t *src = reinterpret_cast<const uint32_t *>(trellis) +
                              static_cast<size_t>(tile) * 12u + quad * 3u;
        d[0] = __builtin_nontemporal_load(src);
        d[1] = __builtin_nontemporal_load(src + 1);
        d[2] = __builtin_nontemporal_load(src + 2);
    }
    const int partner = quad == 3u ? static_cast<int>(lane) - 3 : static_cast<int>(lane) + 1;
    d[3] = static_cast<uint32_t>(__shfl(static_cast<int>(d[0]), partner)) & 0xFFFFu;
}

// The eight decoded states of a quad, each as 8 f16 lattice values (one
// reachable codebook row, component 0 negated by bit 15 of the state hash).
__device__ __forceinline__ void decode_expert_quad(const uint32_t (&d)[4], const uint4 *book,
                                                   uint4 (&e)[8]) {
#define ADI_EXPERT_STATE(K)                                            \
    {                                                                  \
        const uint32_t p = state_product(stream_window<12 * K>(d));    \
        e[K] = book[(p >> 1) & 0x3FFFu];                               \
        e[K].x ^= p & 0x8000u;                                         \
    }
    ADI_EXPERT_STATE(0) ADI_EXPERT_STATE(1) ADI_EXPERT_STATE(2) ADI_EXPERT_STATE(3)
    ADI_EXPERT_STATE(4) ADI_EXPERT_STATE(5) ADI_EXPERT_STATE(6) ADI_EXPERT_STATE(7)
#undef ADI_EXPERT_STATE
}

// NE: four rows = 32 states = bytes [32q, 32q + 34) of the tile's 1024-bit
// stream: words 16q..16q+15 plus word 0 of the next quad (quad 3 wraps,
// src/ne_trellis.hpp:196-200).
__device__ __forceinline__ void load_ne_quad(const uint16_t *trellis, uint32_t tile, uint32_t quad,
                                             bool valid, uint32_t lane, uint32_t (&d)[9]) {
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    u32x4 lo = {0u, 0u, 0u, 0u}, hi = {0u, 0u, 0u, 0u};
    if (valid) {
        const u32x4 *src = reinterpret_cast<const u32x4 *>(trellis) +
                           static_cast<size_t>(tile) * 8u + quad * 2u;
        lo = __builtin_nontemporal_load(src);
        hi = __builtin_nontemporal_load(src + 1);
    }
    d[0] = lo.x; d[1] = lo.y; d[2] = lo.z; d[3] = lo.w;
    d[4] = hi.x; d[5] = hi.y; d[6] = hi.z; d[7] = hi.w;
    const int partner = quad == 3u ? static_cast<int>(lane) - 3 : static_cast<int>(lane) + 1;
    d[8] = static_cast<uint32_t>(__shfl(static_cast<int>(d[0]), partner)) & 0xFFFFu;
}

// Signed-table index of each of the 32 states: (s(s+1) >> 6) & 0x3FF
// (src/codec_cache.cpp:85-115).
__device__ __forceinline__ void decode_ne_quad(const uint32_t (&d)[9], uint32_t (&idx)[32]) {
#define ADI_NE_STATE(K) idx[K] = (state_product(stream_window<8 * K>(d)) >> 6) & 0x3FFu;
    ADI_NE_STATE(0) ADI_NE_STATE(1) ADI_NE_STATE(2) ADI_NE_STATE(3)
    ADI_NE_STATE(4) ADI_NE_STATE(5) ADI_NE_STATE(6) ADI_NE_STATE(7)
    ADI_NE_STATE(8) ADI_NE_STATE(9) ADI_NE_STATE(10) ADI_NE_STATE(11)
    ADI_NE_STATE(12) ADI_NE_STATE(13) ADI_NE_STATE(14) ADI_NE_STATE(15)
    ADI_NE_STATE(16) ADI_NE_STATE(17) ADI_NE_STATE(18) ADI_NE_STATE(19)
    ADI_NE_STATE(20) ADI_NE_STATE(21) ADI_NE_STATE(22) ADI_NE_STATE(23)
    ADI_NE_STATE(24) ADI_NE_STATE(25) ADI_NE_STATE(26) ADI_NE_STATE(27)
    ADI_NE_STATE(28) ADI_NE_STATE(29) ADI_NE_STATE(30) ADI_NE_STATE(31)
#undef ADI_NE_STATE
}

// Dense dump of the decoded weights through the same loads and decode as
// the GEMVs: expert values V[row][column] (before gamma), NE values
// V * Wscale rounded to fp32 (src/kernels.cpp:673-683).
__global__ __launch_bounds__(256) void k_expert_decode(const uint16_t *trellis, const void *codebook,
                                                       uint32_t rows, uint32_t columns,
                                                       float *out) {
    const uint32_t lane = threadIdx.x & 63u, quad = lane & 3u;
    const uint32_t tile_columns = columns / kTile;
    const uint32_t tiles = (rows / kTile) * tile_columns;
    const uint32_t tile = blockIdx.x * 64u + (threadIdx.x >> 6) * 16u + (lane >> 2);
    const bool valid = tile < tiles;
    uint32_t d[4];
    load_expert_quad(trellis, tile, quad, valid, lane, d);
    uint4 e[8];
    decode_expert_quad(d, static_cast<const uint4 *>(codebook), e);
    if (!valid) {
        return;
    }
    const uint32_t tr = tile / tile_columns, tc = tile % tile_columns;
    for (int k = 0; k < 8; ++k) {
        const uint32_t row = tr * kTile + quad * 4u + k / 2;
        float *dst = out + static_cast<size_t>(row) * columns + tc * kTile + (k & 1) * 8;
        const uint32_t w[4] = {e[k].x, e[k].y, e[k].z, e[k].w};
        for (int c = 0; c < 4; ++c) {
            const float2 v = half2_bits_to_float2(w[c]);
            dst[2 * c] = v.x;
            dst[2 * c + 1] = v.y;
        }
    }
}

__global__ __launch_bounds__(256) void k_ne_decode(const uint16_t *trellis, const void *codebook,
                                                   float weight_scale, uint32_t rows,
                                                   uint32_t columns, float *out) {
#pragma clang fp contract(off)
    const uint32_t lane = threadIdx.x & 63u, quad = lane & 3u;
    const uint32_t tile_columns = columns / kTile;
    const uint32_t tiles = (rows / kTile) * tile_columns;
    const uint32_t tile = blockIdx.x * 64u + (threadIdx.x >> 6) * 16u + (lane >> 2);
    const bool valid = tile < tiles;
    uint32_t d[9];
    load_ne_quad(trellis, tile, quad, valid, lane, d);
    uint32_t idx[32];
    decode_ne_quad(d, idx);
    if (!valid) {
        return;
    }
    const uint32_t *book = static_cast<const uint32_t *>(codebook);
    const uint32_t tr = tile / tile_columns, tc = tile % tile_columns;
    for (int k = 0; k < 32; ++k) {
        const uint32_t row = tr * kTile + quad * 4u + k / 8;
        const float2 v = half2_bits_to_float2(book[idx[k]]);
        float *dst = out + static_cast<size_t>(row) * columns + tc * kTile + (k % 8) * 2;
        dst[0] = v.x * weight_scale;
        dst[1] = v.y * weight_scale;
    }
}

// ---- Hadamard prologue / epilogue ----------------------------------------

template <typename Scale>
__device__ __forceinline__ float scale_value(Scale s);
template <>
__device__ __forceinline__ float scale_value<uint16_t>(uint16_t s) {
    return half_bits_to_float(s);
}
template <>
__device__ __forceinline__ float scale_value<int8_t>(int8_t s) {
    return static_cast<float>(s);
}

template <typename Scale>
__global__ __launch_bounds__(256) void k_prologue(
    const float *__restrict__ x, uint32_t n, const Scale *__restrict__ su,
    uint32_t su_stride, const uint32_t *__restrict__ source_row,
    const uint32_t *__restrict__ matrix_index, float scale,
    float *__restrict__ out) {
#pragma clang fp contract(off)
    extern __shared__ float v[];
    const uint32_t vec = blockIdx.x;
    const uint32_t src = source_row != nullptr ? source_row[vec] : vec;
    const uint32_t mat = matrix_index != nullptr ? matrix_index[vec] : 0u;
    const Scale *s = su + static_cast<size_t>(mat) * su_stride;
    const float *row = x + static_cast<size_t>(src) * n;
    for (uint32_t k = threadIdx.x; k < n; k += blockDim.x) {
        v[k] = row[k] * scale_value<Scale>(s[k]);
    }
    block_hadamard(v, n, scale);
    float *dst = out + static_cast<size_t>(vec) * n;
    for (uint32_t k = threadIdx.x; k < n; k += blockDim.x) {
        dst[k] = v[k];
    }
}

template <typename Scale>
__global__ __launch_bounds__(256) void k_epilogue(
    const float *__restrict__ z, uint32_t splits, size_t split_stride, uint32_t n,
    const Scale *__restrict__ sv, uint32_t sv_stride,
    const uint32_t *__restrict__ matrix_index, float scale,
    float *__restrict__ out) {
#pragma clang fp contract(off)
    extern __shared__ float v[];
    const uint32_t vec = blockIdx.x;
    const uint32_t mat = matrix_index != nullptr ? matrix_index[vec] : 0u;
    const Scale *s = sv + static_cast<size_t>(mat) * sv_stride;
    const float *src = z + static_cast<size_t>(vec) * n;
    for (uint32_t k = threadIdx.x; k < n; k += blockDim.x) {
        float sum = src[k];
        for (uint32_t split = 1; split < splits; ++split) {
            sum += src[split * split_stride + k];
        }
        v[k] = sum;
    }
    block_hadamard(v, n, scale);
    float *dst = out + static_cast<size_t>(vec) * n;
    for (uint32_t k = threadIdx.x; k < n; k += blockDim.x) {
        dst[k] = v[k] * scale_value<Scale>(s[k]);
    }
}

// ---- wave-per-vector prologue / epilogue ---------------------------------

template <typename Scale>
__device__ __forceinline__ float scale_at(const Scale *s, uint32_t k) {
    return scale_value<Scale>(s[k]);
}

// Up to four segments of vectors, one wave each: x_hat = H_n(x[src] * su).
template <int VPL>
__global__ __launch_bounds__(256) void k_prologue_wave(PrologueJobs j) {
#pragma clang fp contract(off)
    const uint32_t lane = threadIdx.x & 63u;
    uint32_t v = blockIdx.x * 4u + (threadIdx.x >> 6);
    uint32_t s = 0;
    while (s < j.segments && v >= j.seg[s].count) {
        v -= j.seg[s].count;
        ++s;
    }
    if (s >= j.segments) {
        return;
    }
    const PrologueSegment &g = j.seg[s];
    const uint32_t n = 64u * VPL;
    const uint32_t src = g.source_row != nullptr ? g.source_row[v] : v;
    const uint32_t mat = g.matrix_index != nullptr ? g.matrix_index[v] : 0u;
    const float *x = g.x + static_cast<size_t>(src) * n + lane;
    float val[VPL];
    if (g.su_f16 != nullptr) {
        const uint16_t *su = g.su_f16 + static_cast<size_t>(mat) * g.su_stride + lane;
#pragma unroll
        for (int i = 0; i < VPL; ++i) {
            val[i] = x[i * 64] * half_bits_to_float(su[i * 64]);
        }
    } else {
        const int8_t *su = g.su_sign + lane;
#pragma unroll
        for (int i = 0; i < VPL; ++i) {
            val[i] = x[i * 64] * static_cast<float>(su[i * 64]);
        }
    }
    wave_hadamard<VPL>(val, j.scale, lane);
    float *out = g.out + static_cast<size_t>(v) * n + lane;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
        out[i * 64] = val[i];
    }
}

// y = sv * H_n(sum over splits of z), one wave per vector.
template <int VPL, typename Scale>
__global__ __launch_bounds__(256) void k_epilogue_wave(
    const float *__restrict__ z, uint32_t splits, size_t split_stride, const Scale *__restrict__ sv,
    uint32_t vectors, float scale, float *__restrict__ out) {
#pragma clang fp contract(off)
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t v = blockIdx.x * 4u + (threadIdx.x >> 6);
    if (v >= vectors) {
        return;
    }
    const uint32_t n = 64u * VPL;
    const float *src = z + static_cast<size_t>(v) * n + lane;
    float val[VPL];
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
        val[i] = src[i * 64];
    }
    for (uint32_t sp = 1; sp < splits; ++sp) {
#pragma unroll
        for (int i = 0; i < VPL; ++i) {
            val[i] += src[sp * split_stride + i * 64];
        }
    }
    wave_hadamard<VPL>(val, scale, lane);
    float *dst = out + static_cast<size_t>(v) * n + lane;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
        dst[i * 64] = val[i] * scale_value<Scale>(sv[i * 64u + lane]);
    }
}

// In-place normalised FWHT of `count` vectors, one wave each (64 <= n <= 4096)
// or one block each.
template <int VPL>
__global__ __launch_bounds__(256) void k_hadamard_wave(float *values, uint32_t count, float scale) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t v = blockIdx.x * 4u + (threadIdx.x >> 6);
    if (v >= count) {
        return;
    }
    float *p = values + static_cast<size_t>(v) * 64u * VPL + lane;
    float val[VPL];
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
        val[i] = p[i * 64];
    }
    wave_hadamard<VPL>(val, scale, lane);
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
        p[i * 64] = val[i];
    }
}

__global__ __launch_bounds__(256) void k_hadamard_block(float *values, uint32_t n, float scale) {
    extern __shared__ float v[];
    float *p = values + static_cast<size_t>(blockIdx.x) * n;
    for (uint32_t k = threadIdx.x; k < n; k += blockDim.x) {
        v[k] = p[k];
    }
    block_hadamard(v, n, scale);
    for (uint32_t k = threadIdx.x; k < n; k += blockDim.x) {
        p[k] = v[k];
    }
}

// ---- cross-tile row reduction shared by both GEMVs -----------------------

// Sums a lane's four row values (per token) over the tiles of its tile row
// and stores them to z. `g` = tiles of one tile row inside a wave
// (min(C_t, 16)), `wpr` = waves covering one tile row (C_t / 16 clamped to
// 1..4).
template <int NT>
__device__ __forceinline__ void reduce_rows_and_store(
    float (&acc)[4][NT], uint32_t lane, uint32_t wave, uint32_t tile,
    uint32_t tile_columns, uint32_t tiles, uint32_t rows, uint32_t tok0,
    uint32_t tok_count, float *z, size_t z_split_stride, float *lds, uint32_t bx) {
    const uint32_t slot = lane >> 2;
    const uint32_t quad = lane & 3u;
    const uint32_t g = tile_columns < 16 ? tile_columns : 16u;
#pragma unroll
    for (uint32_t off = 1; off < 16; off <<= 1) {
        if (off < g) {
#pragma unroll
            for (int m = 0; m < 4; ++m) {
#pragma unroll
                for (int j = 0; j < NT; ++j) {
                    acc[m][j] += __shfl_xor(acc[m][j], static_cast<int>(off * 4u));
                }
            }
        }
    }
    const uint32_t wpr = tile_columns >= 64 ? 4u : (tile_columns >= 16 ? tile_columns / 16u : 1u);
    if (wpr == 1) {
        if ((slot % g) == 0 && tile < tiles) {
            const uint32_t tr = tile / tile_columns;
            const uint32_t split = (tile % tile_columns) / 64u;
#pragma unroll
            for (int j = 0; j < NT; ++j) {
                if (static_cast<uint32_t>(j) < tok_count) {
                    float *dst = z + split * z_split_stride +
                                 static_cast<size_t>(tok0 + j) * rows + tr * kTile + quad * 4u;
#pragma unroll
                    for (int m = 0; m < 4; ++m) {
                        dst[m] = acc[m][j];
                    }
                }
            }
        }
        return;
    }
    // Several waves share a tile row: stage the per-wave sums in LDS.
    __syncthreads();
    if (slot == 0) {
#pragma unroll
        for (int m = 0; m < 4; ++m) {
#pragma unroll
            for (int j = 0; j < NT; ++j) {
                lds[(wave * 16u + quad * 4u + m) * NT + j] = acc[m][j];
            }
        }
    }
    __syncthreads();
    const uint32_t tid = threadIdx.x;
    const uint32_t groups = 4u / wpr;  // tile rows in this block
    if (tid < groups * 16u * NT) {
        const uint32_t j = tid % NT;
        const uint32_t r = (tid / NT) % 16u;
        const uint32_t group = tid / (16u * NT);
        float sum = 0.0f;
        for (uint32_t w = 0; w < wpr; ++w) {
            sum += lds[((group * wpr + w) * 16u + r) * NT + j];
        }
        const uint32_t first_tile = bx * 64u + group * wpr * 16u;
        if (first_tile < tiles && j < tok_count) {
            const uint32_t tr = first_tile / tile_columns;
            const uint32_t split = (first_tile % tile_columns) / 64u;
            z[split * z_split_stride + static_cast<size_t>(tok0 + j) * rows + tr * kTile + r] = sum;
        }
    }
}

// ---- expert decode-GEMV ----------------------------------------------------

// Four rows of one expert tile = 8 states = bits [96q, 96q + 112) of the
// 384-bit stream: words 6q..6q+5 of the lane plus word 0 of the next quad.
template <int NT>
__device__ __forceinline__ void expert_gemv_block(const ExpertGemv &a, uint32_t bx, uint32_t by,
                                                  float *lds) {
    uint32_t mat = 0, tok_begin = 0, tok_end = a.batch;
    if (a.active != nullptr) {
        if (by >= *a.active_count) {
            return;
        }
        mat = a.active[by];
        tok_begin = a.offsets[mat];
        tok_end = a.offsets[mat + 1];
    }
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = threadIdx.x >> 6;
    const uint32_t quad = lane & 3u;
    const uint32_t tile_columns = a.columns / kTile;
    const uint32_t tile_rows = a.rows / kTile;
    const uint32_t tiles = tile_rows * tile_columns;
    const uint32_t tile = bx * 64u + wave * 16u + (lane >> 2);
    const bool valid = tile < tiles;
    const uint32_t tr = valid ? tile / tile_columns : 0u;
    const uint32_t tc = valid ? tile % tile_columns : 0u;

    uint32_t d[4];
    load_expert_quad(a.trellis + mat * a.trellis_stride, tile, quad, valid, lane, d);

    const float gamma = valid ? half_bits_to_float(a.gamma[mat * a.gamma_stride +
                                                           wave_slot(tr, tc, tile_rows, tile_columns)])
                              : 0.0f;
    uint4 e[8];
    decode_expert_quad(d, static_cast<const uint4 *>(a.codebook), e);

    for (uint32_t t0 = tok_begin; t0 < tok_end; t0 += NT) {
        const uint32_t count = tok_end - t0 < NT ? tok_end - t0 : NT;
        float acc[4][NT];
#pragma unroll
        for (int j = 0; j < NT; ++j) {
            float x[16];
            if (valid && static_cast<uint32_t>(j) < count) {
                const float4 *src = reinterpret_cast<const float4 *>(
                    a.x_hat + static_cast<size_t>(t0 + j) * a.columns + tc * kTile);
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const float4 v = src[q];
                    x[4 * q] = v.x;
                    x[4 * q + 1] = v.y;
                    x[4 * q + 2] = v.z;
                    x[4 * q + 3] = v.w;
                }
            } else {
#pragma unroll
                for (int q = 0; q < 16; ++q) {
                    x[q] = 0.0f;
                }
            }
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                float partial = 0.0f;
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const uint4 v = e[2 * m + h];
                    const uint32_t words[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                    for (int c = 0; c < 4; ++c) {
                        const float2 w = half2_bits_to_float2(words[c]);
                        partial = fmaf(w.x, x[8 * h + 2 * c], partial);
                        partial = fmaf(w.y, x[8 * h + 2 * c + 1], partial);
                    }
                }
                acc[m][j] = partial * gamma;
            }
        }
        reduce_rows_and_store<NT>(acc, lane, wave, tile, tile_columns, tiles, a.rows, t0, count,
                                  a.z, a.z_split_stride, lds, bx);
    }
}

template <int NT>
__global__ __launch_bounds__(256) void k_expert_gemv(ExpertGemv a) {
    __shared__ float lds[4 * 16 * NT];
    expert_gemv_block<NT>(a, blockIdx.x, blockIdx.y, lds);
}

// ---- NE decode-GEMV --------------------------------------------------------

// Four rows of one NE tile = 32 states = bytes [32q, 32q + 34) of the
// 1024-bit stream: words 16q..16q+15 of the lane plus word 0 of the next
// quad. The 1024-entry signed table, scaled by Wscale in fp32 as the
// reference does per state (src/kernels.cpp:673-683), sits in LDS.
template <int NT>
__device__ __forceinline__ void ne_gemv_block(const NeGemv &a, uint32_t bx, float2 *table,
                                              float *lds) {
    const uint32_t *book = static_cast<const uint32_t *>(a.codebook);
    for (uint32_t i = threadIdx.x; i < 1024u; i += blockDim.x) {
        const float2 v = half2_bits_to_float2(book[i]);
        table[i] = make_float2(v.x * a.weight_scale, v.y * a.weight_scale);
    }
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = threadIdx.x >> 6;
    const uint32_t quad = lane & 3u;
    const uint32_t tile_columns = a.columns / kTile;
    const uint32_t tiles = (a.rows / kTile) * tile_columns;
    const uint32_t tile = bx * 64u + wave * 16u + (lane >> 2);
    const bool valid = tile < tiles;
    const uint32_t tc = valid ? tile % tile_columns : 0u;

    uint32_t d[9];
    load_ne_quad(a.trellis, tile, quad, valid, lane, d);
    __syncthreads();
    uint32_t idx[32];
    decode_ne_quad(d, idx);

    for (uint32_t t0 = 0; t0 < a.batch; t0 += NT) {
        const uint32_t count = a.batch - t0 < NT ? a.batch - t0 : NT;
        float acc[4][NT];
#pragma unroll
        for (int j = 0; j < NT; ++j) {
            float x[16];
            if (valid && static_cast<uint32_t>(j) < count) {
                const float4 *src = reinterpret_cast<const float4 *>(
                    a.x_hat + static_cast<size_t>(t0 + j) * a.columns + tc * kTile);
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const float4 v = src[q];
                    x[4 * q] = v.x;
                    x[4 * q + 1] = v.y;
                    x[4 * q + 2] = v.z;
                    x[4 * q + 3] = v.w;
                }
            } else {
#pragma unroll
                for (int q = 0; q < 16; ++q) {
                    x[q] = 0.0f;
                }
            }
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                float sum = 0.0f;
#pragma unroll
                for (int st = 0; st < 8; ++st) {
                    const float2 w = table[idx[8 * m + st]];
                    sum = fmaf(w.x, x[2 * st], sum);
                    sum = fmaf(w.y, x[2 * st + 1], sum);
                }
                acc[m][j] = sum;
            }
        }
        reduce_rows_and_store<NT>(acc, lane, wave, tile, tile_columns, tiles, a.rows, t0, count,
                                  a.z, a.z_split_stride, lds, bx);
    }
}

template <int NT>
__global__ __launch_bounds__(256) void k_ne_gemv(NeGemv a) {
    __shared__ float2 table[1024];
    __shared__ float lds[4 * 16 * NT];
    ne_gemv_block<NT>(a, blockIdx.x, table, lds);
}

// Several expert and NE GEMVs in one launch (the MoE gate/up pair plus the
// shared expert's, or the down projections): blocks are numbered expert
// matrices first (max_active slots each), then NE matrices.
template <int NT>
__global__ __launch_bounds__(256) void k_moe_gemv(MoeGemv m) {
    __shared__ float2 table[1024];
    __shared__ float lds[4 * 16 * NT];
    uint32_t b = blockIdx.x;
    const uint32_t per_expert = m.expert_blocks * m.max_active;
    if (b < m.expert_count * per_expert) {
        const uint32_t which = b / per_expert;
        const uint32_t rest = b % per_expert;
        expert_gemv_block<NT>(m.expert[which], rest % m.expert_blocks, rest / m.expert_blocks, lds);
        return;
    }
    b -= m.expert_count * per_expert;
    ne_gemv_block<NT>(m.ne[b / m.ne_blocks], b % m.ne_blocks, table, lds);
}

}  // namespace

// ---- launchers -------------------------------------------------------------

bool wave_width(uint32_t n) { return n >= 64 && n <= 4096 && is_power_of_two(n); }

void launch_prologues(adi_hip_context *ctx, PrologueJobs &jobs) {
    uint32_t vectors = 0;
    for (uint32_t s = 0; s < jobs.segments; ++s) {
        vectors += jobs.seg[s].count;
    }
    jobs.scale = hadamard_scale(jobs.n);
    const dim3 grid(ceil_div(vectors, 4));
    switch (jobs.n) {
    case 64: launch(ctx, "hadamard_prologue", k_prologue_wave<1>, grid, dim3(256), 0, jobs); break;
    case 128: launch(ctx, "hadamard_prologue", k_prologue_wave<2>, grid, dim3(256), 0, jobs); break;
    case 256: launch(ctx, "hadamard_prologue", k_prologue_wave<4>, grid, dim3(256), 0, jobs); break;
    case 512: launch(ctx, "hadamard_prologue", k_prologue_wave<8>, grid, dim3(256), 0, jobs); break;
    case 1024: launch(ctx, "hadamard_prologue", k_prologue_wave<16>, grid, dim3(256), 0, jobs); break;
    case 2048: launch(ctx, "hadamard_prologue", k_prologue_wave<32>, grid, dim3(256), 0, jobs); break;
    case 4096: launch(ctx, "hadamard_prologue", k_prologue_wave<64>, grid, dim3(256), 0, jobs); break;
    default:
        for (uint32_t s = 0; s < jobs.segments; ++s) {
            const PrologueSegment &g = jobs.seg[s];
            if (g.su_f16 != nullptr) {
                launch(ctx, "hadamard_prologue", k_prologue<uint16_t>, dim3(g.count), dim3(256),
                       jobs.n * sizeof(float), g.x, jobs.n, g.su_f16, g.su_stride, g.source_row,
                       g.matrix_index, jobs.scale, g.out);
            } else {
                launch(ctx, "hadamard_prologue", k_prologue<int8_t>, dim3(g.count), dim3(256),
                       jobs.n * sizeof(float), g.x, jobs.n, g.su_sign, 0u, g.source_row,
                       static_cast<const uint32_t *>(nullptr), jobs.scale, g.out);
            }
        }
    }
}

template <typename Scale>
void launch_epilogue_any(adi_hip_context *ctx, const float *z, uint32_t splits,
                         size_t split_stride, uint32_t n, const Scale *sv, uint32_t vectors,
                         float *out) {
    const float scale = hadamard_scale(n);
    const dim3 grid(ceil_div(vectors, 4));
    switch (n) {
    case 64: launch(ctx, "hadamard_epilogue", k_epilogue_wave<1, Scale>, grid, dim3(256), 0, z, splits, split_stride, sv, vectors, scale, out); break;
    case 128: launch(ctx, "hadamard_epilogue", k_epilogue_wave<2, Scale>, grid, dim3(256), 0, z, splits, split_stride, sv, vectors, scale, out); break;
    case 256: launch(ctx, "hadamard_epilogue", k_epilogue_wave<4, Scale>, grid, dim3(256), 0, z, splits, split_stride, sv, vectors, scale, out); break;
    case 512: launch(ctx, "hadamard_epilogue", k_epilogue_wave<8, Scale>, grid, dim3(256), 0, z, splits, split_stride, sv, vectors, scale, out); break;
    case 1024: launch(ctx, "hadamard_epilogue", k_epilogue_wave<16, Scale>, grid, dim3(256), 0, z, splits, split_stride, sv, vectors, scale, out); break;
    case 2048: launch(ctx, "hadamard_epilogue", k_epilogue_wave<32, Scale>, grid, dim3(256), 0, z, splits, split_stride, sv, vectors, scale, out); break;
    case 4096: launch(ctx, "hadamard_epilogue", k_epilogue_wave<64, Scale>, grid, dim3(256), 0, z, splits, split_stride, sv, vectors, scale, out); break;
    default:
        launch(ctx, "hadamard_epilogue", k_epilogue<Scale>, dim3(vectors), dim3(256),
               n * sizeof(float), z, splits, split_stride, n, sv, 0u,
               static_cast<const uint32_t *>(nullptr), scale, out);
    }
}

void launch_prologue_f16(adi_hip_context *ctx, const float *x, uint32_t n,
                         const uint16_t *su, uint32_t su_stride,
                         const uint32_t *source_row, const uint32_t *matrix_index,
                         uint32_t vectors, float *out) {
    launch(ctx, "hadamard_prologue", k_prologue<uint16_t>, dim3(vectors), dim3(256),
           n * sizeof(float), x, n, su, su_stride, source_row, matrix_index, hadamard_scale(n), out);
}

void launch_prologue_sign(adi_hip_context *ctx, const float *x, uint32_t n,
                          const int8_t *su, uint32_t vectors, float *out) {
    launch(ctx, "hadamard_prologue", k_prologue<int8_t>, dim3(vectors), dim3(256),
           n * sizeof(float), x, n, su, 0u, static_cast<const uint32_t *>(nullptr),
           static_cast<const uint32_t *>(nullptr), hadamard_scale(n), out);
}

void launch_epilogue_f16(adi_hip_context *ctx, const float *z, uint32_t splits,
                         size_t split_stride, uint32_t n, const uint16_t *sv,
                         uint32_t sv_stride, const uint32_t *matrix_index,
                         uint32_t vectors, float *out) {
    launch(ctx, "hadamard_epilogue", k_epilogue<uint16_t>, dim3(vectors), dim3(256),
           n * sizeof(float), z, splits, split_stride, n, sv, sv_stride, matrix_index,
           hadamard_scale(n), out);
}

void launch_epilogue_sign(adi_hip_context *ctx, const float *z, uint32_t splits,
                          size_t split_stride, uint32_t n, const int8_t *sv,
                          uint32_t vectors, float *out) {
    launch(ctx, "hadamard_epilogue", k_epilogue<int8_t>, dim3(vectors), dim3(256),
           n * sizeof(float), z, splits, split_stride, n, sv, 0u,
           static_cast<const uint32_t *>(nullptr), hadamard_scale(n), out);
}

void launch_expert_gemv(adi_hip_context *ctx, const ExpertGemv &args) {
    const uint32_t tiles = (args.rows / kTile) * (args.columns / kTile);
    const dim3 grid(ceil_div(tiles, 64), args.active != nullptr ? args.max_active : 1u);
    if (args.tokens_per_pass == 1) {
        launch(ctx, "expert_gemv", k_expert_gemv<1>, grid, dim3(256), 0, args);
    } else {
        launch(ctx, "expert_gemv", k_expert_gemv<4>, grid, dim3(256), 0, args);
    }
}

void launch_moe_gemv(adi_hip_context *ctx, MoeGemv &m, bool single_token) {
    m.expert_blocks = ceil_div((m.expert[0].rows / kTile) * (m.expert[0].columns / kTile), 64);
    m.ne_blocks = ceil_div((m.ne[0].rows / kTile) * (m.ne[0].columns / kTile), 64);
    const uint32_t blocks = m.expert_count * m.expert_blocks * m.max_active + m.ne_count * m.ne_blocks;
    if (single_token) {
        launch(ctx, "moe_gemv", k_moe_gemv<1>, dim3(blocks), dim3(256), 0, m);
    } else {
        launch(ctx, "moe_gemv", k_moe_gemv<4>, dim3(blocks), dim3(256), 0, m);
    }
}

void launch_ne_gemv(adi_hip_context *ctx, const NeGemv &args) {
    const uint32_t tiles = (args.rows / kTile) * (args.columns / kTile);
    if (args.batch == 1) {
        launch(ctx, "ne_gemv", k_ne_gemv<1>, dim3(ceil_div(tiles, 64)), dim3(256), 0, args);
    } else {
        launch(ctx, "ne_gemv", k_ne_gemv<4>, dim3(ceil_div(tiles, 64)), dim3(256), 0, args);
    }
}

template void launch_epilogue_any<uint16_t>(adi_hip_context *, const float *, uint32_t, size_t,
                                            uint32_t, const uint16_t *, uint32_t, float *);
template void launch_epilogue_any<int8_t>(adi_hip_context *, const float *, uint32_t, size_t,
                                          uint32_t, const int8_t *, uint32_t, float *);

void validate_expert(const adi_hip_expert_matrix *m) {
    require(m != nullptr, "Mach expert matrix is null");
    require(is_power_of_two(m->rows) && is_power_of_two(m->columns) &&
                m->rows % kTile == 0 && m->columns % kTile == 0,
            "Mach expert dimensions must be tiled powers of two");
    require(m->columns <= kMaxHadamard && m->rows <= kMaxHadamard,
            "Mach expert dimensions exceed the 8192-wide Hadamard block");
    require(m->trellis != nullptr && m->su_f16 != nullptr && m->sv_f16 != nullptr &&
                m->wave_gamma_f16 != nullptr,
            "Mach expert codec tensor is null");
    require(m->codebook != nullptr && m->codebook->kind == adi_hip_codebook::expert,
            "Mach expert matrix needs an expert codebook");
}

void validate_ne(const adi_hip_ne_matrix *m) {
    require(m != nullptr, "Mach NE matrix is null");
    require(is_power_of_two(m->rows) && is_power_of_two(m->columns) &&
                m->rows % kTile == 0 && m->columns % kTile == 0,
            "Mach NE dimensions must be tiled powers of two");
    require(m->columns <= kMaxHadamard && m->rows <= kMaxHadamard,
            "Mach NE dimensions exceed the 8192-wide Hadamard block");
    require(m->trellis != nullptr && m->su != nullptr && m->sv != nullptr,
            "Mach NE codec tensor is null");
    require(m->codebook != nullptr && m->codebook->kind == adi_hip_codebook::ne,
            "Mach NE matrix needs an NE codebook");
}

}  // namespace adi_hip

using namespace adi_hip;

extern "C" {

int adi_hip_expert_matmul(adi_hip_context *ctx, const adi_hip_expert_matrix *m,
                          const float *inputs, uint32_t batch, float *outputs) {
    return guarded(ctx, [&] {
        validate_expert(m);
        require(batch > 0, "Mach expert batch shape mismatch");
        require(inputs != nullptr && outputs != nullptr, "Mach expert vector is null");
        const uint32_t splits = gemv_splits(m->columns);
        auto &ws = ctx->workspace;
        ws.used = 0;
        ws.ensure(Workspace::round(size_t(batch) * m->columns * 4) +
                  Workspace::round(size_t(splits) * batch * m->rows * 4));
        float *x_hat = ws.take<float>(size_t(batch) * m->columns);
        float *z = ws.take<float>(size_t(splits) * batch * m->rows);
        PrologueJobs jobs{};
        jobs.segments = 1;
        jobs.n = m->columns;
        jobs.seg[0] = PrologueSegment{inputs, nullptr, nullptr, m->su_f16, nullptr, 0, x_hat, batch};
        launch_prologues(ctx, jobs);
        ExpertGemv g{};
        g.trellis = m->trellis;
        g.gamma = m->wave_gamma_f16;
        g.codebook = m->codebook->data;
        g.rows = m->rows;
        g.columns = m->columns;
        g.x_hat = x_hat;
        g.z = z;
        g.z_split_stride = size_t(batch) * m->rows;
        g.batch = batch;
        g.tokens_per_pass = batch == 1 ? 1 : 4;
        launch_expert_gemv(ctx, g);
        launch_epilogue_any<uint16_t>(ctx, z, splits, size_t(batch) * m->rows, m->rows, m->sv_f16,
                                      batch, outputs);
    });
}

int adi_hip_expert_matvec(adi_hip_context *ctx, const adi_hip_expert_matrix *m,
                          const float *input, float *output) {
    return adi_hip_expert_matmul(ctx, m, input, 1, output);
}

int adi_hip_ne_matmul(adi_hip_context *ctx, const adi_hip_ne_matrix *m,
                      const float *inputs, uint32_t batch, float *outputs) {
    return guarded(ctx, [&] {
        validate_ne(m);
        require(batch > 0, "Mach NE batch shape mismatch");
        require(inputs != nullptr && outputs != nullptr, "Mach NE vector is null");
        const uint32_t splits = gemv_splits(m->columns);
        auto &ws = ctx->workspace;
        ws.used = 0;
        ws.ensure(Workspace::round(size_t(batch) * m->columns * 4) +
                  Workspace::round(size_t(splits) * batch * m->rows * 4));
        float *x_hat = ws.take<float>(size_t(batch) * m->columns);
        float *z = ws.take<float>(size_t(splits) * batch * m->rows);
        PrologueJobs jobs{};
        jobs.segments = 1;
        jobs.n = m->columns;
        jobs.seg[0] = PrologueSegment{inputs, nullptr, nullptr, nullptr, m->su, 0, x_hat, batch};
        launch_prologues(ctx, jobs);
        NeGemv g{};
        g.trellis = m->trellis;
        g.codebook = m->codebook->data;
        g.weight_scale = m->weight_scale;
        g.rows = m->rows;
        g.columns = m->columns;
        g.x_hat = x_hat;
        g.z = z;
        g.z_split_stride = size_t(batch) * m->rows;
        g.batch = batch;
        launch_ne_gemv(ctx, g);
        launch_epilogue_any<int8_t>(ctx, z, splits, size_t(batch) * m->rows, m->rows, m->sv, batch,
                                    outputs);
    });
}

int adi_hip_ne_matvec(adi_hip_context *ctx, const adi_hip_ne_matrix *m,
                      const float *input, float *output) {
    return adi_hip_ne_matmul(ctx, m, input, 1, output);
}

int adi_hip_hadamard(adi_hip_context *ctx, float *values, uint32_t n, uint32_t count) {
    return guarded(ctx, [&] {
        require(values != nullptr && count > 0, "Hadamard vectors are null or empty");
        require(is_power_of_two(n) && n <= kMaxHadamard, "Hadamard width must be a power of two up to 8192");
        const float scale = hadamard_scale(n);
        const dim3 grid(ceil_div(count, 4));
        switch (n) {
        case 64: launch(ctx, "hadamard", k_hadamard_wave<1>, grid, dim3(256), 0, values, count, scale); break;
        case 128: launch(ctx, "hadamard", k_hadamard_wave<2>, grid, dim3(256), 0, values, count, scale); break;
        case 256: launch(ctx, "hadamard", k_hadamard_wave<4>, grid, dim3(256), 0, values, count, scale); break;
        case 512: launch(ctx, "hadamard", k_hadamard_wave<8>, grid, dim3(256), 0, values, count, scale); break;
        case 1024: launch(ctx, "hadamard", k_hadamard_wave<16>, grid, dim3(256), 0, values, count, scale); break;
        case 2048: launch(ctx, "hadamard", k_hadamard_wave<32>, grid, dim3(256), 0, values, count, scale); break;
        case 4096: launch(ctx, "hadamard", k_hadamard_wave<64>, grid, dim3(256), 0, values, count, scale); break;
        default:
            launch(ctx, "hadamard", k_hadamard_block, dim3(count), dim3(256), n * sizeof(float),
                   values, n, scale);
        }
    });
}

int adi_hip_expert_decode(adi_hip_context *ctx, const adi_hip_expert_matrix *m, float *values) {
    return guarded(ctx, [&] {
        validate_expert(m);
        require(values != nullptr, "decode output is null");
        const uint32_t tiles = (m->rows / kTile) * (m->columns / kTile);
        launch(ctx, "expert_decode", k_expert_decode, dim3(ceil_div(tiles, 64)), dim3(256), 0,
               m->trellis, static_cast<const void *>(m->codebook->data), m->rows, m->columns,
               values);
    });
}

int adi_hip_ne_decode(adi_hip_context *ctx, const adi_hip_ne_matrix *m, float *values) {
    return guarded(ctx, [&] {
        validate_ne(m);
        require(values != nullptr, "decode output is null");
        const uint32_t tiles = (m->rows / kTile) * (m->columns / kTile);
        launch(ctx, "ne_decode", k_ne_decode, dim3(ceil_div(tiles, 64)), dim3(256), 0,
               m->trellis, static_cast<const void *>(m->codebook->data), m->weight_scale,
               m->rows, m->columns, values);
    });
}

}  // extern "C"
