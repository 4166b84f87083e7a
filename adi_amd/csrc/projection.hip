// projection.hip -- decode-GEMV kernels for the expert (K=1.5/V=8) and
// non-expert (K=4/V=2) trellis codecs, the Hadamard prologue/epilogue around
// them, and the Backend entry points expert_matvec/matmul and
// ne_matvec/matmul.
//
// Data flow of one projection y = W x (src/kernels.cpp:385-800):
//   prologue  x_hat = H_C(su * x)                 one wave per vector
//   gemv      Z[r] = sum_tiles decoded(tile) . x_hat   codes read once, decoded
//                                                  in registers
//   epilogue  y = sv * H_R(sum_slices Z)           one wave per vector
//
// The decode-GEMV is persistent: one 512-thread block per CU. Random gathers
// from a 256 KiB expert codebook in global memory run at under half a gather
// per clock per CU, from LDS at seven, so each block holds one component
// plane of the codebook (components 0-3 or 4-7 of every row, 128 KiB) in LDS
// and computes that half of every tile column; half-0 and half-1 blocks walk
// the same tiles. A wave item is up to 64 consecutive tiles of one tile row
// (four groups of 16); four lanes share a tile and own four of its sixteen
// rows ("quads"). A lane loads its quad's slice of the packed stream, decodes
// the states of its rows against the LDS plane, multiplies them with x_hat,
// and the wave sums its tiles with shuffles, so no block barrier follows the
// codebook fill. Each (item column range, half) writes its own slice of Z;
// the consumer adds the slices in a fixed order.
#include "projection.hpp"
#include "grouped.hpp"
#include "route.hpp"
#include "dense.hpp"

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

// The eight states of a quad against one component plane of the expert
// codebook: 4 f16 lattice values per state (components 4h..4h+3 of one
// reachable row; bit 15 of the state hash negates component 0, which lives in
// plane 0).
__device__ __forceinline__ void decode_expert_half(const uint32_t (&d)[4], const uint2 *plane,
                                                   uint32_t half, uint2 (&e)[8]) {
    const uint32_t sign_mask = half == 0 ? 0x8000u : 0u;
#define ADI_EXPERT_STATE(K)                                            \
    {                                                                  \
        const uint32_t p = state_product(stream_window<12 * K>(d));    \
        e[K] = plane[(p >> 1) & 0x3FFFu];                              \
        e[K].x ^= p & sign_mask;                                       \
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
    const uint2 *plane = static_cast<const uint2 *>(codebook);
    uint2 lo[8], hi[8];
    decode_expert_half(d, plane, 0, lo);
    decode_expert_half(d, plane + kExpertRows, 1, hi);
    if (!valid) {
        return;
    }
    const uint32_t tr = tile / tile_columns, tc = tile % tile_columns;
    for (int k = 0; k < 8; ++k) {
        const uint32_t row = tr * kTile + quad * 4u + k / 2;
        float *dst = out + static_cast<size_t>(row) * columns + tc * kTile + (k & 1) * 8;
        const uint32_t w[4] = {lo[k].x, lo[k].y, hi[k].x, hi[k].y};
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
    prologue_vector<VPL>(j, blockIdx.x * 4u + (threadIdx.x >> 6), threadIdx.x & 63u);
}

// y = sv * H_n(sum over splits of z), one wave per vector (the slices' loads
// go out up to eight at a time, so the kernel may hold up to 256 registers).
template <int VPL, typename Scale>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 2))) void k_epilogue_wave(
    const float *__restrict__ z, uint32_t splits, size_t split_stride, const Scale *__restrict__ sv,
    uint32_t vectors, float scale, float *__restrict__ out) {
#pragma clang fp contract(off)
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t v = blockIdx.x * 4u + (threadIdx.x >> 6);
    if (v >= vectors) {
        return;
    }
    const uint32_t n = 64u * VPL;
    float val[VPL];
    float s[VPL];
    if constexpr (sizeof(Scale) == 2) {
        load_wave_f16<VPL>(reinterpret_cast<const uint16_t *>(sv), lane, s);
    } else {
        load_wave_sign<VPL>(reinterpret_cast<const int8_t *>(sv), lane, s);
    }
    sum_slices_deep<VPL>(z + static_cast<size_t>(v) * n, split_stride, splits, lane, val);
    wave_hadamard<VPL>(val, scale, lane);
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
        val[i] = val[i] * s[i];
    }
    store_wave<VPL>(out + static_cast<size_t>(v) * n, lane, val);
}

// z[i] = ((0 + z[i]) + z[stride + i]) + ... over the slices, in place in
// slice 0: the slice-order sum of sum_slices, spread over many CUs. A
// single-vector epilogue would otherwise pull every slice through one CU.
__global__ __launch_bounds__(64) void k_reduce_slices(float *z, uint32_t splits, size_t stride,
                                                      uint32_t count4) {
#pragma clang fp contract(off)
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= count4) {
        return;
    }
    float4 *z4 = reinterpret_cast<float4 *>(z);
    const size_t stride4 = stride / 4;
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (uint32_t s0 = 0; s0 < splits; s0 += 8) {
        float4 a[8];
#pragma unroll
        for (uint32_t g = 0; g < 8; ++g) {
            a[g] = z4[(s0 + g < splits ? s0 + g : splits - 1u) * stride4 + i];
        }
#pragma unroll
        for (uint32_t g = 0; g < 8; ++g) {
            if (s0 + g < splits) {
                acc.x = acc.x + a[g].x;
                acc.y = acc.y + a[g].y;
                acc.z = acc.z + a[g].z;
                acc.w = acc.w + a[g].w;
            }
        }
    }
    z4[i] = acc;
}

// y = sv * H_8192(sum over splits of z): four waves per vector, wave w
// holding values [2048 w, 2048 w + 2048) in the wave layout. Each quarter's
// transform runs the strides 1 .. 1024; strides 2048 and 4096 then pair
// values across quarters in LDS. The butterflies run in the reference's
// stride order, so the result is the reference's transform.
template <typename Scale>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 2))) void k_epilogue_8192(
    const float *__restrict__ z, uint32_t splits, size_t split_stride, const Scale *__restrict__ sv,
    float scale, float *__restrict__ out) {
#pragma clang fp contract(off)
    constexpr uint32_t n = 8192, quarter = 2048;
    __shared__ __align__(16) float v[n];
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    float val[32];
    sum_slices_deep<32>(z + static_cast<size_t>(blockIdx.x) * n + wave * quarter, split_stride,
                        splits, lane, val);
    wave_hadamard<32>(val, 1.0f, lane);  // x * 1 is exact: the scale comes last
    store_wave<32>(v + wave * quarter, lane, val);
    for (uint32_t stride = quarter; stride < n; stride <<= 1) {
        __syncthreads();
        for (uint32_t k = threadIdx.x; k < n / 2; k += blockDim.x) {
            const uint32_t lo = ((k & ~(stride - 1)) << 1) | (k & (stride - 1));
            const float a = v[lo];
            const float b = v[lo + stride];
            v[lo] = a + b;
            v[lo + stride] = a - b;
        }
    }
    __syncthreads();
    // four consecutive values per thread and pass, every scale load issued
    // before the first store
    float4 *dst = reinterpret_cast<float4 *>(out + static_cast<size_t>(blockIdx.x) * n);
    const float4 *v4 = reinterpret_cast<const float4 *>(v);
    constexpr uint32_t kPasses = n / 4 / 256;
    float s[kPasses][4];
#pragma unroll
    for (uint32_t p = 0; p < kPasses; ++p) {
        const uint32_t k = (p * 256 + threadIdx.x) * 4;
#pragma unroll
        for (uint32_t e = 0; e < 4; ++e) {
            s[p][e] = scale_value<Scale>(sv[k + e]);
        }
    }
#pragma unroll
    for (uint32_t p = 0; p < kPasses; ++p) {
        const float4 a = v4[p * 256 + threadIdx.x];
        dst[p * 256 + threadIdx.x] = make_float4(a.x * scale * s[p][0], a.y * scale * s[p][1],
                                                 a.z * scale * s[p][2], a.w * scale * s[p][3]);
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
    float *p = values + static_cast<size_t>(v) * 64u * VPL;
    float val[VPL];
    load_wave<VPL>(p, lane, val);
    wave_hadamard<VPL>(val, scale, lane);
    store_wave<VPL>(p, lane, val);
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

// ---- persistent decode-GEMV ------------------------------------------------

constexpr uint32_t kGemvThreads = 512;
constexpr uint32_t kGemvWaves = kGemvThreads / kWave;

// A thread's share of the 4 KiB NE table (threads 0 .. kGemvThreads - 1),
// loaded into registers so that other loads can go out before it is stored.
constexpr uint32_t kTableWords = 1024u / kGemvThreads;
__device__ __forceinline__ void load_table_share(const uint32_t *src, uint32_t (&v)[kTableWords]) {
#pragma unroll
    for (uint32_t k = 0; k < kTableWords; ++k) {
        v[k] = src[threadIdx.x + k * kGemvThreads];
    }
}
__device__ __forceinline__ void store_table_share(const uint32_t (&v)[kTableWords], uint32_t *dst) {
#pragma unroll
    for (uint32_t k = 0; k < kTableWords; ++k) {
        dst[threadIdx.x + k * kGemvThreads] = v[k];
    }
}
constexpr size_t kPlaneBytes = size_t(kExpertRows) * 8;  // one component plane
constexpr uint32_t kMaxSlots = 1024;                     // routed slots staged in LDS

// The loads of one expert wave item, issued one item ahead of its arithmetic
// so that a wave's next item is in flight while the current one computes.
struct ExpertStage {
    uint4 info;         // {matrix, first position, end position, -}; empty when end == first
    uint32_t d[4][3];   // the lane's three stream dwords in each group of 16 tiles
    uint32_t gamma[4];  // f16 bits of each group's wave gamma, converted at use so
                        // that nothing waits on these loads when they are issued
    float4 x[4][2];     // x_hat of the first position: columns c0..c0+3, c0+8..c0+11
};

struct ExpertItem {
    uint32_t which, slot, item;
};

// Item i of the expert phase: matrix entry, routed slot, item within the slot
// (items per slot is a power of two, so no division).
__device__ __forceinline__ ExpertItem expert_item_of(const MoeGemv &m, uint32_t i) {
    const uint32_t per_matrix = m.max_active << m.item_shift;
    const uint32_t which = i >= per_matrix ? 1u : 0u;
    const uint32_t rest = i - which * per_matrix;
    return {which, rest >> m.item_shift, rest & ((1u << m.item_shift) - 1u)};
}

__device__ __forceinline__ void load_x_pair(const float *x_hat, uint32_t columns, uint32_t position,
                                            const uint32_t (&column)[4], uint32_t groups,
                                            const bool (&valid)[4], float4 (&x)[4][2]) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        x[g][0] = x[g][1] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (static_cast<uint32_t>(g) < groups && valid[g]) {
            const float *src = x_hat + static_cast<size_t>(position) * columns + column[g];
            x[g][0] = *reinterpret_cast<const float4 *>(src);
            x[g][1] = *reinterpret_cast<const float4 *>(src + 8);
        }
    }
}

// Tiles [item*16S, item*16S + 16S) of the item's matrix, S = item_groups.
__device__ __forceinline__ void expert_tiles(const ExpertGemv &a, uint32_t item, uint32_t half,
                                             uint32_t lane, uint32_t (&column)[4],
                                             bool (&valid)[4], uint32_t (&tile)[4]) {
    const uint32_t tiles = a.tile_rows << a.tc_shift;
    const uint32_t tc_mask = (1u << a.tc_shift) - 1u;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        tile[g] = (item << (4u + a.group_shift)) + g * 16u + (lane >> 2);
        valid[g] = (static_cast<uint32_t>(g) >> a.group_shift) == 0 && tile[g] < tiles;
        column[g] = valid[g] ? ((tile[g] & tc_mask) << 4) + 4u * half : 0u;
    }
}

__device__ __forceinline__ void expert_prefetch(const MoeGemv &m, const uint4 *slots, uint32_t i,
                                                uint32_t half, uint32_t lane, ExpertStage &st,
                                                const float *x_lds = nullptr, bool with_x = true) {
    const ExpertItem it = expert_item_of(m, i);
    const ExpertGemv &a = m.expert[it.which];
    const uint4 info = slots[it.slot];
    st.info = make_uint4(__builtin_amdgcn_readfirstlane(info.x), __builtin_amdgcn_readfirstlane(info.y),
                         __builtin_amdgcn_readfirstlane(info.z), 0u);
    const uint32_t quad = lane & 3u;
    const uint32_t tile_columns = 1u << a.tc_shift;
    const uint32_t groups = 1u << a.group_shift;
    const bool live = st.info.z > st.info.y;
    uint32_t column[4], tile[4];
    bool valid[4];
    expert_tiles(a, it.item, half, lane, column, valid, tile);
    // a slot past the active count may name any expert: its stage reads
    // expert 0 and is never computed
    const uint32_t expert = live ? st.info.x : 0u;
    const uint32_t *words = reinterpret_cast<const uint32_t *>(a.trellis + expert * a.trellis_stride);
    const uint16_t *gamma_row = a.gamma + expert * a.gamma_stride;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        valid[g] = valid[g] && live;
        if (static_cast<uint32_t>(g) < groups) {
            // no lane branches here: a lane past the matrix reads tile 0 and
            // expert_compute zeroes its gamma, so the loads go straight to
            // their registers and nothing waits on them until the compute
            const uint32_t t = valid[g] ? tile[g] : 0u;
            const uint32_t *src = words + static_cast<size_t>(t) * 12u + quad * 3u;
            // the lane's three dwords in one 12-byte load (each load
            // instruction takes the CU's address path once)
            typedef uint32_t u32x3 __attribute__((ext_vector_type(3)));
            const u32x3 w = __builtin_nontemporal_load(reinterpret_cast<const u32x3 *>(src));
            st.d[g][0] = w.x;
            st.d[g][1] = w.y;
            st.d[g][2] = w.z;
            const uint32_t tr = t >> a.tc_shift, tc = t & (tile_columns - 1u);
            st.gamma[g] = gamma_row[wave_slot(tr, tc, a.tile_rows, tile_columns)];
        }
    }
    // a fused SwiGLU's x_hat sits in LDS for the item's single position
    if (with_x) {
        load_x_pair(x_lds != nullptr ? x_lds : a.x_hat, a.columns, x_lds != nullptr ? 0u : st.info.y,
                    column, groups, valid, st.x);
    }
}

// The x_hat loads of expert_prefetch for a stage whose words were loaded
// without them (with_x false): the item's single position from x_lds.
__device__ __forceinline__ void expert_prefetch_x(const MoeGemv &m, uint32_t i, uint32_t half,
                                                  uint32_t lane, ExpertStage &st, const float *x_lds) {
    const ExpertItem it = expert_item_of(m, i);
    const ExpertGemv &a = m.expert[it.which];
    uint32_t column[4], tile[4];
    bool valid[4];
    expert_tiles(a, it.item, half, lane, column, valid, tile);
    const bool live = st.info.z > st.info.y;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        valid[g] = valid[g] && live;
    }
    load_x_pair(x_lds, a.columns, 0u, column, 1u << a.group_shift, valid, st.x);
}

template <bool COHERENT = false>
__device__ __forceinline__ void expert_compute(const MoeGemv &m, uint32_t i, uint32_t half,
                                               const uint2 *plane, uint32_t lane,
                                               ExpertStage &st) {
    if (st.info.z <= st.info.y) {
        return;  // slot past the active count (wave-uniform)
    }
    const ExpertItem it = expert_item_of(m, i);
    const ExpertGemv &a = m.expert[it.which];
    const uint32_t quad = lane & 3u, tslot = lane >> 2;
    const uint32_t tile_columns = 1u << a.tc_shift;
    const uint32_t groups = 1u << a.group_shift;
    uint32_t column[4], tile[4];
    bool valid[4];
    expert_tiles(a, it.item, half, lane, column, valid, tile);
    // the states of the lane's rows: its 3 dwords plus word 0 of the next quad
    // (quad 3 wraps to word 0 of the tile, src/expert_trellis.hpp:79-80)
    uint32_t next_word[4];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        next_word[g] = quad_next(st.d[g][0]) & 0xFFFFu;
    }
    const uint32_t span = tile_columns < 16u ? tile_columns : 16u;  // tiles of one row in a group
    const uint32_t tile0 = tile[0];
    const uint32_t split = ((tile0 & (tile_columns - 1u)) >> (4u + a.group_shift)) * 2u + half;
    const uint32_t tr = tile0 >> a.tc_shift;
    const bool writer = (tslot % span) == 0 && valid[0];
    float4 (&x)[4][2] = st.x;  // the first position's, then reloaded per position
    for (uint32_t position = st.info.y; position < st.info.z; ++position) {
        // keeps the codebook gathers of every group inside the loop (hoisted,
        // the decoded states of all groups would stay live at once)
        asm volatile("" ::: "memory");
        if (position != st.info.y) {
            load_x_pair(a.x_hat, a.columns, position, column, groups, valid, x);
        }
        float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            if (static_cast<uint32_t>(g) >= groups) {
                continue;
            }
            // decoded per group (and per position) to bound register use
            const uint32_t d[4] = {st.d[g][0], st.d[g][1], st.d[g][2], next_word[g]};
            uint2 e[8];
            decode_expert_half(d, plane, half, e);
            // row r: state 2r covers columns c0..c0+3, state 2r+1 c0+8..c0+11;
            // the four rows' chains are interleaved so they hide each other's latency
            const float xs[8] = {x[g][0].x, x[g][0].y, x[g][0].z, x[g][0].w,
                                 x[g][1].x, x[g][1].y, x[g][1].z, x[g][1].w};
            float partial[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int c = 0; c < 8; ++c) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const uint2 v = e[2 * r + (c >> 2)];
                    const float2 w = half2_bits_to_float2((c & 2) ? v.y : v.x);
                    partial[r] = fmaf((c & 1) ? w.y : w.x, xs[c], partial[r]);
                }
            }
            // the opaque copy keeps the conversion (and the wait for the
            // load) here rather than where the load was issued
            uint32_t gamma_bits = st.gamma[g];
            asm volatile("" : "+v"(gamma_bits));
            const float gamma = valid[g] ? half_bits_to_float(gamma_bits) : 0.0f;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                acc[r] = fmaf(partial[r], gamma, acc[r]);
            }
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            acc[r] = sum_over_quads(acc[r], span);
        }
        if (writer) {
            float *dst = a.z + split * a.z_split_stride + static_cast<size_t>(position) * a.rows +
                         tr * kTile + quad * 4u;
            store4<COHERENT>(dst, make_float4(acc[0], acc[1], acc[2], acc[3]));
        }
    }
}

// The loads of one NE wave item (16 consecutive tiles of one matrix, all 16
// columns of each tile), issued one item ahead.
struct NeStage {
    uint32_t d[8];   // the lane's 8 stream dwords
    float x[16];     // x_hat of position 0 over the tile's columns
};

__device__ __forceinline__ void ne_tile(const NeGemv &a, uint32_t item, uint32_t lane,
                                        uint32_t &tile, bool &valid, uint32_t &column) {
    tile = item * 16u + (lane >> 2);
    valid = tile < (a.tile_rows << a.tc_shift);
    column = valid ? (tile & ((1u << a.tc_shift) - 1u)) << 4 : 0u;
}

// NE item k of a launch: matrix entry and item within it.
__device__ __forceinline__ uint2 ne_item_of(const MoeGemv &m, uint32_t k) {
    const uint32_t which = k >= m.ne_items_per_matrix ? 1u : 0u;
    return make_uint2(which, k - which * m.ne_items_per_matrix);
}

template <bool COHERENT = false>
__device__ __forceinline__ void load_x16(const float *x_hat, uint32_t columns, uint32_t position,
                                         uint32_t column, bool valid, float (&x)[16]) {
#pragma unroll
    for (int q = 0; q < 16; ++q) {
        x[q] = 0.0f;
    }
    if (valid) {
        const float *src = x_hat + static_cast<size_t>(position) * columns + column;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float4 v = load4<COHERENT>(src + 4 * q);
            x[4 * q] = v.x;
            x[4 * q + 1] = v.y;
            x[4 * q + 2] = v.z;
            x[4 * q + 3] = v.w;
        }
    }
}

template <bool COHERENT = false>
__device__ __forceinline__ void ne_prefetch(const MoeGemv &m, uint32_t k, uint32_t lane,
                                            NeStage &st, const float *x_lds = nullptr, uint32_t first = 0) {
    const uint2 it = ne_item_of(m, k);
    const NeGemv &a = m.ne[it.x];
    uint32_t tile, column;
    bool valid;
    ne_tile(a, it.y, lane, tile, valid, column);
    // no branch around the code loads (a lane past the matrix reads tile 0:
    // its x_hat is zero, so its sums stay +0 whatever its codes), so that
    // nothing waits for them here
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    const u32x4 *src = reinterpret_cast<const u32x4 *>(a.trellis) +
                       static_cast<size_t>(valid ? tile : 0u) * 8u + (lane & 3u) * 2u;
    const u32x4 lo = __builtin_nontemporal_load(src), hi = __builtin_nontemporal_load(src + 1);
    st.d[0] = lo.x; st.d[1] = lo.y; st.d[2] = lo.z; st.d[3] = lo.w;
    st.d[4] = hi.x; st.d[5] = hi.y; st.d[6] = hi.z; st.d[7] = hi.w;
    if (x_lds != nullptr) {
        load_x16(x_lds, a.columns, 0, column, valid && a.batch > 0, st.x);
    } else {
        load_x16<COHERENT>(a.x_hat, a.columns, first, column, valid && first < a.batch, st.x);
    }
}

// ne_prefetch in two parts: the codes (no dependence on the launch's data),
// then the x_hat of position `first` once it is in.
__device__ __forceinline__ void ne_prefetch_codes(const MoeGemv &m, uint32_t k, uint32_t lane, NeStage &st) {
    const uint2 it = ne_item_of(m, k);
    const NeGemv &a = m.ne[it.x];
    uint32_t tile, column;
    bool valid;
    ne_tile(a, it.y, lane, tile, valid, column);
    // no branch around the loads, as in ne_prefetch
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    const u32x4 *src =
        reinterpret_cast<const u32x4 *>(a.trellis) + static_cast<size_t>(valid ? tile : 0u) * 8u + (lane & 3u) * 2u;
    const u32x4 lo = __builtin_nontemporal_load(src), hi = __builtin_nontemporal_load(src + 1);
    st.d[0] = lo.x; st.d[1] = lo.y; st.d[2] = lo.z; st.d[3] = lo.w;
    st.d[4] = hi.x; st.d[5] = hi.y; st.d[6] = hi.z; st.d[7] = hi.w;
}
__device__ __forceinline__ void ne_prefetch_x(const MoeGemv &m, uint32_t k, uint32_t lane, NeStage &st,
                                              uint32_t first) {
    const uint2 it = ne_item_of(m, k);
    const NeGemv &a = m.ne[it.x];
    uint32_t tile, column;
    bool valid;
    ne_tile(a, it.y, lane, tile, valid, column);
    load_x16(a.x_hat, a.columns, first, column, valid && first < a.batch, st.x);
}

// Row sums over all 16 columns of each tile with the signed table in LDS,
// scaled by Wscale once after the tile sums.
template <bool COHERENT = false>
__device__ __forceinline__ void ne_compute(const MoeGemv &m, uint32_t k, const uint32_t *table,
                                           uint32_t lane, NeStage &st, uint32_t first = 0,
                                           uint32_t end = 0xFFFFFFFFu) {
    const uint2 it = ne_item_of(m, k);
    const NeGemv &a = m.ne[it.x];
    const uint32_t quad = lane & 3u, tslot = lane >> 2;
    const uint32_t tile_columns = 1u << a.tc_shift;
    uint32_t tile, column;
    bool valid;
    ne_tile(a, it.y, lane, tile, valid, column);
    // word 0 of the next quad (quad 3 wraps, src/ne_trellis.hpp:196-200)
    const uint32_t d[9] = {st.d[0], st.d[1], st.d[2], st.d[3], st.d[4], st.d[5], st.d[6], st.d[7],
                           quad_next(st.d[0]) & 0xFFFFu};
    uint32_t idx[32];
    decode_ne_quad(d, idx);
    const uint32_t span = tile_columns < 16u ? tile_columns : 16u;
    const uint32_t split = (tile & (tile_columns - 1u)) >> 4;
    const uint32_t tr = tile >> a.tc_shift;
    const bool writer = (tslot % span) == 0 && valid;
    float (&x)[16] = st.x;  // position first's, then reloaded per position
    const uint32_t stop = end < a.batch ? end : a.batch;
    for (uint32_t position = first; position < stop; ++position) {
        if (position != first) {
            load_x16(a.x_hat, a.columns, position, column, valid, x);
        }
        float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int s = 0; s < 8; ++s) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float2 w = half2_bits_to_float2(table[idx[8 * r + s]]);
                acc[r] = fmaf(w.x, x[2 * s], acc[r]);
                acc[r] = fmaf(w.y, x[2 * s + 1], acc[r]);
            }
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            acc[r] = sum_over_quads(acc[r], span);
        }
        if (writer) {
            float *dst = a.z + split * a.z_split_stride + static_cast<size_t>(position) * a.rows +
                         tr * kTile + quad * 4u;
            store4<COHERENT>(dst, make_float4(acc[0] * a.weight_scale, acc[1] * a.weight_scale,
                                              acc[2] * a.weight_scale, acc[3] * a.weight_scale));
        }
    }
}

// One row's SwiGLU into x_hat (width 512, the wave layout), as the MoE's
// swiglu launch computes it (src/executor.cpp:300-312): the routed row of
// grouped position `row` with expert `expert`'s f16 scales, or the shared
// expert's row `row` with its signs. Split in two so that the scale and first four
// slice loads go out before the codebook plane's (loads return in order).
struct SwigluInputs {
    float sa[kFusedSwigluWidth / 64], sb[kFusedSwigluWidth / 64], sc[kFusedSwigluWidth / 64];
    float g[4][kFusedSwigluWidth / 64], u[4][kFusedSwigluWidth / 64];
};

__device__ __forceinline__ void swiglu_issue_scales(const GemvSwiglu &f, bool shared, uint32_t expert,
                                                    uint32_t lane, SwigluInputs &in) {
    constexpr int VPL = kFusedSwigluWidth / 64;
    constexpr uint32_t n = kFusedSwigluWidth;
    if (shared) {
        load_wave_sign<VPL>(f.shared_sv_gate, lane, in.sa);
        load_wave_sign<VPL>(f.shared_sv_up, lane, in.sb);
        load_wave_sign<VPL>(f.shared_su_down, lane, in.sc);
    } else {
        const size_t mat = static_cast<size_t>(expert) * n;
        load_wave_f16<VPL>(f.sv_gate + mat, lane, in.sa);
        load_wave_f16<VPL>(f.sv_up + mat, lane, in.sb);
        load_wave_f16<VPL>(f.su_down + mat, lane, in.sc);
    }
}

template <bool COHERENT = false>
__device__ __forceinline__ void swiglu_issue_slices(const GemvSwiglu &f, bool shared, uint32_t row,
                                                    uint32_t lane, SwigluInputs &in) {
    constexpr int VPL = kFusedSwigluWidth / 64;
    constexpr uint32_t n = kFusedSwigluWidth;
    const float *zg = (shared ? f.shared_z_gate : f.z_gate) + static_cast<size_t>(row) * n;
    const float *zu = (shared ? f.shared_z_up : f.z_up) + static_cast<size_t>(row) * n;
    const size_t stride = shared ? f.shared_split_stride : f.split_stride;
    const uint32_t splits = shared ? f.shared_splits : f.splits;
#pragma unroll
    for (uint32_t s = 0; s < 4; ++s) {
        const uint32_t at = s < splits ? s : splits - 1u;  // a missing slice reloads the last
        load_wave<VPL, COHERENT>(zg + at * stride, lane, in.g[s]);
        load_wave<VPL, COHERENT>(zu + at * stride, lane, in.u[s]);
    }
}

template <bool COHERENT = false>
__device__ __forceinline__ void swiglu_issue(const GemvSwiglu &f, bool shared, uint32_t row,
                                             uint32_t expert, uint32_t lane, SwigluInputs &in) {
    swiglu_issue_scales(f, shared, expert, lane, in);
    swiglu_issue_slices<COHERENT>(f, shared, row, lane, in);
}

template <bool COHERENT = false>
__device__ __forceinline__ void swiglu_finish(const GemvSwiglu &f, bool shared, uint32_t row,
                                              uint32_t lane, SwigluInputs &in,
                                              float (&out)[kFusedSwigluWidth / 64]) {
#pragma clang fp contract(off)
    constexpr int VPL = kFusedSwigluWidth / 64;
    constexpr uint32_t n = kFusedSwigluWidth;
    const float *zg = (shared ? f.shared_z_gate : f.z_gate) + static_cast<size_t>(row) * n;
    const float *zu = (shared ? f.shared_z_up : f.z_up) + static_cast<size_t>(row) * n;
    const size_t stride = shared ? f.shared_split_stride : f.split_stride;
    const uint32_t splits = shared ? f.shared_splits : f.splits;
    float gv[VPL], uv[VPL];
    // the slice-order sums of sum_slices: 0 + slice 0 + slice 1 + ...
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
        gv[i] = 0.0f + in.g[0][i];
        uv[i] = 0.0f + in.u[0][i];
    }
#pragma unroll
    for (uint32_t s = 1; s < 4; ++s) {
#pragma unroll
        for (int i = 0; i < VPL; ++i) {
            gv[i] = s < splits ? gv[i] + in.g[s][i] : gv[i];
            uv[i] = s < splits ? uv[i] + in.u[s][i] : uv[i];
        }
    }
    if (splits > 4) {
        // slices 4 .. 7 in one round of loads (a missing one reloads the
        // last and is not added), the rest one at a time
        float a[4][VPL], c[4][VPL];
#pragma unroll
        for (uint32_t t = 0; t < 4; ++t) {
            const uint32_t at = 4 + t < splits ? 4 + t : splits - 1u;
            load_wave<VPL, COHERENT>(zg + at * stride, lane, a[t]);
            load_wave<VPL, COHERENT>(zu + at * stride, lane, c[t]);
        }
#pragma unroll
        for (uint32_t t = 0; t < 4; ++t) {
#pragma unroll
            for (int i = 0; i < VPL; ++i) {
                gv[i] = 4 + t < splits ? gv[i] + a[t][i] : gv[i];
                uv[i] = 4 + t < splits ? uv[i] + c[t][i] : uv[i];
            }
        }
    }
    for (uint32_t s = 8; s < splits; ++s) {
        float a[VPL], c[VPL];
        load_wave<VPL, COHERENT>(zg + s * stride, lane, a);
        load_wave<VPL, COHERENT>(zu + s * stride, lane, c);
#pragma unroll
        for (int i = 0; i < VPL; ++i) {
            gv[i] = gv[i] + a[i];
            uv[i] = uv[i] + c[i];
        }
    }
    wave_hadamard<VPL>(gv, f.scale, lane);
    wave_hadamard<VPL>(uv, f.scale, lane);
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
        const float g = gv[i] * in.sa[i];
        gv[i] = g / (1.0f + expf(-g)) * (uv[i] * in.sb[i]) * in.sc[i];
    }
    wave_hadamard<VPL>(gv, f.scale, lane);
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
        out[i] = gv[i];
    }
}

// Slot of expert item i (one expert entry).
__device__ __forceinline__ uint32_t item_slot(const MoeGemv &m, uint32_t i) {
    return expert_item_of(m, i).slot;
}

// Block b serves component plane (b / 8) % 2 as worker ((b / 16) * 8 + b % 8),
// so the two blocks that walk the same tiles sit on the same XCD (blocks are
// dealt to the eight XCDs round robin) and share its L2. Each wave walks its
// expert items, then its share of the NE items, with the loads of item k+1
// issued before the arithmetic of item k.
__global__ __launch_bounds__(kGemvThreads) void k_trellis_gemv(MoeGemv m) {
    // [slot_capacity] slots, then the plane; with a fused SwiGLU then the
    // shared expert's x_hat and one routed x_hat per wave
    extern __shared__ uint4 lds_dynamic[];
    __shared__ uint32_t ne_table[1024];
    uint4 *slots = lds_dynamic;
    uint4 *plane_lds = lds_dynamic + m.slot_capacity;
    float *shared_x_lds = reinterpret_cast<float *>(plane_lds + (m.expert_count > 0 ? kPlaneBytes / 16 : 0));
    const uint32_t b = blockIdx.x;
    const uint32_t half = (b >> 3) & 1u;
    const uint32_t worker = ((b >> 4) << 3) | (b & 7u);
    const uint32_t workers = gridDim.x >> 1;
    const uint32_t my_wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // A fused SwiGLU: the first wave of each run of items with the same slot
    // in this block builds that slot's x_hat (the block's items are
    // consecutive, so usually wave 0 alone), the last wave the shared
    // expert's; their loads go out before the plane's.
    const uint32_t item0 = worker * kGemvWaves;
    uint32_t owner = my_wave;  // the wave whose LDS x_hat this wave's expert item reads
    bool routed_owner = false, shared_owner = false;
    uint4 owner_info = make_uint4(0u, 0u, 0u, 0u);
    SwigluInputs routed_in, shared_in;
    if (m.fused_swiglu != 0) {
        const uint32_t lane = threadIdx.x & 63u;
        const uint32_t item = item0 + my_wave;
        if (item < m.expert_items) {
            while (owner > 0 && item_slot(m, item0 + owner - 1u) == item_slot(m, item0 + owner)) {
                --owner;
            }
            routed_owner = owner == my_wave;
            if (routed_owner) {
                const uint4 info = m.slot_info[item_slot(m, item)];
                owner_info = make_uint4(__builtin_amdgcn_readfirstlane(info.x),
                                        __builtin_amdgcn_readfirstlane(info.y),
                                        __builtin_amdgcn_readfirstlane(info.z), 0u);
                routed_owner = owner_info.z > owner_info.y;
                if (routed_owner) {
                    swiglu_issue(m.swiglu, false, owner_info.y, owner_info.x, lane, routed_in);
                }
            }
        }
        shared_owner = my_wave == kGemvWaves - 1u && m.ne_count > 0;
        if (shared_owner) {
            swiglu_issue(m.swiglu, true, 0u, 0u, lane, shared_in);
        }
    }
    float *wave_x_lds = shared_x_lds + kFusedSwigluWidth * (1u + owner);
    // the NE table's words load before the plane: the load counter completes
    // in order, so the plane's wait covers them
    uint32_t tab[kTableWords];
    if (m.ne_count > 0) {
        load_table_share(static_cast<const uint32_t *>(m.ne_book), tab);
    }
    if (m.expert_count > 0) {
        // 8192 16-byte rows per plane, 16 per thread, all loads issued first
        constexpr uint32_t kPer = static_cast<uint32_t>(kPlaneBytes / 16) / kGemvThreads;
        const uint4 *src = static_cast<const uint4 *>(m.expert_book) + half * (kPlaneBytes / 16);
        uint4 v[kPer];
#pragma unroll
        for (uint32_t u = 0; u < kPer; ++u) {
            v[u] = src[u * kGemvThreads + threadIdx.x];
        }
        for (uint32_t s = threadIdx.x; s < m.max_active; s += kGemvThreads) {
            slots[s] = m.slot_info != nullptr
                           ? m.slot_info[s]
                           : make_uint4(0u, 0u, s == 0 ? m.expert[0].batch : 0u, 0u);
        }
        // while the plane is in flight: the owners' x_hat into LDS
        if (routed_owner || shared_owner) {
            const uint32_t lane = threadIdx.x & 63u;
            float x[kFusedSwigluWidth / 64];
            if (routed_owner) {
                swiglu_finish(m.swiglu, false, owner_info.y, lane, routed_in, x);
                store_wave<kFusedSwigluWidth / 64>(wave_x_lds, lane, x);
            }
            if (shared_owner) {
                swiglu_finish(m.swiglu, true, 0u, lane, shared_in, x);
                store_wave<kFusedSwigluWidth / 64>(shared_x_lds, lane, x);
            }
        }
#pragma unroll
        for (uint32_t u = 0; u < kPer; ++u) {
            plane_lds[u * kGemvThreads + threadIdx.x] = v[u];
        }
    }
    if (m.ne_count > 0) {
        store_table_share(tab, ne_table);
    }
    __syncthreads();
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t stride = workers * kGemvWaves;
    const uint2 *plane = reinterpret_cast<const uint2 *>(plane_lds);
    // the wave index is uniform: in scalar registers, the item bookkeeping and
    // every branch on it stay scalar
    uint32_t i = worker * kGemvWaves + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (i < m.expert_items) {
        ExpertStage s0, s1;
        expert_prefetch(m, slots, i, half, lane, s0, m.fused_swiglu != 0 ? wave_x_lds : nullptr);
        while (true) {
            uint32_t j = i + stride;
            if (j < m.expert_items) {
                expert_prefetch(m, slots, j, half, lane, s1);
            }
            expert_compute(m, i, half, plane, lane, s0);
            i = j;
            if (i >= m.expert_items) {
                break;
            }
            j = i + stride;
            if (j < m.expert_items) {
                expert_prefetch(m, slots, j, half, lane, s0);
            }
            expert_compute(m, i, half, plane, lane, s1);
            i = j;
            if (i >= m.expert_items) {
                break;
            }
        }
    }
    // NE items: index k = (i - expert_items) * 2 + half
    const uint32_t end = m.half_items[half];
    if (i < end) {
        NeStage s0, s1;
        ne_prefetch(m, (i - m.expert_items) * 2u + half, lane, s0,
                    m.fused_swiglu != 0 ? shared_x_lds : nullptr);
        while (true) {
            uint32_t j = i + stride;
            if (j < end) {
                ne_prefetch(m, (j - m.expert_items) * 2u + half, lane, s1,
                            m.fused_swiglu != 0 ? shared_x_lds : nullptr);
            }
            ne_compute(m, (i - m.expert_items) * 2u + half, ne_table, lane, s0);
            i = j;
            if (i >= end) {
                break;
            }
            j = i + stride;
            if (j < end) {
                ne_prefetch(m, (j - m.expert_items) * 2u + half, lane, s0,
                            m.fused_swiglu != 0 ? shared_x_lds : nullptr);
            }
            ne_compute(m, (i - m.expert_items) * 2u + half, ne_table, lane, s1);
            i = j;
            if (i >= end) {
                break;
            }
        }
    }
}

// ---- the MoE block of one row in one launch ----------------------------------
//
// Phases (B = 1; items and slices as in the separate launches):
//   P0  every block: codebook plane and NE table into LDS; wave 7 computes one
//       or two router logits (rows b and b + blocks; row `experts` is the
//       shared-expert gate) in the CPU's ISA order and takes a ticket; the
//       last block to do so runs top_experts and publishes the routes. Wave 0
//       of blocks 0 and 1 publishes the shared expert's gate and up x_hat.
//   P1  wave 7 copies the routes into the block's slot table and builds the
//       x_hat of the block's (entry, slot); each wave runs its routed gate/up
//       item (its codes in flight meanwhile). The last wave of the block to
//       finish adds the block's items to its slot's counter. Waves 4 and 5 then
//       run the shared gate/up NE items.
//   P2  wave 0 waits for the slot of the block's down items, builds its
//       SwiGLU x_hat; each wave runs its down item; wave 1 builds the shared
//       SwiGLU x_hat and runs a shared down NE item.
//   P3  the last block to finish combines the eight routes and the shared
//       expert in route order (the combine launch's arithmetic) and clears the
//       counters for the next call.
// The grid is one block per CU and every block is resident (LDS admits one
// per CU); waits are bounded and a wait that runs out sets a bit of the error
// word (the host reports it), so no call can hang.
// Hand-over data (logits, routes, x_hat, Z slices) is written with coherent
// (write-through) stores and waited for before the counter that publishes
// it; consumers read it after the counter with ordinary loads, which are
// their first touch of those lines in the launch (the launch starts with
// clean caches, every line holds one producer's data), so no cache can hold
// a stale copy. Counters and flags themselves are read with coherent loads.

// The sync buffer is cut into lines of kMoeSyncLine words (4 KiB), one per
// counter or flag, so that pollers and atomics of different words meet in
// different memory channels. A flag that every block polls is written to
// eight replica lines; block b polls replica b % 8 (its XCD's, as blocks are
// dealt to the XCDs round robin), and the counters behind it are polled by
// one wave only (the publisher), so they take their atomics undisturbed.
// Grid-wide tickets count in two levels: eight group lines of up to 32
// blocks each, then a top line. The logits
// line holds the router logits as complemented bits, so its cleared state
// (zero) reads as "not written yet" (a logit whose bits are all ones, one
// particular NaN, would never read as written: its wait runs out).
namespace moe_sync {
constexpr uint32_t kSharedGroup = 0, kSharedReady = 8, kSlotCount = 16, kDownCount = 24,
                   kSharedDownGroup = 32, kSharedDownTop = 40, kCombineTicket = 41, kCounterLines = 42,
                   kLogits = 42,
                   kError = kMoeSyncError / kMoeSyncLine, kParts = 46;
// kParts: the combine's nine rows (routes 0-7, then the shared expert), two
// lines each
// words of a block's route record in LDS
constexpr uint32_t kToGrouped = 0, kRouteWeight = 8;
}  // namespace moe_sync

__device__ __forceinline__ uint32_t *sync_line(uint32_t *sync, uint32_t line) {
    return sync + static_cast<size_t>(line) * kMoeSyncLine;
}

constexpr uint32_t kFusedThreads = kGemvThreads + kWave;  // eight GEMV waves and a helper
constexpr uint32_t kFusedSlots = 8;
constexpr uint32_t kSpinLimit = 1u << 20;  // about a second of polling
constexpr size_t kFusedRegion = 16384;     // LDS after the plane: staging and x_hat rows

// Polls (the whole wave) until *word is nonzero and returns it; bounded (0
// after a timeout, which sets `bit` of the error word).
__device__ __forceinline__ uint32_t wait_nonzero(uint32_t *word, uint32_t *error, uint32_t bit) {
    uint32_t older = coherent_load(word);
    for (uint32_t spins = 0;; ++spins) {
        __builtin_amdgcn_s_sleep(1);
        const uint32_t newer = coherent_load(word);
        const uint32_t v = __builtin_amdgcn_readfirstlane(older);
        if (v != 0u) {
            return v;
        }
        if (spins >= kSpinLimit) {
            if ((threadIdx.x & 63u) == 0) {
                __hip_atomic_fetch_or(error, bit, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            return 0u;
        }
        older = newer;
    }
}

// Polls the logits line (16-byte coherent loads, lane l words 4l .. 4l + 3)
// until the first `count` words are all written (nonzero), then stores the
// logits (the words complemented back) into `out` in LDS; bounded (a timeout
// sets error bit 1 and leaves zeros, which still route).
__device__ __forceinline__ void wait_logits(uint32_t *words, uint32_t count, uint32_t lane, float *out,
                                            uint32_t *error) {
    typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(words, 0, 1024, 0x00020000);
    u32x4_t q = __builtin_amdgcn_raw_buffer_load_b128(rs, lane * 16u, 0, 16 /* sc1 */);
    for (uint32_t spins = 0;; ++spins) {
        bool in = true;
#pragma unroll
        for (uint32_t i = 0; i < 4; ++i) {
            in = in && (4u * lane + i >= count || q[i] != 0u);
        }
        if (__all(in ? 1 : 0)) {
            break;
        }
        if (spins >= kSpinLimit) {
            if (lane == 0) {
                __hip_atomic_fetch_or(error, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            break;
        }
        __builtin_amdgcn_s_sleep(1);
        q = __builtin_amdgcn_raw_buffer_load_b128(rs, lane * 16u, 0, 16);
    }
#pragma unroll
    for (uint32_t i = 0; i < 4; ++i) {
        if (4u * lane + i < count) {
            out[4u * lane + i] = __uint_as_float(~q[i]);
        }
    }
}

// Polls (the whole wave, uniformly) until *word >= target; bounded. Two
// loads are in flight at a time, so a change is seen about half a load
// latency after it lands rather than up to a whole one.
__device__ __forceinline__ void wait_count(uint32_t *word, uint32_t target, uint32_t *error,
                                           uint32_t bit) {
    uint32_t older = coherent_load(word);
    for (uint32_t spins = 0;; ++spins) {
        __builtin_amdgcn_s_sleep(1);
        const uint32_t newer = coherent_load(word);
        if (__builtin_amdgcn_readfirstlane(older) >= target) {
            return;
        }
        if (spins >= kSpinLimit) {
            if ((threadIdx.x & 63u) == 0) {
                __hip_atomic_fetch_or(error, bit, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            return;
        }
        older = newer;
    }
}

// An LDS flag of the block: set (release) by one wave, awaited (acquire;
// bounded like wait_count, error bit 16).
__device__ __forceinline__ void set_flag(uint32_t *flag) {
    __hip_atomic_store(flag, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ void wait_flag(uint32_t *flag, uint32_t *error) {
    for (uint32_t spins = 0; __builtin_amdgcn_readfirstlane(__hip_atomic_load(
                                 flag, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP)) == 0u;
         ++spins) {
        if (spins >= 16u * kSpinLimit) {
            if ((threadIdx.x & 63u) == 0) {
                __hip_atomic_fetch_or(error, 16u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            return;
        }
        __builtin_amdgcn_s_sleep(1);
    }
}

// count_block without a result: the device add is fire-and-forget.
__device__ __forceinline__ void count_block_quiet(uint32_t *lds_count, uint32_t waves, uint32_t *word) {
    wait_stores();
    if ((threadIdx.x & 63u) == 0 && atomicAdd(lds_count, 1u) + 1u == waves) {
        (void)__hip_atomic_fetch_add(word, waves, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// Waits (bounded) until an LDS word reaches at least `at_least`, returns it.
__device__ __forceinline__ uint32_t wait_lds_value(uint32_t *word, uint32_t at_least, uint32_t *error) {
    for (uint32_t spins = 0;; ++spins) {
        const uint32_t v = __builtin_amdgcn_readfirstlane(
            __hip_atomic_load(word, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP));
        if (v >= at_least) {
            return v;
        }
        if (spins >= 16u * kSpinLimit) {
            if ((threadIdx.x & 63u) == 0) {
                __hip_atomic_fetch_or(error, 16u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            return at_least;
        }
        __builtin_amdgcn_s_sleep(1);
    }
}

// An LDS arrival counter of the block: count the wave in (release), then
// wait (acquire, bounded) until `target` waves have arrived.
__device__ __forceinline__ void arrive_and_wait(uint32_t *count, uint32_t target, uint32_t *error) {
    if ((threadIdx.x & 63u) == 0) {
        __hip_atomic_fetch_add(count, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
    for (uint32_t spins = 0; __builtin_amdgcn_readfirstlane(__hip_atomic_load(
                                 count, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP)) < target;
         ++spins) {
        if (spins >= 16u * kSpinLimit) {
            if ((threadIdx.x & 63u) == 0) {
                __hip_atomic_fetch_or(error, 16u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            return;
        }
        __builtin_amdgcn_s_sleep(1);
    }
}

// Counts the wave into the block's LDS counter; the wave that completes
// `waves` adds them to the device counter (its own stores and those of the
// counted waves are complete: each waits for them before counting). True in
// the wave whose add brings the device counter to `total`.
__device__ __forceinline__ bool count_block(uint32_t *lds_count, uint32_t waves, uint32_t *word,
                                           uint32_t total = 0xFFFFFFFFu) {
    wait_stores();
    uint32_t completes = 0;
    if ((threadIdx.x & 63u) == 0) {
        if (atomicAdd(lds_count, 1u) + 1u == waves) {
            completes = coherent_add(word, waves) + waves == total ? 1u : 0u;
        }
    }
    return __builtin_amdgcn_readfirstlane(completes) != 0u;
}

// One row of the combine (k_combine_wave): weight * (sv * H(sum of the Z
// slices)), written through to `dst`. sv is f16 (a routed expert's, in LDS)
// or +-1 (the shared expert's).
template <int VPL>
__device__ __forceinline__ void combine_row(const float *z, size_t stride, uint32_t splits,
                                            const uint16_t *sv_f16, const int8_t *sv_sign,
                                            float weight, float scale_h, uint32_t lane, float *dst) {
#pragma clang fp contract(off)
    float val[VPL], sv[VPL];
    sum_slices<VPL>(z, stride, splits, lane, val);
    if (sv_f16 != nullptr) {
        load_wave_f16<VPL>(sv_f16, lane, sv);
    } else {
        load_wave_sign<VPL>(sv_sign, lane, sv);
    }
    wave_hadamard<VPL>(val, scale_h, lane);
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
        val[i] = weight * (val[i] * sv[i]);
    }
    store_wave_through<VPL>(dst, lane, val);
}

// Two-level ticket over the grid, taken by one thread per block once the
// block's stores are complete: true in the one block that completes it.
__device__ __forceinline__ bool grid_ticket(uint32_t *sync, uint32_t group_line, uint32_t top_line,
                                            uint32_t b, uint32_t blocks) {
    const uint32_t group = b & 7u;
    const uint32_t members = (blocks - group + 7u) >> 3;
    if (coherent_add(sync_line(sync, group_line + group), 1u) + 1u != members) {
        return false;
    }
    const uint32_t groups = blocks < 8u ? blocks : 8u;
    return coherent_add(sync_line(sync, top_line), 1u) + 1u == groups;
}

// Polls (the whole wave) the eight group lines from `first` until group g
// (the blocks b with b % 8 == g) has counted `per_block` for each of its
// blocks; lane g loads group g's line, so each round is one load latency.
// Bounded: a timeout sets `bit` of the error word.
__device__ __forceinline__ void wait_groups(uint32_t *sync, uint32_t first, uint32_t per_block,
                                            uint32_t blocks, uint32_t lane, uint32_t *error,
                                            uint32_t bit) {
    const uint32_t g = lane & 7u;
    const uint32_t target = g < blocks ? per_block * ((blocks - g + 7u) >> 3) : 0u;
    uint32_t *word = sync_line(sync, first + g);
    for (uint32_t spins = 0;; ++spins) {
        if (__all(coherent_load(word) >= target ? 1 : 0)) {
            return;
        }
        if (spins >= kSpinLimit) {
            if (lane == 0) {
                __hip_atomic_fetch_or(error, bit, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            return;
        }
        __builtin_amdgcn_s_sleep(1);
    }
}

// Sets the eight replicas of a flag every block polls.
__device__ __forceinline__ void publish_flag(uint32_t *sync, uint32_t line) {
#pragma unroll
    for (uint32_t x = 0; x < 8; ++x) {
        coherent_store(sync_line(sync, line + x), 1u);
    }
}

// The 2048-point transform of x * m by the eight GEMV waves of a block, in
// two steps with a block barrier between them. Step one: wave w transforms
// elements 256 w .. 256 w + 255 (index bits 0-7; element 64 i + lane of its
// chunk in register i) into `dst`. Step two: each wave takes 32 of the 256
// columns across the eight chunks (index bits 8-10) and scales. Every
// butterfly is the one-wave transform's (wave_hadamard over 2048), in the
// same order, so the result is bit-identical to it.
__device__ __forceinline__ void hadamard_chunk(const float *x, const float (&m)[4], uint32_t wave,
                                               uint32_t lane, float *dst) {
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        v[i] = x[256u * wave + 64u * i + lane] * m[i];
    }
    wave_hadamard<4>(v, 1.0f, lane);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        dst[256u * wave + 64u * i + lane] = v[i];
    }
}
// Step two for any chunk of SPAN elements (SPAN / 8 columns per wave).
template <uint32_t SPAN>
__device__ __forceinline__ void hadamard_cross_span(float *dst, float scale, uint32_t wave, uint32_t lane) {
#pragma clang fp contract(off)
    constexpr uint32_t per_wave = SPAN / 8u;
    for (uint32_t j = per_wave * wave + lane; j < per_wave * (wave + 1u); j += 64u) {
        float u[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            u[k] = dst[SPAN * k + j];
        }
#pragma unroll
        for (int stride = 1; stride < 8; stride <<= 1) {
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                if ((k & stride) == 0) {
                    const float p = u[k], q = u[k + stride];
                    u[k] = p + q;
                    u[k + stride] = p - q;
                }
            }
        }
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            dst[SPAN * k + j] = u[k] * scale;
        }
    }
}
// hadamard_cross_span with the result times a sign row written to `out`
// instead of back into `src`: out[i] = (u * scale) * signs[i], the values
// the in-place transform and a sign pass over it give.
template <uint32_t SPAN>
__device__ __forceinline__ void hadamard_cross_span_out(const float *src, float scale, uint32_t wave, uint32_t lane,
                                                        const int8_t *signs, float *out) {
#pragma clang fp contract(off)
    constexpr uint32_t per_wave = SPAN / 8u;
    for (uint32_t j = per_wave * wave + lane; j < per_wave * (wave + 1u); j += 64u) {
        float u[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            u[k] = src[SPAN * k + j];
        }
#pragma unroll
        for (int stride = 1; stride < 8; stride <<= 1) {
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                if ((k & stride) == 0) {
                    const float p = u[k], q = u[k + stride];
                    u[k] = p + q;
                    u[k + stride] = p - q;
                }
            }
        }
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const float v = u[k] * scale;
            out[SPAN * k + j] = v * static_cast<float>(signs[SPAN * k + j]);
        }
    }
}
// ---- block-per-vector prologue / epilogue (n = 2048, 4096; 8192 too) -----
//
// A launch of few vectors (a prefill chunk's attention projections: 128-384)
// leaves most CUs idle with one wave a vector, each wave running a whole
// 2048- or 4096-point transform. Here a vector takes a block of eight waves:
// wave w transforms elements w n/8 .. (w + 1) n/8 - 1 (the index bits below
// 8 or 9, in the wave layout of that chunk), then the waves run the last
// three index bits across the chunks in LDS (hadamard_cross_span): every
// butterfly is the one-wave transform's, in the same order, so the results
// are bit-identical to the one-wave kernels'.
constexpr uint32_t kBlockVectors = 512;  // vectors up to which a vector takes a block

// x_hat of vector v from LDS (n values, already scaled) in out's layout, by
// the block's 512 threads: f32 rows, f16 hi/lo rows, or the two codebook
// planes of each 16-column tile (store_xhat's layouts).
__device__ __forceinline__ void store_xhat_lds(const XhatOut &out, uint32_t v, const float *x, uint32_t n) {
#pragma clang fp contract(off)
    if (out.planes == 0) {
        float4 *dst = reinterpret_cast<float4 *>(out.f32 + static_cast<size_t>(v) * n);
        for (uint32_t i = threadIdx.x; i < n / 4u; i += 512u) {
            dst[i] = reinterpret_cast<const float4 *>(x)[i];
        }
        return;
    }
    const auto split = [](float f, uint32_t &hi, uint32_t &lo) {
        hi = f16_bits_rne(f);
        lo = f16_bits_rne(f - half_bits_to_float(hi));
    };
    if (out.planes == 1) {
        for (uint32_t i = threadIdx.x; i < n / 4u; i += 512u) {
            const float4 q = reinterpret_cast<const float4 *>(x)[i];
            uint32_t h[4], l[4];
            split(q.x, h[0], l[0]);
            split(q.y, h[1], l[1]);
            split(q.z, h[2], l[2]);
            split(q.w, h[3], l[3]);
            *reinterpret_cast<uint2 *>(out.hi + static_cast<size_t>(v) * n + 4u * i) =
                make_uint2(h[0] | h[1] << 16, h[2] | h[3] << 16);
            *reinterpret_cast<uint2 *>(out.lo + static_cast<size_t>(v) * n + 4u * i) =
                make_uint2(l[0] | l[1] << 16, l[2] | l[3] << 16);
        }
        return;
    }
    // (tile, plane) pairs: the plane's columns 4 p .. 4 p + 3 and 8 + 4 p ..
    // 8 + 4 p + 3 of the tile, in that order, one 16-byte store each
    for (uint32_t t = threadIdx.x; t < n / 8u; t += 512u) {
        const uint32_t tile = t >> 1, plane = t & 1u, c = tile * 16u + 4u * plane;
        const float4 a = *reinterpret_cast<const float4 *>(x + c);
        const float4 b = *reinterpret_cast<const float4 *>(x + c + 8u);
        const float f[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
        uint32_t h[8], l[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            split(f[k], h[k], l[k]);
        }
        const size_t at = static_cast<size_t>(plane) * out.vectors * (n / 2u) + static_cast<size_t>(v) * (n / 2u) +
                          tile * 8u;
        *reinterpret_cast<uint4 *>(out.hi + at) =
            make_uint4(h[0] | h[1] << 16, h[2] | h[3] << 16, h[4] | h[5] << 16, h[6] | h[7] << 16);
        *reinterpret_cast<uint4 *>(out.lo + at) =
            make_uint4(l[0] | l[1] << 16, l[2] | l[3] << 16, l[4] | l[5] << 16, l[6] | l[7] << 16);
    }
}

// prologue_vector for vector blockIdx.x by a block: x_hat = H_n(x[src] * su).
template <int VC>
__global__ __launch_bounds__(512) void k_prologue_block(PrologueJobs j) {
#pragma clang fp contract(off)
    constexpr uint32_t n = 512u * VC, CH = 64u * VC;
    __shared__ __align__(16) float x_lds[n];
    uint32_t v = blockIdx.x, s = 0;
    while (s < j.segments && v >= j.seg[s].count) {
        v -= j.seg[s].count;
        ++s;
    }
    if (s >= j.segments) {
        return;  // the whole block
    }
    const PrologueSegment &g = j.seg[s];
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    const uint32_t src = g.source_row != nullptr ? g.source_row[v] : v;
    const uint32_t mat = g.matrix_index != nullptr ? g.matrix_index[v] : 0u;
    float val[VC], su[VC];
    load_wave<VC>(g.x + static_cast<size_t>(src) * n + wave * CH, lane, val);
    if (g.su_f16 != nullptr) {
        load_wave_f16<VC>(g.su_f16 + static_cast<size_t>(mat) * g.su_stride + wave * CH, lane, su);
    } else {
        load_wave_sign<VC>(g.su_sign + wave * CH, lane, su);
    }
#pragma unroll
    for (int i = 0; i < VC; ++i) {
        val[i] = val[i] * su[i];
    }
    wave_hadamard<VC>(val, 1.0f, lane);
    store_wave<VC>(x_lds + wave * CH, lane, val);
    __syncthreads();
    hadamard_cross_span<CH>(x_lds, j.scale, wave, lane);
    __syncthreads();
    store_xhat_lds(g.out, v, x_lds, n);
}

// k_epilogue_wave (k_epilogue_8192 at 8192 points) for vector blockIdx.x by
// a block: y = sv * H_n(sum over splits of z), the last butterflies writing
// y.
template <int VC, typename Scale>
__global__ __launch_bounds__(512) void k_epilogue_block(const float *__restrict__ z, uint32_t splits,
                                                        size_t split_stride, const Scale *__restrict__ sv,
                                                        float scale, float *__restrict__ out) {
#pragma clang fp contract(off)
    constexpr uint32_t n = 512u * VC, CH = 64u * VC;
    __shared__ __align__(16) float y_lds[n];
    const uint32_t v = blockIdx.x, wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    float val[VC];
    sum_slices_deep<VC>(z + static_cast<size_t>(v) * n + wave * CH, split_stride, splits, lane, val);
    wave_hadamard<VC>(val, 1.0f, lane);
    store_wave<VC>(y_lds + wave * CH, lane, val);
    __syncthreads();
    float *dst = out + static_cast<size_t>(v) * n;
    for (uint32_t jj = CH / 8u * wave + lane; jj < CH / 8u * (wave + 1u); jj += 64u) {
        float u[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            u[k] = y_lds[CH * k + jj];
        }
#pragma unroll
        for (int stride = 1; stride < 8; stride <<= 1) {
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                if ((k & stride) == 0) {
                    const float p = u[k], q = u[k + stride];
                    u[k] = p + q;
                    u[k + stride] = p - q;
                }
            }
        }
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const float w = u[k] * scale;
            dst[CH * k + jj] = w * scale_value<Scale>(sv[CH * k + jj]);
        }
    }
}

__device__ __forceinline__ void hadamard_cross(float *dst, float scale, uint32_t wave, uint32_t lane) {
#pragma clang fp contract(off)
    if (lane < 32) {
        const uint32_t j = 32u * wave + lane;
        float u[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            u[k] = dst[256u * k + j];
        }
#pragma unroll
        for (int stride = 1; stride < 8; stride <<= 1) {
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                if ((k & stride) == 0) {
                    const float p = u[k], q = u[k + stride];
                    u[k] = p + q;
                    u[k + stride] = p - q;
                }
            }
        }
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            dst[256u * k + j] = u[k] * scale;
        }
    }
}

// The thread's share of a codebook plane into LDS: all loads, then the stores.
__device__ __forceinline__ void fill_plane_share(const uint4 *src, uint4 *dst) {
    constexpr uint32_t kPer = static_cast<uint32_t>(kPlaneBytes / 16) / kGemvThreads;
    uint4 v[kPer];
#pragma unroll
    for (uint32_t u = 0; u < kPer; ++u) {
        v[u] = src[u * kGemvThreads + threadIdx.x];
    }
#pragma unroll
    for (uint32_t u = 0; u < kPer; ++u) {
        dst[u * kGemvThreads + threadIdx.x] = v[u];
    }
}

// A combine row is in (the calling wave's stores and those it waited for
// are complete): true for the ninth of the eight route rows and the shared
// row to arrive, whose block then adds them. Every other wait of the launch
// has ended by then: each row needs all its slot's down items (whose waves
// have polled everything) and the shared row every helper's down item.
__device__ __forceinline__ bool combine_ticket(uint32_t *sync, uint32_t lane) {
    wait_stores();
    uint32_t ticket = 0;
    if (lane == 0) {
        ticket = coherent_add(sync_line(sync, moe_sync::kCombineTicket), 1u);
    }
    return __builtin_amdgcn_readfirstlane(ticket) == 8u;
}

// The last combine ticket's block (`threads` threads from `first`): clears
// the counters and route words for the next call, then adds the nine rows
// in route order, then the shared expert (the combine launch's order).
__device__ __forceinline__ void finish_combine(const MoeDecodeOne &a, uint32_t *sync, uint32_t t0,
                                               uint32_t threads) {
    for (uint32_t t = t0; t < moe_sync::kCounterLines; t += threads) {
        coherent_store(sync_line(sync, t), 0u);
    }
    for (uint32_t t = t0; t < 257u; t += threads) {
        coherent_store(sync_line(sync, moe_sync::kLogits) + t, 0u);
    }
    constexpr uint32_t H = kFusedHidden;
    float4 *row_out = reinterpret_cast<float4 *>(a.out);
    for (uint32_t c = t0; c < H / 4u; c += threads) {
        float4 v[9];
#pragma unroll
        for (uint32_t r = 0; r < 9; ++r) {
            v[r] = reinterpret_cast<const float4 *>(sync_line(sync, moe_sync::kParts + 2u * r))[c];
        }
        float4 acc = v[0];
#pragma unroll
        for (uint32_t r = 1; r < 9; ++r) {
            acc.x = acc.x + v[r].x;
            acc.y = acc.y + v[r].y;
            acc.z = acc.z + v[r].z;
            acc.w = acc.w + v[r].w;
        }
        row_out[c] = acc;
    }
}

template <int LANES>
__global__ __launch_bounds__(kFusedThreads) void k_moe_decode_one(MoeDecodeOne a) {
#pragma clang fp contract(off)
    extern __shared__ uint4 lds_dynamic[];  // the codebook plane, then kFusedRegion bytes
    __shared__ uint32_t ne_table[1024];
    __shared__ uint4 slots[kFusedSlots];
    // the block's routing: expert and weight bits of each route (top8_wave's
    // output), then the route record: grouped position and weight bits of
    // each route, the shared gate logit
    __shared__ uint32_t routes[16];
    __shared__ uint32_t record_lds[16];
    __shared__ uint16_t su_lds[kFusedHidden];  // su (f16) of the block's gate/up entry and slot
    __shared__ float bias_lds[kFusedMaxExperts];  // the routing bias, staged before the logits arrive
    // the logits as the helper collects them (the region is busy with the
    // shared x_hat meanwhile)
    __shared__ float logits_lds[kFusedMaxExperts];
    // 0: waves that filled their plane share and table part; 1: slot table;
    // 2, 8: waves through the two halves of the routed x_hat (2 again for the
    // combine row); 3: gate/up items counted; 4: down x_hat; 5: shared
    // gate/up items counted; 6: down items counted; 7: the router's staged
    // rows read (their space free); 9: the block's slot-completion state;
    // 10: combine row stores counted; 11: P0 barrier arrivals
    __shared__ uint32_t flags[12];
    constexpr uint32_t H = kFusedHidden;
    constexpr int VPL = kFusedHidden / 64;
    constexpr int VPLI = kFusedSwigluWidth / 64;
    uint4 *plane_lds = lds_dynamic;
    float *region = reinterpret_cast<float *>(lds_dynamic + kPlaneBytes / 16);
    float *x_routed = region;       // P1: x_hat of the block's (entry, slot)
    float *x_staged = region + H;   // P0-P1: x as the router staged it
    float *x_down = region + H;     // P2: the slot's SwiGLU x_hat (x no longer needed)
    float *x_shared_down = region + H + kFusedSwigluWidth;  // P1: the shared SwiGLU x_hat
    uint16_t *sv_slot = reinterpret_cast<uint16_t *>(region + H + 2 * kFusedSwigluWidth);  // P2: f16 sv
    const uint32_t b = blockIdx.x, blocks = gridDim.x;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t lane = threadIdx.x & 63u;
    const bool helper = wave == kGemvWaves;
    const uint32_t half = (b >> 3) & 1u;
    // Routed slot s lives on XCD s (blocks are dealt to the eight XCDs round
    // robin, XCD b % 8): its gate and up items, the down x_hat built from
    // their Z slices, its down items and its combine row all run on one XCD,
    // so the hand-over data is read from that XCD's L2. Block b, the m-th of
    // its (XCD, half) pair, takes gate or up items (m below or above half the
    // pair's blocks) and its share of the slot's down items.
    const uint32_t xcd = b & 7u, m_block = b >> 4;
    const uint32_t per_entry = a.gu.expert_items_per_slot / kGemvWaves;  // blocks per (entry, half)
    const uint32_t gu_which = m_block >= per_entry ? 1u : 0u;
    const uint32_t item_gu = ((gu_which * kFusedSlots + xcd) * per_entry + (m_block - gu_which * per_entry)) *
                                 kGemvWaves + wave;
    const uint32_t item_dn = (xcd * (a.dn.expert_items_per_slot / kGemvWaves) + m_block) * kGemvWaves + wave;
    uint32_t *sync = a.sync;
    uint32_t *error = sync_line(sync, moe_sync::kError);
    uint32_t *logit_words = sync_line(sync, moe_sync::kLogits);  // complemented bits
    auto part = [&](uint32_t r) { return reinterpret_cast<float *>(sync_line(sync, moe_sync::kParts + 2u * r)); };
    // the block's routed slots: gate/up items (P1) and down items (P2)
    const uint32_t slot1 = expert_item_of(a.gu, item_gu - wave).slot;
    const uint32_t slot2 = expert_item_of(a.dn, item_dn - wave).slot;
    if (threadIdx.x < 12) {
        flags[threadIdx.x] = 0u;
    }
    __syncthreads();
    // waits (bounded) until the eight GEMV waves have counted into an LDS
    // counter: flags[0] says the plane and the NE table are complete,
    // flags[2] that the staged x has been read for the routed x_hat
    auto wait_waves = [&](uint32_t *count) {
        for (uint32_t spins = 0; __builtin_amdgcn_readfirstlane(__hip_atomic_load(
                                     count, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP)) < kGemvWaves;
             ++spins) {
            if (spins >= 16u * kSpinLimit) {
                if (lane == 0) {
                    __hip_atomic_fetch_or(error, 16u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
                return;
            }
            __builtin_amdgcn_s_sleep(1);
        }
    };
    auto wait_plane = [&]() { wait_waves(&flags[0]); };

    // ---- P0 ----
    if (!helper) {
        // the NE table's words go out first; the plane's wait covers them
        uint32_t tab[kTableWords];
        load_table_share(static_cast<const uint32_t *>(a.gu.ne_book), tab);
        fill_plane_share(static_cast<const uint4 *>(a.gu.expert_book) + half * (kPlaneBytes / 16),
                         plane_lds);
        store_table_share(tab, ne_table);
        if (lane == 0) {
            __hip_atomic_fetch_add(&flags[0], 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
        }
    } else {
        // router rows b and 2 blocks - 1 - b (the second rows, the shared
        // gate's among them, on the last blocks), staged with x in the region
        const uint32_t rows_total = a.experts + 1u;
        uint16_t *wl = reinterpret_cast<uint16_t *>(region);
        const uint32_t r0 = b;
        const uint32_t r1 = 2u * blocks - 1u - b;
        auto row = [&](uint32_t r) {
            return reinterpret_cast<const uint4 *>(r < a.experts ? a.router + static_cast<size_t>(r) * H
                                                                 : a.shared_gate_row);
        };
        uint4 w0[4], w1[4];
        float4 xv[8];
#pragma unroll
        for (uint32_t u = 0; u < 4; ++u) {
            w0[u] = r0 < rows_total ? row(r0)[u * 64u + lane] : make_uint4(0u, 0u, 0u, 0u);
            w1[u] = r1 < rows_total ? row(r1)[u * 64u + lane] : make_uint4(0u, 0u, 0u, 0u);
        }
#pragma unroll
        for (uint32_t u = 0; u < 8; ++u) {
            xv[u] = reinterpret_cast<const float4 *>(a.x)[u * 64u + lane];
        }
#pragma unroll
        for (uint32_t u = 0; u < 4; ++u) {
            reinterpret_cast<uint4 *>(wl)[u * 64u + lane] = w0[u];
            reinterpret_cast<uint4 *>(wl + H)[u * 64u + lane] = w1[u];
        }
#pragma unroll
        for (uint32_t u = 0; u < 8; ++u) {
            reinterpret_cast<float4 *>(x_staged)[u * 64u + lane] = xv[u];
        }
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        const uint32_t group = lane / LANES;  // 0: row r0, 1: row r1, others unused
        const float acc = router_chain<LANES>(wl + (group == 1u ? H : 0u), x_staged, H, lane % LANES);
        const float s0 = router_lane_sum<LANES>(acc, 0u);
        const float s1 = router_lane_sum<LANES>(acc, 1u);
        set_flag(&flags[7]);  // the staged rows are read
        // rows 0 .. experts - 1 are the router's, row `experts` the shared
        // gate's; every block's helper polls them (no ticket)
        if (lane == 0) {
            if (r0 < rows_total) {
                coherent_store(logit_words + r0, ~__float_as_uint(s0));
            }
            if (r1 < rows_total) {
                coherent_store(logit_words + r1, ~__float_as_uint(s1));
            }
        }
    }
    // the shared expert's gate/up NE items while the router finishes: the
    // first half of the blocks takes the gate's items, the second the up's,
    // two consecutive ones per block on waves 6 and 7, so that a block needs
    // the x_hat of one matrix only. The eight waves build it in x_routed's
    // space (free until the routes) as in P1; waves 6 and 7 take their x
    // from it, run the items and count them, all before the routed codes
    // load the memory system. Each block counts into its group line (b % 8)
    // without waiting for the count; block 0's helper publishes the shared
    // flag once every group line is full.
    const uint32_t shared_which = b < blocks / 2u ? 0u : 1u;
    const uint32_t shared_first = 2u * (b - shared_which * (blocks / 2u));  // within the matrix
    const uint32_t shared_mine = (shared_first < a.gu.ne_items_per_matrix ? 1u : 0u) +
                                 (shared_first + 1u < a.gu.ne_items_per_matrix ? 1u : 0u);
    const bool shared_item = !helper && wave >= 6u && wave - 6u < shared_mine;
    const uint32_t shared_k = shared_which * a.gu.ne_items_per_matrix + shared_first + (wave - 6u);
    if (!helper) {
        float sign[4];
        const int8_t *su_shared = shared_which == 0u ? a.shared_su_gate : a.shared_su_up;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            sign[i] = static_cast<float>(su_shared[256u * wave + 64u * i + lane]);
        }
        // arrivals of the eight waves at the n-th P0 barrier: flags[11] >= 8 n
        // (each wave's LDS reads and writes complete before it arrives)
        uint32_t barriers = 0;
        auto p0_barrier = [&]() {
            __builtin_amdgcn_s_waitcnt(kWaitLds);
            if (lane == 0) {
                __hip_atomic_fetch_add(&flags[11], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            }
            wait_lds_value(&flags[11], kGemvWaves * ++barriers, error);
        };
        wait_lds_value(&flags[7], 1u, error);
        NeStage st;
        hadamard_chunk(x_staged, sign, wave, lane, x_routed);
        p0_barrier();
        hadamard_cross(x_routed, a.scale_hidden, wave, lane);
        p0_barrier();
        if (shared_item) {
            ne_prefetch(a.gu, shared_k, lane, st, x_routed);
        }
        p0_barrier();  // x_routed is free again
        if (shared_item) {
            wait_plane();
            ne_compute<true>(a.gu, shared_k, ne_table, lane, st);
        }
        if (wave >= 6u) {
            // both waves count (also one without an item): 2 per block
            count_block_quiet(&flags[5], 2u, sync_line(sync, moe_sync::kSharedGroup + (b & 7u)));
        }
    }

    // ---- P1 ----
    const uint2 *plane = reinterpret_cast<const uint2 *>(plane_lds);
    if (helper) {
        // every block routes the row itself once all logits are in: the
        // same top_experts over the same logits in every block
        float *logits = logits_lds;
        if (a.logit_bias != nullptr) {
            for (uint32_t e = lane; e < a.experts; e += 64u) {
                bias_lds[e] = a.logit_bias[e];
            }
        }
        wait_logits(logit_words, a.experts, lane, logits, error);
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        uint32_t chosen[8];
        top8_wave<4>(logits, a.logit_bias != nullptr ? bias_lds : nullptr, a.experts, lane, routes,
                     reinterpret_cast<float *>(routes + 8), nullptr, chosen);
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        // slot s: the s-th smallest chosen expert (the counting sort's
        // grouped order for one row); route r sits at grouped position rank(r)
        if (lane < 8) {
            uint32_t e = chosen[0];
#pragma unroll
            for (uint32_t q = 1; q < 8; ++q) {
                e = lane == q ? chosen[q] : e;
            }
            uint32_t rank = 0;
#pragma unroll
            for (uint32_t q = 0; q < 8; ++q) {
                rank += chosen[q] < e ? 1u : 0u;
            }
            slots[rank] = make_uint4(e, rank, rank + 1u, 0u);
            record_lds[moe_sync::kToGrouped + lane] = rank;
            record_lds[moe_sync::kRouteWeight + lane] = routes[8 + lane];
            if (b == 0 && a.route_expert_out != nullptr) {
                a.route_expert_out[lane] = e;
            }
            if (b == 0 && a.route_weight_out != nullptr) {
                a.route_weight_out[lane] = __uint_as_float(routes[8 + lane]);
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        {
            // su of the block's (entry, slot) into LDS, loaded before the
            // GEMV waves' codes flood the memory queues
            const ExpertItem it = expert_item_of(a.gu, item_gu - wave);
            const uint4 *src = reinterpret_cast<const uint4 *>(
                (it.which == 0 ? a.su_gate : a.su_up) + static_cast<size_t>(slots[slot1].x) * H);
            uint4 q[4];
#pragma unroll
            for (uint32_t u = 0; u < 4; ++u) {
                q[u] = src[u * 64u + lane];
            }
#pragma unroll
            for (uint32_t u = 0; u < 4; ++u) {
                reinterpret_cast<uint4 *>(su_lds)[u * 64u + lane] = q[u];
            }
        }
        set_flag(&flags[1]);
        // the shared expert's SwiGLU x_hat (every block's helper builds it
        // from the published gate/up slices), then its down NE item b; the
        // block that completes those builds the shared combine row
        wait_plane();
        if (b == 0) {
            wait_groups(sync, moe_sync::kSharedGroup, 2u, blocks, lane, error, 8u);
            if (lane == 0) {
                publish_flag(sync, moe_sync::kSharedReady);
            }
        } else {
            wait_count(sync_line(sync, moe_sync::kSharedReady + (b & 7u)), 1u, error, 8u);
        }
        SwigluInputs in;
        float xd[VPLI];
        swiglu_issue(a.dn.swiglu, true, 0u, 0u, lane, in);
        swiglu_finish(a.dn.swiglu, true, 0u, lane, in, xd);
        wait_waves(&flags[2]);  // x_shared_down overlays the staged x
        store_wave<VPLI>(x_shared_down, lane, xd);
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        NeStage st;
        ne_prefetch(a.dn, b, lane, st, x_shared_down);
        ne_compute<true>(a.dn, b, ne_table, lane, st);
        wait_stores();
        uint32_t finisher = 0;
        if (lane == 0) {
            finisher = grid_ticket(sync, moe_sync::kSharedDownGroup, moe_sync::kSharedDownTop, b, blocks) ? 1u : 0u;
        }
        if (__builtin_amdgcn_readfirstlane(finisher) != 0u) {
            const float g = __uint_as_float(~wait_nonzero(logit_words + a.experts, error, 1u));
            combine_row<VPL>(a.dn.ne[0].z, a.dn.ne[0].z_split_stride, a.shared_down_splits, nullptr,
                             a.shared_sv_down, 1.0f / (1.0f + expf(-g)), a.scale_hidden, lane, part(8));
            if (combine_ticket(sync, lane)) {
                finish_combine(a, sync, lane, 64u);
            }
        }
    } else {
        ExpertStage st;
        wait_flag(&flags[1], error);
        // x_hat = H(su[expert] * x) of the block's (entry, slot) by the eight
        // waves, su from the helper's LDS copy; the item's codes go out once
        // the wave's chunk is stored, so the transform does not queue behind
        // their issue
        const uint16_t *su = su_lds + 256u * wave;
        float sv4[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            sv4[i] = half_bits_to_float(su[64 * i + lane]);
        }
        hadamard_chunk(x_staged, sv4, wave, lane, x_routed);
        expert_prefetch(a.gu, slots, item_gu, half, lane, st, nullptr, false);
        arrive_and_wait(&flags[2], kGemvWaves, error);
        hadamard_cross(x_routed, a.scale_hidden, wave, lane);
        wait_plane();
        arrive_and_wait(&flags[8], kGemvWaves, error);
        expert_prefetch_x(a.gu, item_gu, half, lane, st, x_routed);
        // plain stores: only the slot's down blocks read these Z slices, on
        // this XCD, so they only have to reach its L2 (the block's count
        // goes out once they have)
        expert_compute<false>(a.gu, item_gu, half, plane, lane, st);
        count_block_quiet(&flags[3], kGemvWaves, sync_line(sync, moe_sync::kSlotCount + slot1));
    }

    // ---- P2 ----
    if (!helper) {
        ExpertStage st;
        expert_prefetch(a.dn, slots, item_dn, half, lane, st, nullptr, false);
        const uint4 info = slots[slot2];
        if (wave == 1) {  // off the helper's SIMD
            SwigluInputs in;
            swiglu_issue_scales(a.dn.swiglu, false, info.x, lane, in);
            wait_count(sync_line(sync, moe_sync::kSlotCount + slot2), a.expect_slot, error, 4u);
            float xd[VPLI];
            swiglu_issue_slices(a.dn.swiglu, false, info.y, lane, in);
            swiglu_finish(a.dn.swiglu, false, info.y, lane, in, xd);
            store_wave<VPLI>(x_down, lane, xd);
            set_flag(&flags[4]);
        } else {
            if (wave == 2) {
                // the slot's sv row (f16) for the combine row, should this
                // block complete the slot's down items
                const uint4 *src = reinterpret_cast<const uint4 *>(a.sv_down + static_cast<size_t>(info.x) * H);
                uint4 q[4];
#pragma unroll
                for (uint32_t u = 0; u < 4; ++u) {
                    q[u] = src[u * 64u + lane];
                }
#pragma unroll
                for (uint32_t u = 0; u < 4; ++u) {
                    reinterpret_cast<uint4 *>(sv_slot)[u * 64u + lane] = q[u];
                }
            }
            wait_flag(&flags[4], error);
        }
        expert_prefetch_x(a.dn, item_dn, half, lane, st, x_down);
        expert_compute<false>(a.dn, item_dn, half, plane, lane, st);  // read on this XCD only, as above
        // the block's count; flags[9]: 1 = another block completes the slot,
        // 2 = this block does, 3 = its row is in, 4 = and it was the last
        wait_stores();
        if (lane == 0 && atomicAdd(&flags[6], 1u) + 1u == kGemvWaves) {
            const bool completes =
                coherent_add(sync_line(sync, moe_sync::kDownCount + slot2), kGemvWaves) + kGemvWaves ==
                a.expect_down;
            __hip_atomic_store(&flags[9], completes ? 2u : 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
        }
        if (wait_lds_value(&flags[9], 1u, error) == 1u) {
            return;
        }
        // the slot's last down items are in: its route's combine row, by the
        // eight waves (chunks of 256, then the top three butterfly stages
        // across chunks, as for the routed x_hat)
        uint32_t r = 0;
#pragma unroll
        for (uint32_t q = 0; q < 8; ++q) {
            r = record_lds[moe_sync::kToGrouped + q] == slot2 ? q : r;
        }
        const float weight = __uint_as_float(record_lds[moe_sync::kRouteWeight + r]);
        const float *z = a.dn.expert[0].z + static_cast<size_t>(slot2) * H + 256u * wave;
        const size_t zs = a.dn.expert[0].z_split_stride;
        float v[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            v[i] = 0.0f;
        }
        for (uint32_t sl = 0; sl < a.down_splits; ++sl) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                v[i] = v[i] + z[sl * zs + 64u * i + lane];
            }
        }
        wave_hadamard<4>(v, 1.0f, lane);
        float *row = x_routed;  // free in P2
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            row[256u * wave + 64u * i + lane] = v[i];
        }
        arrive_and_wait(&flags[2], 2u * kGemvWaves, error);
        float *out_row = part(r);
        if (lane < 32) {
            const uint32_t j = 32u * wave + lane;
            float u[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                u[k] = row[256u * k + j];
            }
#pragma unroll
            for (int stride = 1; stride < 8; stride <<= 1) {
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    if ((k & stride) == 0) {
                        const float p = u[k], q = u[k + stride];
                        u[k] = p + q;
                        u[k + stride] = p - q;
                    }
                }
            }
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const float h = u[k] * a.scale_hidden;
                coherent_store(out_row + 256u * k + j,
                               weight * (h * half_bits_to_float(sv_slot[256u * k + j])));
            }
        }
        // the row is complete once every wave's stores are: the last to
        // arrive takes the combine ticket
        wait_stores();
        if (lane == 0 && atomicAdd(&flags[10], 1u) + 1u == kGemvWaves) {
            uint32_t t = coherent_add(sync_line(sync, moe_sync::kCombineTicket), 1u);
            __hip_atomic_store(&flags[9], t == 8u ? 4u : 3u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
        }
        if (wait_lds_value(&flags[9], 3u, error) == 4u) {
            finish_combine(a, sync, threadIdx.x, kGemvThreads);
        }
    }
}



// ---- the MoE block of a few rows in one launch ---------------------------------
//
// B = 2 .. kFewMaxRows rows. Phases (items, slices and every sum as in the
// separate launches, so results are bit-identical to theirs):
//   P0  every block: codebook plane and NE table into LDS; router rows b and
//       2 blocks - 1 - b (row `experts` is the shared gate) for every row of
//       the batch, in the CPU's ISA order, counted in per XCD. Blocks
//       0 .. 2B - 1 build the shared expert's gate and up x_hat of one row.
//       The helper wave then runs two shared gate/up NE items (all B rows).
//   P1  the GEMV waves route every row (top_experts, then the stable
//       counting sort by expert: slot s is the s-th smallest chosen expert,
//       its positions in route order) once all logits are in, and build
//       their share of the gate and up x_hat rows of their XCD's slots (slot
//       s runs on XCD s % 8, whose 32 blocks take the rows in turn).
//   P2  each GEMV wave runs one gate/up item of every slot of its XCD, as
//       soon as that slot's x_hat rows are in (the codes are in flight
//       meanwhile); Z slices stay on the XCD.
//   P3  the helper builds the SwiGLU x_hat rows of its share of the XCD's
//       routes once their slot's gate/up items are in; the helpers of blocks
//       0 .. B - 1 build the shared expert's, and every helper then runs one
//       shared down NE item.
//   P4  each GEMV wave runs one down item of every slot of its XCD; the wave
//       that completes a slot's down items builds its combine rows (one wave
//       each, the combine launch's arithmetic). The helpers of blocks
//       0 .. B - 1 build the shared combine rows once every shared down item
//       is in. Whoever adds a row's ninth combine row adds the nine in route
//       order, then the shared expert's, into the output.
// The last block through clears the counters for the next call. Every block
// is resident (one per CU) and every wait is bounded: a wait that runs out
// sets a bit of the error word.
namespace few_sync {
constexpr uint32_t kStride = 32;  // words between counters: a 128-byte line each
constexpr uint32_t kLogits = 0,        // 8 group counters (block b adds to b % 8): blocks with their logits out
                   kSharedX = 8,       // 8: shared gate/up x_hat rows written
                   kSharedGu = 16,     // 8: shared gate/up NE items done
                   kSharedDownX = 24,  // 8: shared SwiGLU x_hat rows written
                   kSharedDown = 32,   // 8 and a top counter (40): shared down NE items done
                   kSharedDone = 41,   // 8 replicas: every shared down item is in
                   kExit = 49,         // 8 and a top counter (57): blocks that are through
                   kXReady = 64,       // per (slot, entry): x_hat row chunks written (8 per row)
                   kGuDone = kXReady + 2 * kFewMaxRoutes,  // per slot: gate/up wave items done
                   kDownX = kGuDone + kFewMaxRoutes,       // per slot: SwiGLU x_hat rows written
                   kDnDone = kDownX + kFewMaxRoutes,       // per slot: down wave items done
                   kPosition = kDnDone + kFewMaxRoutes,    // per row: combine rows in
                   kCounters = kPosition + kFewMaxRows;
}  // namespace few_sync
static_assert(kMoeSyncFew >= (moe_sync::kParts + 18u) * kMoeSyncLine &&
                  kMoeSyncFew + few_sync::kCounters * few_sync::kStride <= kMoeSyncLinear,
              "the few-row counters sit after the one-row block's lines, before the DeltaNet tickets");

__device__ __forceinline__ uint32_t *few_word(uint32_t *sync, uint32_t i) {
    return sync + static_cast<size_t>(i) * few_sync::kStride;
}

// Polls (the whole wave) until the eight group counters from `first` add up
// to at least `total`; bounded (a timeout sets `bit` of the error word).
__device__ __forceinline__ void few_wait_total(uint32_t *sync, uint32_t first, uint32_t total, uint32_t lane,
                                               uint32_t *error, uint32_t bit) {
    for (uint32_t spins = 0;; ++spins) {
        const uint32_t v = lane < 8u ? coherent_load(few_word(sync, first + lane)) : 0u;
        uint32_t sum = 0;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            sum += static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), j));
        }
        if (sum >= total) {
            return;
        }
        if (spins >= kSpinLimit) {
            if (lane == 0) {
                __hip_atomic_fetch_or(error, bit, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            return;
        }
        __builtin_amdgcn_s_sleep(1);
    }
}

// Waits until word(t) >= target(t) for every t < n (n <= 64): one lane a
// counter, all of them polled in one round of loads (bounded like
// wait_count, error bit `bit`). One wait before a run of prefetched items
// instead of one per item: a coherent poll issued behind an item's prefetch
// loads would wait for them too (vmcnt counts in order).
template <typename Word, typename Target>
__device__ __forceinline__ void few_wait_each(Word &&word, Target &&target, uint32_t n, uint32_t lane,
                                              uint32_t *error, uint32_t bit) {
    for (uint32_t spins = 0;; ++spins) {
        bool ready = true;
        if (lane < n) {
            ready = coherent_load(word(lane)) >= target(lane);
        }
        if (__builtin_amdgcn_ballot_w64(!ready) == 0u) {
            return;
        }
        if (spins >= kSpinLimit) {
            if (lane == 0) {
                __hip_atomic_fetch_or(error, bit, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            return;
        }
        __builtin_amdgcn_s_sleep(1);
    }
}

// Two-level ticket over the grid from group counters `first` and top counter
// `top`: true in the one caller that completes it.
__device__ __forceinline__ bool few_ticket(uint32_t *sync, uint32_t first, uint32_t top, uint32_t b,
                                           uint32_t blocks) {
    const uint32_t group = b & 7u;
    const uint32_t members = (blocks - group + 7u) >> 3;
    if (coherent_add(few_word(sync, first + group), 1u) + 1u != members) {
        return false;
    }
    const uint32_t groups = blocks < 8u ? blocks : 8u;
    return coherent_add(few_word(sync, top), 1u) + 1u == groups;
}

// The x_hat loads of expert_prefetch for a stage whose words were loaded
// without them: the item's first position, from the entry's x_hat rows.
__device__ __forceinline__ void expert_load_x(const MoeGemv &m, uint32_t i, uint32_t half, uint32_t lane,
                                              ExpertStage &st) {
    const ExpertItem it = expert_item_of(m, i);
    const ExpertGemv &a = m.expert[it.which];
    uint32_t column[4], tile[4];
    bool valid[4];
    expert_tiles(a, it.item, half, lane, column, valid, tile);
    const bool live = st.info.z > st.info.y;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        valid[g] = valid[g] && live;
    }
    load_x_pair(a.x_hat, a.columns, st.info.y, column, 1u << a.group_shift, valid, st.x);
}

// expert_prefetch (without x_hat) and expert_load_x for G tile groups (the
// matrix's), with every load issued: a slot past the active count reads
// expert 0's first tile and x_hat row 0 and is never computed, and the items
// of the one-launch geometry cover their matrices exactly (no tile past one).
// With no branch around a load the compiler counts them, so the waits of the
// item that runs meanwhile leave them in flight.
template <uint32_t G>
__device__ __forceinline__ void few_prefetch(const MoeGemv &m, const uint4 *slots, uint32_t i, uint32_t half,
                                             uint32_t lane, ExpertStage &st) {
    const ExpertItem it = expert_item_of(m, i);
    const ExpertGemv &a = m.expert[it.which];
    const uint4 info = slots[it.slot];
    st.info = make_uint4(__builtin_amdgcn_readfirstlane(info.x), __builtin_amdgcn_readfirstlane(info.y),
                         __builtin_amdgcn_readfirstlane(info.z), 0u);
    const uint32_t quad = lane & 3u;
    const uint32_t tile_columns = 1u << a.tc_shift;
    const bool live = st.info.z > st.info.y;
    uint32_t column[4], tile[4];
    bool valid[4];
    expert_tiles(a, it.item, half, lane, column, valid, tile);
    const uint32_t expert = live ? st.info.x : 0u;
    const uint32_t *words = reinterpret_cast<const uint32_t *>(a.trellis + expert * a.trellis_stride);
    const uint16_t *gamma_row = a.gamma + expert * a.gamma_stride;
#pragma unroll
    for (uint32_t g = 0; g < G; ++g) {
        const uint32_t t = valid[g] && live ? tile[g] : 0u;
        typedef uint32_t u32x3 __attribute__((ext_vector_type(3)));
        const u32x3 w = __builtin_nontemporal_load(reinterpret_cast<const u32x3 *>(words + static_cast<size_t>(t) * 12u + quad * 3u));
        st.d[g][0] = w.x;
        st.d[g][1] = w.y;
        st.d[g][2] = w.z;
        const uint32_t tr = t >> a.tc_shift, tc = t & (tile_columns - 1u);
        st.gamma[g] = gamma_row[wave_slot(tr, tc, a.tile_rows, tile_columns)];
    }
}
template <uint32_t G>
__device__ __forceinline__ void few_load_x(const MoeGemv &m, uint32_t i, uint32_t half, uint32_t lane,
                                           ExpertStage &st) {
    const ExpertItem it = expert_item_of(m, i);
    const ExpertGemv &a = m.expert[it.which];
    uint32_t column[4], tile[4];
    bool valid[4];
    expert_tiles(a, it.item, half, lane, column, valid, tile);
    const bool live = st.info.z > st.info.y;
    const float *row = a.x_hat + static_cast<size_t>(live ? st.info.y : 0u) * a.columns;
#pragma unroll
    for (uint32_t g = 0; g < G; ++g) {
        const float *src = row + (valid[g] && live ? column[g] : 0u);
        st.x[g][0] = *reinterpret_cast<const float4 *>(src);
        st.x[g][1] = *reinterpret_cast<const float4 *>(src + 8);
    }
}

// 256 consecutive floats (a wave's chunk, 4 a lane) written through to memory.
__device__ __forceinline__ void store_chunk_through(float *dst, uint32_t lane, float4 v) {
    typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(dst, 0, 1024, 0x00020000);
    const u32x4_t q = {__float_as_uint(v.x), __float_as_uint(v.y), __float_as_uint(v.z), __float_as_uint(v.w)};
    __builtin_amdgcn_raw_buffer_store_b128(q, rs, lane * 16u, 0, 16 /* sc1 */);
}

// Row p of the output: its eight routed combine rows in route order, then the
// shared expert's (the combine launch's sum), by one wave.
__device__ __forceinline__ void few_finish_row(const MoeDecodeFew &a, uint32_t p, uint32_t lane) {
#pragma clang fp contract(off)
    constexpr uint32_t n4 = kFusedHidden / 4u;
    const float4 *rows = reinterpret_cast<const float4 *>(a.parts + static_cast<size_t>(p) * 9u * kFusedHidden);
    float4 *row_out = reinterpret_cast<float4 *>(a.out + static_cast<size_t>(p) * kFusedHidden);
    for (uint32_t c = lane; c < n4; c += 64u) {
        float4 v[9];
#pragma unroll
        for (uint32_t r = 0; r < 9; ++r) {
            v[r] = rows[r * n4 + c];
        }
        float4 acc = v[0];
#pragma unroll
        for (uint32_t r = 1; r < 9; ++r) {
            acc.x = acc.x + v[r].x;
            acc.y = acc.y + v[r].y;
            acc.z = acc.z + v[r].z;
            acc.w = acc.w + v[r].w;
        }
        row_out[c] = acc;
    }
}

// Counts combine row (p, *) in (the wave's stores complete first); the wave
// that adds the ninth writes output row p.
__device__ __forceinline__ void few_row_in(const MoeDecodeFew &a, uint32_t p, uint32_t lane) {
    wait_stores();
    uint32_t old = 0;
    if (lane == 0) {
        old = coherent_add(few_word(a.sync, few_sync::kPosition + p), 1u);
    }
    if (__builtin_amdgcn_readfirstlane(old) == 8u) {
        few_finish_row(a, p, lane);
    }
}

template <int LANES>
__global__ __launch_bounds__(kGemvThreads) void k_moe_decode_few(MoeDecodeFew a) {
#pragma clang fp contract(off)
    extern __shared__ uint4 lds_dynamic[];  // the codebook plane (first the staged rows), then kFusedRegion bytes
    __shared__ uint32_t ne_table[1024];
    __shared__ uint4 slots[kFewMaxRoutes];          // {expert, first, end, 0} by slot
    __shared__ uint32_t route_e[kFewMaxRoutes];     // route r = 8 p + k: expert
    __shared__ float route_w[kFewMaxRoutes];        // and weight
    __shared__ uint32_t grouped_route[kFewMaxRoutes];  // the route at each grouped position
    __shared__ uint32_t hist[kFusedMaxExperts];     // routes per expert, then its first grouped position
    __shared__ uint32_t posmask[kFusedMaxExperts];  // rows choosing each expert (bit p)
    __shared__ uint32_t counts[40];                 // LDS arrival counters
    __shared__ uint8_t xcd_slot[8][kFewMaxRoutes / 8];  // the slots each XCD runs, in order
    __shared__ uint32_t slot_count, last;
    constexpr uint32_t H = kFusedHidden;
    constexpr int VPLI = kFusedSwigluWidth / 64;
    // counts: 0 routing done, 1 slot table, 2 wave barrier,
    // 3 .. 18 gate/up items per XCD slot, 19 .. 34 down items per XCD slot
    constexpr uint32_t kRouted = 0, kTable = 1, kBar = 2, kGuCount = 3, kDnCount = 19;
    uint4 *plane_lds = lds_dynamic;
    float *x_lds = reinterpret_cast<float *>(lds_dynamic);  // P0: the batch's rows, before the plane
    float *region = reinterpret_cast<float *>(lds_dynamic + kPlaneBytes / 16);
    const uint32_t b = blockIdx.x, blocks = gridDim.x;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t lane = threadIdx.x & 63u;
    // block b is the k-th of XCD b % 8 (blocks are dealt round robin);
    // plane half k % 2, and the m-th of its (XCD, half) pair
    const uint32_t xcd = b & 7u, k = b >> 3, half = k & 1u, m_block = k >> 1;
    const uint32_t xcd_blocks = blocks >> 3;
    const uint32_t B = a.batch, routes_total = 8u * B, E = a.experts, row_words = E + 1u;
    uint32_t *sync = a.sync;
    uint32_t *error = a.error;
    for (uint32_t i = threadIdx.x; i < kFusedMaxExperts; i += kGemvThreads) {
        hist[i] = 0u;
        posmask[i] = 0u;
    }
    if (threadIdx.x < 40) {
        counts[threadIdx.x] = 0u;
    }
    // The shared expert's NE items in units of (item, group of rows), at most
    // one a wave: unit u runs on wave u % 8 of block blocks - 1 - u / 8 (from
    // the last block down, away from the blocks that build the routed SwiGLU
    // and combine rows). The gate/up units take up to four groups of rows,
    // the down units up to eight; their codes are loaded at the start.
    const uint32_t from_top = (blocks - 1u - b) * kGemvWaves + wave;
    const uint32_t gu_groups = B < 4u ? B : 4u, gu_per = (B + gu_groups - 1u) / gu_groups;
    const uint32_t dn_groups = B < 8u ? (B < 4u ? B : 4u) : 8u, dn_per = (B + dn_groups - 1u) / dn_groups;
    const bool gu_unit = from_top < a.gu.ne_items * gu_groups;
    const bool dn_unit = from_top < a.dn.ne_items * dn_groups;
    const uint32_t gu_k = from_top % a.gu.ne_items, gu_first = (from_top / a.gu.ne_items) * gu_per;
    const uint32_t dn_k = from_top % a.dn.ne_items, dn_first = (from_top / a.dn.ne_items) * dn_per;
    NeStage gu_st;
    uint32_t barriers = 0;
    auto block_barrier = [&]() {
        __builtin_amdgcn_s_waitcnt(kWaitLds);
        if (lane == 0) {
            __hip_atomic_fetch_add(&counts[kBar], 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
        }
        wait_lds_value(&counts[kBar], kGemvWaves * ++barriers, error);
    };

    // ---- P0: router rows b and 2 blocks - 1 - b (row `experts` is the
    // shared gate) of every row of the batch, x staged in LDS ----
    const uint32_t r0 = b, r1 = 2u * blocks - 1u - b;
    const uint32_t nrows = (r0 < row_words ? 1u : 0u) + (r1 < row_words ? 1u : 0u);
    uint16_t *wl = reinterpret_cast<uint16_t *>(region);  // the block's router rows
    {
        auto row = [&](uint32_t r) {
            return reinterpret_cast<const uint4 *>(r < E ? a.router + static_cast<size_t>(r) * H : a.shared_gate_row);
        };
        // row 0 of the LDS copy is the block's first valid row, row 1 its second
        const uint32_t first = r0 < row_words ? r0 : r1;
        const uint32_t u = threadIdx.x;  // 512 uint4 = the two rows
        uint4 w = make_uint4(0u, 0u, 0u, 0u);
        if (u < 256u && nrows > 0) {
            w = row(first)[u];
        } else if (u >= 256u && nrows > 1) {
            w = row(r1)[u - 256u];
        }
        reinterpret_cast<uint4 *>(wl)[u] = w;
        // the rows in rounds of eight loads (a row past the batch reloads the last)
#pragma unroll
        for (uint32_t p0 = 0; p0 < kFewMaxRows; p0 += 8u) {
            if (p0 < B) {
                float4 xv[8];
#pragma unroll
                for (uint32_t j = 0; j < 8u; ++j) {
                    const uint32_t p = p0 + j < B ? p0 + j : B - 1u;
                    xv[j] = reinterpret_cast<const float4 *>(a.x + static_cast<size_t>(p) * H)[u];
                }
#pragma unroll
                for (uint32_t j = 0; j < 8u; ++j) {
                    if (p0 + j < B) {
                        reinterpret_cast<float4 *>(x_lds + static_cast<size_t>(p0 + j) * H)[u] = xv[j];
                    }
                }
            }
        }
    }
    __syncthreads();
    {
        // chain c = (row sel, input row p) = (c / B, c % B), 64 / LANES chains a wave
        constexpr uint32_t kChains = 64u / LANES;
        const uint32_t chains = nrows * B;
        if (wave * kChains < chains) {
            const uint32_t c = wave * kChains + lane / LANES;
            const uint32_t cc = c < chains ? c : chains - 1u;
            const float acc = router_chain<LANES>(wl + (cc / B) * H, x_lds + static_cast<size_t>(cc % B) * H, H,
                                                  lane % LANES);
#pragma unroll
            for (uint32_t g = 0; g < kChains; ++g) {
                const float s = router_lane_sum<LANES>(acc, g);
                const uint32_t cg = wave * kChains + g;
                if (lane == 0 && cg < chains) {
                    const uint32_t sel = cg / B, p = cg % B;
                    const uint32_t r = sel == 0 && r0 < row_words ? r0 : r1;
                    coherent_store(a.logits + static_cast<size_t>(p) * row_words + r, s);
                }
            }
        }
    }
    wait_stores();
    __syncthreads();  // every chain's logits out; the staged rows are free
    if (threadIdx.x == 0) {
        coherent_add(few_word(sync, few_sync::kLogits + xcd), 1u);
    }
    // the shared gate/up unit's codes, needed after the routing (issued
    // before the router chains, their wait held the chains back)
    if (gu_unit) {
        ne_prefetch_codes(a.gu, gu_k, lane, gu_st);
    }
    // the codebook plane and the NE table (its words first; the plane's wait
    // covers them)
    {
        uint32_t tab[kTableWords];
        load_table_share(static_cast<const uint32_t *>(a.gu.ne_book), tab);
        fill_plane_share(static_cast<const uint4 *>(a.gu.expert_book) + half * (kPlaneBytes / 16), plane_lds);
        store_table_share(tab, ne_table);
    }
    // the shared expert's gate (blocks 0 .. B - 1) and up (B .. 2B - 1) x_hat of one row
    if (b < 2u * B) {
        const uint32_t which = b / B, p = b % B;
        float *xs = region;
        const int8_t *su = which == 0 ? a.shared_su_gate : a.shared_su_up;
        float sign[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            sign[i] = static_cast<float>(su[256u * wave + 64u * i + lane]);
        }
        hadamard_chunk(a.x + static_cast<size_t>(p) * H, sign, wave, lane, xs);
        block_barrier();
        hadamard_cross(xs, a.scale_hidden, wave, lane);
        block_barrier();
        float *dst = const_cast<float *>(a.gu.ne[which].x_hat) + static_cast<size_t>(p) * H + 256u * wave;
        store_chunk_through(dst, lane, reinterpret_cast<const float4 *>(xs + 256u * wave)[lane]);
        wait_stores();
        block_barrier();
        if (threadIdx.x == 0) {
            coherent_add(few_word(sync, few_sync::kSharedX + xcd), 1u);
        }
    }
    __syncthreads();  // the plane and the table are complete
    const uint2 *plane = reinterpret_cast<const uint2 *>(plane_lds);

    // ---- P1: routing (top_experts of row p on wave p % 8, then the stable
    // counting sort by expert: slot s is the s-th smallest chosen expert, its
    // positions in route order) ----
    if (wave < B) {
        few_wait_total(sync, few_sync::kLogits, blocks, lane, error, 1u);
        for (uint32_t p = wave; p < B; p += kGemvWaves) {
            top8_wave<4>(a.logits + static_cast<size_t>(p) * row_words, a.logit_bias, E, lane, route_e + 8u * p,
                         route_w + 8u * p);
        }
    }
    arrive_and_wait(&counts[kRouted], kGemvWaves, error);
    if (wave == 0) {
        // the counting sort: routes per expert and the rows choosing it,
        // then each expert's first grouped position and slot
        for (uint32_t r = lane; r < routes_total; r += 64u) {
            const uint32_t e = route_e[r];
            atomicAdd(&hist[e], 1u);
            atomicOr(&posmask[e], 1u << (r >> 3));
        }
        __builtin_amdgcn_s_waitcnt(kWaitLds);
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        uint32_t cnt[4], run = 0, nz = 0;
#pragma unroll
        for (uint32_t j = 0; j < 4; ++j) {
            const uint32_t e = 4u * lane + j;
            cnt[j] = e < E ? hist[e] : 0u;
            run += cnt[j];
            nz += cnt[j] != 0u ? 1u : 0u;
        }
        // exclusive prefix sums over the lanes (lane order = expert order)
        uint32_t run_ex = run, nz_ex = nz;
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
            const uint32_t a1 = static_cast<uint32_t>(__shfl_up(static_cast<int>(run_ex), d, 64));
            const uint32_t a2 = static_cast<uint32_t>(__shfl_up(static_cast<int>(nz_ex), d, 64));
            if (lane >= static_cast<uint32_t>(d)) {
                run_ex += a1;
                nz_ex += a2;
            }
        }
        run_ex -= run;
        nz_ex -= nz;
        if (lane == 63u) {
            slot_count = nz_ex + nz;
        }
#pragma unroll
        for (uint32_t j = 0; j < 4; ++j) {
            const uint32_t e = 4u * lane + j;
            if (e < E) {
                hist[e] = run_ex;
                if (cnt[j] != 0u) {
                    slots[nz_ex] = make_uint4(e, run_ex, run_ex + cnt[j], 0u);
                    ++nz_ex;
                }
                run_ex += cnt[j];
            }
        }
        __builtin_amdgcn_s_waitcnt(kWaitLds);
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        {
            // slots to XCDs: by rows held, most first (ties by slot), dealt in
            // snake order 0..7, 7..0, ... so the XCDs' rows stay even
            const uint32_t total = __builtin_amdgcn_readfirstlane(slot_count);
            uint32_t size[2], rank[2] = {0u, 0u};
#pragma unroll
            for (uint32_t h = 0; h < 2u; ++h) {
                const uint32_t sl = 64u * h + lane;
                size[h] = sl < total ? slots[sl].z - slots[sl].y : 0u;
            }
            const uint64_t below = (uint64_t(1) << lane) - 1u;
            uint32_t base = 0;
            for (uint32_t c = kFewMaxRows; c >= 1u; --c) {
                const uint64_t m0 = __ballot(size[0] == c), m1 = __ballot(size[1] == c);
                const uint32_t n0 = static_cast<uint32_t>(__builtin_popcountll(m0));
                if (size[0] == c) {
                    rank[0] = base + static_cast<uint32_t>(__builtin_popcountll(m0 & below));
                }
                if (size[1] == c) {
                    rank[1] = base + n0 + static_cast<uint32_t>(__builtin_popcountll(m1 & below));
                }
                base += n0 + static_cast<uint32_t>(__builtin_popcountll(m1));
            }
#pragma unroll
            for (uint32_t h = 0; h < 2u; ++h) {
                const uint32_t sl = 64u * h + lane;
                if (sl < total) {
                    const uint32_t round = rank[h] >> 3, at = rank[h] & 7u;
                    xcd_slot[(round & 1u) != 0u ? 7u - at : at][round] = static_cast<uint8_t>(sl);
                }
            }
        }
        __builtin_amdgcn_s_waitcnt(kWaitLds);
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        for (uint32_t r = lane; r < routes_total; r += 64u) {
            const uint32_t e = route_e[r], p = r >> 3;
            const uint32_t g = hist[e] + __builtin_popcount(posmask[e] & ((1u << p) - 1u));
            grouped_route[g] = r;
            if (b == 0 && a.route_expert_out != nullptr) {
                a.route_expert_out[r] = e;
            }
            if (b == 0 && a.route_weight_out != nullptr) {
                a.route_weight_out[r] = route_w[r];
            }
        }
        set_flag(&counts[kTable]);
    }
    wait_flag(&counts[kTable], error);
    const uint32_t slot_total = slot_count;
    // the XCD's slots: one per full round of the deal, and one in the last
    // round when the snake reaches it
    const uint32_t rounds = slot_total >> 3, rest = slot_total & 7u;
    const uint32_t at_last = (rounds & 1u) != 0u ? 7u - xcd : xcd;
    const uint32_t n_slots = rounds + (at_last < rest ? 1u : 0u);
    auto slot_of = [&](uint32_t t) { return static_cast<uint32_t>(xcd_slot[xcd][t]); };
    // the XCD's routes (grouped positions of its slots, slot by slot) are
    // shared out: route q to block q % 32 of the XCD, wave (q / 32) % 8
    // (SwiGLU rows), and block q % 32 (combine rows)

    if (gu_unit) {
        few_wait_total(sync, few_sync::kSharedX, 2u * B, lane, error, 2u);
        ne_prefetch_x(a.gu, gu_k, lane, gu_st, gu_first);
    }
    // ---- P1: the block's share of its XCD's gate and up x_hat rows ----
    {
        float *xs = region;
        uint32_t j = 0;
        for (uint32_t t = 0; t < n_slots; ++t) {
            const uint32_t s = slot_of(t);
            const uint4 info = slots[s];
            for (uint32_t g = info.y; g < info.z; ++g) {
                for (uint32_t which = 0; which < 2u; ++which, ++j) {
                    if (j % xcd_blocks != k) {
                        continue;
                    }
                    const uint32_t p = grouped_route[g] >> 3;
                    const uint16_t *su = (which == 0 ? a.su_gate : a.su_up) + static_cast<size_t>(info.x) * H +
                                         256u * wave;
                    float m4[4];
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        m4[i] = half_bits_to_float(su[64 * i + lane]);
                    }
                    hadamard_chunk(a.x + static_cast<size_t>(p) * H, m4, wave, lane, xs);
                    block_barrier();
                    hadamard_cross(xs, a.scale_hidden, wave, lane);
                    block_barrier();
                    float *dst = const_cast<float *>(a.gu.expert[which].x_hat) + static_cast<size_t>(g) * H;
                    reinterpret_cast<float4 *>(dst)[64u * wave + lane] =
                        reinterpret_cast<const float4 *>(xs)[64u * wave + lane];
                    block_barrier();  // xs is free again
                    wait_stores();
                    if (lane == 0) {
                        coherent_add(few_word(sync, few_sync::kXReady + 2u * s + which), 1u);
                    }
                }
            }
        }
    }
    // the shared gate/up unit, while the first slot's x_hat rows come in
    if (gu_unit) {
        ne_compute<true>(a.gu, gu_k, ne_table, lane, gu_st, gu_first, gu_first + gu_per);
        wait_stores();
        if (lane == 0) {
            coherent_add(few_word(sync, few_sync::kSharedGu + xcd), 1u);
        }
    }
    // ---- P2: item m_block * 8 + wave of every slot of the XCD, the next
    // slot's codes and x_hat in flight during the arithmetic ----
    const uint32_t il = m_block * kGemvWaves + wave;
    {
        const uint32_t which = il / a.gu.expert_items_per_slot;
        const uint32_t item = il % a.gu.expert_items_per_slot;
        auto index = [&](uint32_t t) { return ((which * a.gu.max_active + slot_of(t)) << a.gu.item_shift) + item; };
        // every slot's x_hat rows of this entry (built in P1) before the
        // first item, so no poll waits behind a prefetch
        few_wait_each([&](uint32_t t) { return few_word(sync, few_sync::kXReady + 2u * slot_of(t) + which); },
                      [&](uint32_t t) {
                          const uint4 info = slots[slot_of(t)];
                          return kGemvWaves * (info.z - info.y);
                      },
                      n_slots, lane, error, 4u);
        // every slot's stage is issued, the one past the last staging the last
        // again (unused): see few_prefetch
        auto stage = [&](uint32_t t, ExpertStage &st) {
            t = t < n_slots ? t : n_slots - 1u;
            few_prefetch<kFewGuGroups>(a.gu, slots, index(t), half, lane, st);
            few_load_x<kFewGuGroups>(a.gu, index(t), half, lane, st);
        };
        // plain stores: only this XCD's SwiGLU rows read these Z slices
        auto run = [&](uint32_t t, ExpertStage &st) {
            expert_compute<false>(a.gu, index(t), half, plane, lane, st);
            count_block_quiet(&counts[kGuCount + t], kGemvWaves, few_word(sync, few_sync::kGuDone + slot_of(t)));
        };
        ExpertStage s0, s1;
        if (n_slots > 0) {
            stage(0, s0);
        }
        for (uint32_t t = 0; t < n_slots; t += 2u) {
            stage(t + 1u, s1);
            run(t, s0);
            if (t + 1u >= n_slots) {
                break;
            }
            stage(t + 2u, s0);
            run(t + 1u, s1);
        }
    }
    NeStage dn_st;
    if (dn_unit) {
        ne_prefetch_codes(a.dn, dn_k, lane, dn_st);
    }
    // ---- P3: the wave's SwiGLU rows of its XCD's routes (waves 0 .. 6 below
    // 224 routes per XCD), and the shared expert's SwiGLU row p on wave 7 of
    // block p ----
    {
        uint32_t q = 0;
        for (uint32_t t = 0; t < n_slots; ++t) {
            const uint32_t s = slot_of(t);
            const uint4 info = slots[s];
            for (uint32_t g = info.y; g < info.z; ++g, ++q) {
                if (q % xcd_blocks != k || (q / xcd_blocks) % kGemvWaves != wave) {
                    continue;
                }
                SwigluInputs in;
                swiglu_issue_scales(a.dn.swiglu, false, info.x, lane, in);
                wait_count(few_word(sync, few_sync::kGuDone + s), a.expect_gu, error, 4u);
                float xd[VPLI];
                swiglu_issue_slices(a.dn.swiglu, false, g, lane, in);
                swiglu_finish(a.dn.swiglu, false, g, lane, in, xd);
                store_wave<VPLI>(const_cast<float *>(a.dn.expert[0].x_hat) + static_cast<size_t>(g) * kFusedSwigluWidth,
                                 lane, xd);
                wait_stores();
                if (lane == 0) {
                    coherent_add(few_word(sync, few_sync::kDownX + s), 1u);
                }
            }
        }
    }
    if (wave == kGemvWaves - 1u && b < B) {
        const uint32_t p = b;
        few_wait_total(sync, few_sync::kSharedGu, a.gu.ne_items * gu_groups, lane, error, 8u);
        SwigluInputs in;
        float xd[VPLI];
        swiglu_issue(a.dn.swiglu, true, p, 0u, lane, in);
        swiglu_finish(a.dn.swiglu, true, p, lane, in, xd);
        store_wave_through<VPLI>(const_cast<float *>(a.dn.ne[0].x_hat) + static_cast<size_t>(p) * kFusedSwigluWidth,
                                 lane, xd);
        wait_stores();
        if (lane == 0) {
            coherent_add(few_word(sync, few_sync::kSharedDownX + xcd), 1u);
        }
    }
    // ---- P4: down item m_block * 8 + wave of every slot of the XCD, the
    // next slot's codes and x_hat in flight during the arithmetic ----
    {
        auto index = [&](uint32_t t) { return (slot_of(t) << a.dn.item_shift) + il; };
        // the slot's x_hat count is read before its codes go out: when it is
        // already complete (the usual case), that read's wait leaves the codes
        // in flight; otherwise the poll waits for everything
        auto stage = [&](uint32_t t, ExpertStage &st) {
            t = t < n_slots ? t : n_slots - 1u;
            const uint4 info = slots[slot_of(t)];
            uint32_t *word = few_word(sync, few_sync::kDownX + slot_of(t));
            const uint32_t seen = coherent_load(word);
            __builtin_amdgcn_sched_barrier(0);
            few_prefetch<kFewDnGroups>(a.dn, slots, index(t), half, lane, st);
            __builtin_amdgcn_sched_barrier(0);
            if (__builtin_amdgcn_readfirstlane(seen) < info.z - info.y) {
                wait_count(word, info.z - info.y, error, 4u);
            }
            few_load_x<kFewDnGroups>(a.dn, index(t), half, lane, st);
        };
        auto run = [&](uint32_t t, ExpertStage &st) {
            expert_compute<false>(a.dn, index(t), half, plane, lane, st);  // read on this XCD only
            count_block_quiet(&counts[kDnCount + t], kGemvWaves, few_word(sync, few_sync::kDnDone + slot_of(t)));
        };
        ExpertStage s0, s1;
        if (n_slots > 0) {
            stage(0, s0);
        }
        for (uint32_t t = 0; t < n_slots; t += 2u) {
            stage(t + 1u, s1);
            run(t, s0);
            if (t + 1u >= n_slots) {
                break;
            }
            stage(t + 2u, s0);
            run(t + 1u, s1);
        }
    }
    // the shared down unit; the last one in (two-level count: each group
    // line b % 8 takes an eighth of them) sets the shared flag
    if (dn_unit) {
        const uint32_t per_line = a.dn.ne_items * dn_groups / 8u;
        few_wait_total(sync, few_sync::kSharedDownX, B, lane, error, 8u);
        ne_prefetch_x(a.dn, dn_k, lane, dn_st, dn_first);
        ne_compute<true>(a.dn, dn_k, ne_table, lane, dn_st, dn_first, dn_first + dn_per);
        wait_stores();
        uint32_t finisher = 0;
        if (lane == 0 && coherent_add(few_word(sync, few_sync::kSharedDown + xcd), 1u) + 1u == per_line &&
            coherent_add(few_word(sync, few_sync::kSharedDown + 8u), 1u) + 1u == 8u) {
            finisher = 1u;
        }
        if (__builtin_amdgcn_readfirstlane(finisher) != 0u && lane < 8u) {
            coherent_store(few_word(sync, few_sync::kSharedDone + lane), 1u);
        }
    }
    // ---- P5: combine rows by the eight waves (chunks of 256, then the top
    // three butterfly stages across chunks: combine_row's values); route q
    // of the XCD on block q % 32, once its slot's down items are in ----
    float *row = region;
    auto block_combine_row = [&](const float *z, size_t zs, uint32_t splits, const uint16_t *sv_f16,
                                 const int8_t *sv_sign, float weight, float *dst) {
        float v[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            v[i] = 0.0f;
        }
        for (uint32_t sl = 0; sl < splits; ++sl) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                v[i] = v[i] + z[sl * zs + 256u * wave + 64u * i + lane];
            }
        }
        wave_hadamard<4>(v, 1.0f, lane);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            row[256u * wave + 64u * i + lane] = v[i];
        }
        block_barrier();
        if (lane < 32) {
            const uint32_t j = 32u * wave + lane;
            float u[8];
#pragma unroll
            for (int qq = 0; qq < 8; ++qq) {
                u[qq] = row[256u * qq + j];
            }
#pragma unroll
            for (int stride = 1; stride < 8; stride <<= 1) {
#pragma unroll
                for (int qq = 0; qq < 8; ++qq) {
                    if ((qq & stride) == 0) {
                        const float x0 = u[qq], x1 = u[qq + stride];
                        u[qq] = x0 + x1;
                        u[qq + stride] = x0 - x1;
                    }
                }
            }
#pragma unroll
            for (int qq = 0; qq < 8; ++qq) {
                const float h = u[qq] * a.scale_hidden;
                const float sv = sv_f16 != nullptr ? half_bits_to_float(sv_f16[256u * qq + j])
                                                   : static_cast<float>(sv_sign[256u * qq + j]);
                coherent_store(dst + 256u * qq + j, weight * (h * sv));
            }
        }
        wait_stores();
        block_barrier();  // every wave's stores are complete, the LDS row is free
    };
    {
        uint32_t q = 0;
        for (uint32_t t = 0; t < n_slots; ++t) {
            const uint32_t s = slot_of(t);
            const uint4 info = slots[s];
            for (uint32_t g = info.y; g < info.z; ++g, ++q) {
                if (q % xcd_blocks != k) {
                    continue;
                }
                wait_count(few_word(sync, few_sync::kDnDone + s), a.expect_dn, error, 4u);
                const uint32_t r = grouped_route[g];
                const uint32_t p = r >> 3;
                block_combine_row(a.dn.expert[0].z + static_cast<size_t>(g) * H, a.dn.expert[0].z_split_stride,
                                  a.down_splits, a.sv_down + static_cast<size_t>(info.x) * H, nullptr, route_w[r],
                                  a.parts + (static_cast<size_t>(p) * 9u + (r & 7u)) * H);
                if (wave == 0) {
                    few_row_in(a, p, lane);
                }
            }
        }
    }
    // the shared expert's combine row p on block blocks / 2 + p
    if (b >= blocks / 2u && b - blocks / 2u < B) {
        const uint32_t p = b - blocks / 2u;
        wait_count(few_word(sync, few_sync::kSharedDone + xcd), 1u, error, 8u);
        const float gate = a.logits[static_cast<size_t>(p) * row_words + E];
        block_combine_row(a.dn.ne[0].z + static_cast<size_t>(p) * H, a.dn.ne[0].z_split_stride, a.shared_down_splits,
                          nullptr, a.shared_sv_down, 1.0f / (1.0f + expf(-gate)),
                          a.parts + (static_cast<size_t>(p) * 9u + 8u) * H);
        if (wave == 0) {
            few_row_in(a, p, lane);
        }
    }
    // ---- the last block through clears the counters ----
    wait_stores();
    __syncthreads();
    if (threadIdx.x == 0) {
        last = few_ticket(sync, few_sync::kExit, few_sync::kExit + 8u, b, blocks) ? 1u : 0u;
    }
    __syncthreads();
    if (last != 0u) {
        for (uint32_t i = threadIdx.x; i < few_sync::kCounters; i += kGemvThreads) {
            coherent_store(few_word(sync, i), 0u);
        }
    }
}

// ---- one-launch NE projection of a few rows -------------------------------
//
// y = sv * H_rows(W x_hat) * scale_rows with x_hat = H_columns(su * x) *
// scale_columns (src/kernels.cpp:899-979), for up to kNeFusedRows input rows,
// in one launch instead of prologue, GEMV and epilogue. A launch carries up to
// kNeFusedJobs matrices of one column count over the same input rows, each on
// a range of blocks of its own; block b of a matrix takes its tile rows b,
// b + blocks, ... whole: it builds every input row's x_hat itself (eight
// waves' cooperative transform, bit-identical to the one-wave one), runs the
// tile row's NE items (16 tiles each, the GEMV's arithmetic, the table values
// gathered once per item), and adds the items' partial sums in item (slice)
// order in LDS, so the sum is the one the separate epilogue forms. With two or
// more input rows the grid is two halves: half g takes input rows g, g + 2,
// ... of every tile row (each half decodes the codes itself), so the VALU work
// of the input rows spreads over all CUs. The block of a matrix and half that
// completes its last tile row (a ticket each; nobody waits) runs the row
// transform over that half's sums.
template <int VR>
__device__ void ne_fused_rows(const NeFusedJob &job, float *ne_lds, const int8_t *sv_lds, uint32_t group,
                              uint32_t halves, uint32_t batch, uint32_t w8, uint32_t lane, float (*norm_sums)[4],
                              float *norm_scale) {
    constexpr uint32_t R = 512u * VR, RH = R / 8u;
    // with the next norm (2048 rows): its residual rows and weights load
    // after the sums, so that their latency runs under the transform; a
    // half holds at most two rows, one on each 256-thread half of the block
    const bool tail = R <= 2048u && job.tail_row != nullptr;
    const uint32_t pair = threadIdx.x >> 8, t256 = threadIdx.x & 255u;
    const uint32_t tail_p = group + halves * pair;
    const uint32_t tail_q = tail_p < batch ? tail_p : group;
    float tail_r[8];
    uint16_t tail_w[8];
    // every sum of the half's input rows is in (first touch here, ordinary
    // loads; all the loads first)
    {
        float v[kNeFusedRows][VR];
#pragma unroll
        for (uint32_t i = 0; i < kNeFusedRows; ++i) {
            const uint32_t p = group + halves * i;
            if (p < batch) {
                load_wave<VR>(job.zsum + static_cast<size_t>(p) * R + w8 * RH, lane, v[i]);
            }
        }
        if (tail) {
            const float *row = job.tail_row + static_cast<size_t>(tail_q) * R;
#pragma unroll
            for (uint32_t k = 0; k < 8u; ++k) {
                tail_r[k] = row[t256 + 256u * k];
                tail_w[k] = job.tail_weight[t256 + 256u * k];
            }
        }
#pragma unroll
        for (uint32_t i = 0; i < kNeFusedRows; ++i) {
            const uint32_t p = group + halves * i;
            if (p < batch) {
                wave_hadamard<VR>(v[i], 1.0f, lane);
                store_wave<VR>(ne_lds + p * R + w8 * RH, lane, v[i]);
            }
        }
    }
    __syncthreads();
    if (!tail) {
        // the last butterflies write the outputs
        for (uint32_t p = group; p < batch; p += halves) {
            hadamard_cross_span_out<RH>(ne_lds + p * R, job.scale_rows, w8, lane, sv_lds, job.out + p * R);
        }
        return;
    }
    for (uint32_t p = group; p < batch; p += halves) {
        hadamard_cross_span<RH>(ne_lds + p * R, job.scale_rows, w8, lane);
    }
    __syncthreads();
    for (uint32_t e = threadIdx.x; e < R; e += kNeFusedThreads) {
        const float sign = static_cast<float>(sv_lds[e]);
#pragma unroll
        for (uint32_t i = 0; i < kNeFusedRows; ++i) {
            const uint32_t p = group + halves * i;
            if (p < batch) {
                job.out[p * R + e] = ne_lds[p * R + e] * sign;
            }
        }
    }
    // the residual add and the next RMS norm of the half's rows
    float *row = job.tail_row + static_cast<size_t>(tail_q) * R;
    const float *y = ne_lds + tail_q * R;
    float v[8], w[8];
#pragma unroll
    for (uint32_t k = 0; k < 8u; ++k) {
        const uint32_t e = t256 + 256u * k;
        v[k] = tail_r[k] + y[e] * static_cast<float>(sv_lds[e]);
        w[k] = bf16_bits_to_float(tail_w[k]);
    }
    block_rms_norm_held(v, w, [&](uint32_t e, float x) { row[e] = x; }, R, 1.0f, 1.0e-6f,
                        job.tail_out + static_cast<size_t>(tail_q) * R, norm_sums[pair], &norm_scale[pair],
                        tail_p < batch ? t256 : 256u);
}

template <int VC, int ROWS, bool NORM>
__global__ __launch_bounds__(kNeFusedThreads) void k_ne_fused(NeFused a) {
#pragma clang fp contract(off)
    extern __shared__ float ne_lds[];  // x_hat [batch][C], then the outputs [batch][rows]
    __shared__ uint32_t table[1024];
    __shared__ float part[kNeFusedMaxItems][16][kNeFusedRows];  // [item in tile row][row][input row]
    __shared__ uint32_t last;
    __shared__ float norm_sums[2][4], norm_scale[2];  // block_rms_norm's block sums, two rows at a time
    __shared__ int8_t sv_lds[kNeFusedMaxRows];  // the output signs, staged by every block for whichever ends last
    constexpr uint32_t C = 512u * VC, CH = C / 8u;
    constexpr uint32_t tile_columns = C / kTile, per_row = tile_columns / 16u;
    constexpr uint32_t kMine = kNeFusedRows;  // input rows of a half, at most
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t w8 = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t quad = lane & 3u, tslot = lane >> 2;
    const uint32_t halves = a.halves;
    const uint32_t group = blockIdx.x % halves;  // the half: input rows group, group + halves, ...
    const uint32_t g = blockIdx.x / halves;      // block within the half
    // the block's matrix (constant indexes only, so the arguments stay in
    // the kernel argument segment)
    uint32_t j = 0;
    if (a.jobs > 1u && g >= a.job[1].first_block) {
        j = 1;
    }
    if (a.jobs > 2u && g >= a.job[2].first_block) {
        j = 2;
    }
    const NeFusedJob job = j == 0 ? a.job[0] : (j == 1 ? a.job[1] : a.job[2]);
    const uint32_t R = job.rows, tile_rows = R / kTile;
    const uint32_t b = g - job.first_block, blocks = job.blocks;  // within the matrix and half
    uint32_t *ticket = a.ticket + 32u * (2u * j + group);
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    // A round takes ROWS of the block's tile rows (tr, tr + blocks, ...), so
    // that a wave runs ROWS items between the round's barriers (their x_hat
    // reads shared).
    constexpr uint32_t kWaveItems = per_row > 8u ? per_row / 8u : 1u;
    constexpr uint32_t kRoundRows = ROWS;
    static_assert(kRoundRows * per_row <= kNeFusedMaxItems, "a round's items fit the partial sums");
    u32x4 code[kRoundRows][kWaveItems][2];
    // the codes of the round from tile row tr; a tile row past the matrix
    // loads the block's first one again, unused (the loads stay unconditional
    // so that the waits before the first round count them)
    auto load_codes = [&](uint32_t tr) {
#pragma unroll
        for (uint32_t u = 0; u < kRoundRows; ++u) {
            const uint32_t t = tr + u * blocks < tile_rows ? tr + u * blocks : b;
#pragma unroll
            for (uint32_t q = 0; q < kWaveItems; ++q) {
                const uint32_t i = w8 + 8u * q;
                const uint32_t tile = (t * per_row + (i < per_row ? i : 0u)) * 16u + tslot;
                const u32x4 *src =
                    reinterpret_cast<const u32x4 *>(job.trellis) + static_cast<size_t>(tile) * 8u + quad * 2u;
                code[u][q][0] = __builtin_nontemporal_load(src);
                code[u][q][1] = __builtin_nontemporal_load(src + 1);
            }
        }
    };
    // The block's shares of the NE table and the output signs, and the x_hat
    // inputs, load before the codes: the load counter completes in order, so
    // the waits for them leave the codes in flight.
    constexpr uint32_t kTablePer = 1024u / kNeFusedThreads;
    constexpr uint32_t kSignPer = kNeFusedMaxRows / 4u / kNeFusedThreads;
    const uint32_t sign_words = R / 4u;
    const uint32_t *sv_words = reinterpret_cast<const uint32_t *>(job.sv);
    uint32_t tab[kTablePer], signs[kSignPer];
#pragma unroll
    for (uint32_t k = 0; k < kTablePer; ++k) {
        tab[k] = job.table[threadIdx.x + k * kNeFusedThreads];
    }
#pragma unroll
    for (uint32_t k = 0; k < kSignPer; ++k) {
        signs[k] = sv_words[min(threadIdx.x + k * kNeFusedThreads, sign_words - 1u)];
    }
    float xs[VC], xv[kMine][VC];
    load_wave_sign<VC>(job.su + w8 * CH, lane, xs);
    // the input norm (a.norm_row set; 2048 columns only), known at compile
    // time so that its loads go out with the others without a branch
    constexpr bool normed = NORM;
    static_assert(!NORM || C == 2048u, "the input norm runs at 2048 columns");
    // With a norm: the half's input rows two at a time, one on each 256-thread
    // half of the block (a half holds at most two rows: two halves from two
    // rows on), thread t of a half holding columns t + 256 k of its row, the
    // residual and the weights.
    static_assert(kNeFusedRows <= 4u, "a half holds at most two input rows");
    const uint32_t pair = threadIdx.x >> 8, t256 = threadIdx.x & 255u;
    const uint32_t norm_p = group + halves * pair;
    const uint32_t norm_q = norm_p < a.batch ? norm_p : group;  // a row in range for an idle half's loads
    float norm_row[8], norm_add[8];
    uint16_t norm_w[8];
    if constexpr (normed) {
        const float *row = a.norm_row + static_cast<size_t>(norm_q) * C;
        const float *add = a.norm_add != nullptr ? a.norm_add + static_cast<size_t>(norm_q) * C : row;
#pragma unroll
        for (uint32_t k = 0; k < 8u; ++k) {
            norm_row[k] = row[t256 + 256u * k];
            norm_add[k] = add[t256 + 256u * k];
            norm_w[k] = a.norm_weight[t256 + 256u * k];
        }
    } else {
#pragma unroll
        for (uint32_t i = 0; i < kMine; ++i) {
            const uint32_t p = group + halves * i;
            if (p < a.batch) {
                load_wave<VC>(a.x + static_cast<size_t>(p) * C + w8 * CH, lane, xv[i]);
            }
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    load_codes(b);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (uint32_t k = 0; k < kTablePer; ++k) {
        table[threadIdx.x + k * kNeFusedThreads] = tab[k];
    }
#pragma unroll
    for (uint32_t k = 0; k < kSignPer; ++k) {
        const uint32_t i = threadIdx.x + k * kNeFusedThreads;
        if (i < sign_words) {
            reinterpret_cast<uint32_t *>(sv_lds)[i] = signs[k];
        }
    }
    // with a norm the half's input rows are computed here, into the x_hat
    // rows' place; the first block of the half writes them out
    if constexpr (normed) {
        {
            float v[8], w[8];
#pragma unroll
            for (uint32_t k = 0; k < 8u; ++k) {
                v[k] = a.norm_add != nullptr ? norm_row[k] + norm_add[k] : norm_row[k];
                w[k] = bf16_bits_to_float(norm_w[k]);
            }
            block_rms_norm_held(v, w, [](uint32_t, float) {}, C, 1.0f, 1.0e-6f, ne_lds + norm_q * C,
                                norm_sums[pair], &norm_scale[pair], norm_p < a.batch ? t256 : 256u);
            __syncthreads();
            if (g == 0) {
                for (uint32_t p = group; p < a.batch; p += halves) {
                    for (uint32_t e = threadIdx.x; e < C / 4u; e += kNeFusedThreads) {
                        reinterpret_cast<float4 *>(a.x_out + static_cast<size_t>(p) * C)[e] =
                            reinterpret_cast<const float4 *>(ne_lds + p * C)[e];
                    }
                }
                __syncthreads();  // copied before the x_hat rows overwrite them
            }
#pragma unroll
            for (uint32_t i = 0; i < kMine; ++i) {
                const uint32_t p = group + halves * i;
                if (p < a.batch) {
                    load_wave<VC>(ne_lds + p * C + w8 * CH, lane, xv[i]);
                }
            }
        }
    }
    // x_hat of the half's input rows
#pragma unroll
    for (uint32_t i = 0; i < kMine; ++i) {
        const uint32_t p = group + halves * i;
        if (p < a.batch) {
#pragma unroll
            for (int e = 0; e < VC; ++e) {
                xv[i][e] = xv[i][e] * xs[e];
            }
            wave_hadamard<VC>(xv[i], 1.0f, lane);
            store_wave<VC>(ne_lds + p * C + w8 * CH, lane, xv[i]);
        }
    }
    __syncthreads();
    for (uint32_t p = group; p < a.batch; p += halves) {
        hadamard_cross_span<CH>(ne_lds + p * C, a.scale_columns, w8, lane);
    }
    __syncthreads();
    for (uint32_t tr = b; tr < tile_rows; tr += kRoundRows * blocks) {
#pragma unroll
        for (uint32_t q = 0; q < kWaveItems; ++q) {
            const uint32_t i8 = w8 + 8u * q;
            if (i8 < per_row) {
                // the table values of the item in each of the round's tile rows
                uint32_t w[kRoundRows][32];
#pragma unroll
                for (uint32_t u = 0; u < kRoundRows; ++u) {
                    if (tr + u * blocks >= tile_rows) {
                        break;
                    }
                    const uint32_t d[9] = {code[u][q][0].x, code[u][q][0].y, code[u][q][0].z, code[u][q][0].w,
                                           code[u][q][1].x, code[u][q][1].y, code[u][q][1].z, code[u][q][1].w,
                                           quad_next(code[u][q][0].x) & 0xFFFFu};
                    uint32_t idx[32];
                    decode_ne_quad(d, idx);
#pragma unroll
                    for (int k = 0; k < 32; ++k) {
                        w[u][k] = table[idx[k]];
                    }
                }
                const uint32_t column = (i8 * 16u + tslot) << 4;
#pragma unroll
                for (uint32_t i = 0; i < kMine; ++i) {
                    const uint32_t p = group + halves * i;
                    if (p >= a.batch) {
                        break;
                    }
                    float x[16];
                    const float4 *src = reinterpret_cast<const float4 *>(ne_lds + p * C + column);
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const float4 t = src[e];
                        x[4 * e] = t.x;
                        x[4 * e + 1] = t.y;
                        x[4 * e + 2] = t.z;
                        x[4 * e + 3] = t.w;
                    }
#pragma unroll
                    for (uint32_t u = 0; u < kRoundRows; ++u) {
                        if (tr + u * blocks >= tile_rows) {
                            break;
                        }
                        float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                        for (int s = 0; s < 8; ++s) {
#pragma unroll
                            for (int r = 0; r < 4; ++r) {
                                const float2 wv = half2_bits_to_float2(w[u][8 * r + s]);
                                acc[r] = fmaf(wv.x, x[2 * s], acc[r]);
                                acc[r] = fmaf(wv.y, x[2 * s + 1], acc[r]);
                            }
                        }
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            acc[r] = sum_over_quads(acc[r], 16u);
                        }
                        if (tslot == 0) {
#pragma unroll
                            for (int r = 0; r < 4; ++r) {
                                part[u * per_row + i8][quad * 4u + r][p] = acc[r] * job.weight_scale;
                            }
                        }
                    }
                }
            }
        }
        if (tr + kRoundRows * blocks < tile_rows) {
            load_codes(tr + kRoundRows * blocks);
        }
        __syncthreads();
        // the slice-order sum of each tile row's items: ((0 + item 0) + item 1) + ...
        {
            const uint32_t r = threadIdx.x & 15u, i = (threadIdx.x >> 4) % kMine, u = (threadIdx.x >> 4) / kMine;
            const uint32_t p = group + halves * i, t = tr + u * blocks;
            if (u < kRoundRows && p < a.batch && t < tile_rows) {
                float sum = 0.0f;
                for (uint32_t k = 0; k < per_row; ++k) {
                    sum = sum + part[u * per_row + k][r][p];
                }
                coherent_store(reinterpret_cast<uint32_t *>(job.zsum) + static_cast<size_t>(p) * R + t * kTile + r,
                               __float_as_uint(sum));
            }
        }
        __syncthreads();
    }
    wait_stores();
    __syncthreads();
    if (threadIdx.x == 0) {
        last = coherent_add(ticket, 1u) + 1u == blocks ? 1u : 0u;
    }
    __syncthreads();
    if (last != 0u) {
        // the last block of the matrix and half: the row transform
        switch (R) {
        case 512u: ne_fused_rows<1>(job, ne_lds, sv_lds, group, halves, a.batch, w8, lane, norm_sums, norm_scale); break;
        case 2048u: ne_fused_rows<4>(job, ne_lds, sv_lds, group, halves, a.batch, w8, lane, norm_sums, norm_scale); break;
        case 4096u: ne_fused_rows<8>(job, ne_lds, sv_lds, group, halves, a.batch, w8, lane, norm_sums, norm_scale); break;
        default: ne_fused_rows<16>(job, ne_lds, sv_lds, group, halves, a.batch, w8, lane, norm_sums, norm_scale); break;
        }
        if (threadIdx.x == 0) {
            coherent_store(ticket, 0u);
        }
    }
    if (a.norm_row != nullptr && a.norm_add != nullptr) {
        // the residual sum back into the input rows, by the last block
        // through (every block has read them by then)
        __syncthreads();
        if (threadIdx.x == 0) {
            last = coherent_add(a.ticket + 256u, 1u) + 1u == gridDim.x ? 1u : 0u;
        }
        __syncthreads();
        if (last != 0u) {
            for (uint32_t p = 0; p < a.batch; ++p) {
                float4 *row = reinterpret_cast<float4 *>(a.norm_row + static_cast<size_t>(p) * C);
                const float4 *add = reinterpret_cast<const float4 *>(a.norm_add + static_cast<size_t>(p) * C);
                for (uint32_t e = threadIdx.x; e < C / 4u; e += kNeFusedThreads) {
                    const float4 u = row[e], v = add[e];
                    row[e] = make_float4(u.x + v.x, u.y + v.y, u.z + v.z, u.w + v.w);
                }
            }
            if (threadIdx.x == 0) {
                coherent_store(a.ticket + 256u, 0u);
            }
        }
    }
}

}  // namespace

// ---- launchers -------------------------------------------------------------

bool launch_ne_fused(adi_hip_context *ctx, const adi_hip_ne_matrix *const *m, uint32_t count,
                     const float *inputs, uint32_t batch, float *const *outputs, float *zsum,
                     const NeNormIn *in, const NeNormTail *tail) {
    if (batch == 0 || batch > kNeFusedRows || count == 0 || count > kNeFusedJobs || ctx->moe_sync == nullptr ||
        !aligned_to(zsum, 16) || (in == nullptr && !aligned_to(inputs, 16))) {
        return false;
    }
    if (in != nullptr && (m[0]->columns != 2048u || in->row == nullptr || in->weight == nullptr ||
                          in->out == nullptr || !aligned_to(in->row, 16) || !aligned_to(in->add, 16) ||
                          !aligned_to(in->out, 16))) {
        return false;
    }
    if (tail != nullptr && (m[0]->rows != 2048u || tail->row == nullptr || tail->weight == nullptr ||
                            tail->out == nullptr)) {
        return false;
    }
    const uint32_t columns = m[0]->columns;
    uint32_t widest = columns, tile_rows = 0;
    for (uint32_t j = 0; j < count; ++j) {
        const uint32_t rows = m[j]->rows;
        if (m[j]->columns != columns || (rows != 512u && rows != 2048u && rows != 4096u && rows != 8192u)) {
            return false;
        }
        widest = std::max(widest, rows);
        tile_rows += rows / kTile;
    }
    if (columns != 2048u && columns != 4096u) {
        return false;
    }
    NeFused a{};
    a.jobs = count;
    a.x = inputs;
    if (in != nullptr) {
        a.x = nullptr;
        a.norm_row = in->row;
        a.norm_add = in->add;
        a.norm_weight = in->weight;
        a.x_out = in->out;
    }
    a.ticket = ctx->moe_sync + kMoeSyncNeTicket;
    a.scale_columns = hadamard_scale(columns);
    a.batch = batch;
    a.halves = batch >= 2 ? 2u : 1u;
    // Each matrix gets ceil(tile rows / rounds) blocks, with the fewest rounds
    // of tile rows per block whose blocks fit a half's share of the CUs (one
    // matrix: min(tile rows, share) blocks).
    const uint32_t share = std::max(ctx->cu_count / a.halves, count);
    uint32_t rounds = ceil_div(tile_rows, share), blocks = 0;
    for (;; ++rounds) {
        blocks = 0;
        for (uint32_t j = 0; j < count; ++j) {
            blocks += ceil_div(m[j]->rows / kTile, rounds);
        }
        if (blocks <= share) {
            break;
        }
    }
    // two tile rows a round at 2048 columns (one item a wave each) when a
    // block has more than one; a 4096-column tile row has two items a wave
    using Kernel = void (*)(NeFused);
    const bool norm = in != nullptr;
    const Kernel kernel =
        columns == 4096u ? k_ne_fused<8, 1, false>
                         : (rounds > 1u ? (norm ? k_ne_fused<4, 2, true> : k_ne_fused<4, 2, false>)
                                        : (norm ? k_ne_fused<4, 1, true> : k_ne_fused<4, 1, false>));
    float *sums = zsum;
    uint32_t first = 0;
    for (uint32_t j = 0; j < count; ++j) {
        NeFusedJob &job = a.job[j];
        job.trellis = m[j]->trellis;
        job.su = m[j]->su;
        job.sv = m[j]->sv;
        job.table = static_cast<const uint32_t *>(m[j]->codebook->data);
        job.zsum = sums;
        job.out = outputs[j];
        job.weight_scale = m[j]->weight_scale;
        job.scale_rows = hadamard_scale(m[j]->rows);
        job.rows = m[j]->rows;
        job.first_block = first;
        job.blocks = ceil_div(m[j]->rows / kTile, rounds);
        if (j == 0 && tail != nullptr) {
            job.tail_row = tail->row;
            job.tail_weight = tail->weight;
            job.tail_out = tail->out;
        }
        first += job.blocks;
        sums += size_t(batch) * m[j]->rows;
    }
    const size_t lds = size_t(batch) * widest * sizeof(float);
    require(lds <= 65536 || set_lds_limit(reinterpret_cast<const void *>(kernel), lds),
            "one-launch NE projection: LDS limit");
    launch(ctx, "ne_fused", kernel, dim3(a.halves * blocks), dim3(kNeFusedThreads), lds, a);
    return true;
}

bool wave_width(uint32_t n) { return n >= 64 && n <= 4096 && is_power_of_two(n); }

void prepare_prologues(PrologueJobs &jobs) {
    jobs.scale = hadamard_scale(jobs.n);
    for (uint32_t s = 0; s < jobs.segments; ++s) {
        const PrologueSegment &g = jobs.seg[s];
        require(aligned_to(g.x, 16) && aligned_to(g.su_f16, 8) && aligned_to(g.su_sign, 4) &&
                    aligned_to(g.out.f32, 16) && aligned_to(g.out.hi, 16) && aligned_to(g.out.lo, 16),
                "vectors must be 16-byte aligned, f16 scale rows 8-byte and sign rows 4-byte");
    }
}

void launch_prologues(adi_hip_context *ctx, PrologueJobs &jobs) {
    uint32_t vectors = 0;
    for (uint32_t s = 0; s < jobs.segments; ++s) {
        vectors += jobs.seg[s].count;
    }
    prepare_prologues(jobs);
    if ((jobs.n == 2048u || jobs.n == 4096u) && vectors <= kBlockVectors) {
        if (jobs.n == 2048u) {
            launch(ctx, "hadamard_prologue", k_prologue_block<4>, dim3(vectors), dim3(512), 0, jobs);
        } else {
            launch(ctx, "hadamard_prologue", k_prologue_block<8>, dim3(vectors), dim3(512), 0, jobs);
        }
        return;
    }
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
            require(g.out.planes == 0, "f16 x_hat output needs a width of 64..4096");
            if (g.su_f16 != nullptr) {
                launch(ctx, "hadamard_prologue", k_prologue<uint16_t>, dim3(g.count), dim3(256),
                       jobs.n * sizeof(float), g.x, jobs.n, g.su_f16, g.su_stride, g.source_row,
                       g.matrix_index, jobs.scale, g.out.f32);
            } else {
                launch(ctx, "hadamard_prologue", k_prologue<int8_t>, dim3(g.count), dim3(256),
                       jobs.n * sizeof(float), g.x, jobs.n, g.su_sign, 0u, g.source_row,
                       static_cast<const uint32_t *>(nullptr), jobs.scale, g.out.f32);
            }
        }
    }
}

template <typename Scale>
void launch_epilogue_any(adi_hip_context *ctx, const float *z, uint32_t splits,
                         size_t split_stride, uint32_t n, const Scale *sv, uint32_t vectors,
                         float *out) {
    const float scale = hadamard_scale(n);
    require(aligned_to(z, 16) && aligned_to(out, 16) && aligned_to(sv, sizeof(Scale) == 2 ? 8 : 4),
            "vectors must be 16-byte aligned, f16 scale rows 8-byte and sign rows 4-byte");
    // few vectors over many slice bytes (128 KiB and up): add the slices
    // across the GPU first
    if (splits > 1 && vectors <= 8 && size_t(splits) * vectors * n >= 32768 && n % 4 == 0 &&
        split_stride % 4 == 0) {
        const uint32_t count4 = vectors * n / 4;
        launch(ctx, "reduce_slices", k_reduce_slices, dim3(ceil_div(count4, 64)), dim3(64), 0,
               const_cast<float *>(z), splits, split_stride, count4);
        splits = 1;
    }
    if ((n == 2048u || n == 4096u || n == 8192u) && vectors <= kBlockVectors) {
        if (n == 2048u) {
            launch(ctx, "hadamard_epilogue", k_epilogue_block<4, Scale>, dim3(vectors), dim3(512), 0, z, splits,
                   split_stride, sv, scale, out);
        } else if (n == 4096u) {
            launch(ctx, "hadamard_epilogue", k_epilogue_block<8, Scale>, dim3(vectors), dim3(512), 0, z, splits,
                   split_stride, sv, scale, out);
        } else {
            launch(ctx, "hadamard_epilogue", k_epilogue_block<16, Scale>, dim3(vectors), dim3(512), 0, z, splits,
                   split_stride, sv, scale, out);
        }
        return;
    }
    const dim3 grid(ceil_div(vectors, 4));
    switch (n) {
    case 64: launch(ctx, "hadamard_epilogue", k_epilogue_wave<1, Scale>, grid, dim3(256), 0, z, splits, split_stride, sv, vectors, scale, out); break;
    case 128: launch(ctx, "hadamard_epilogue", k_epilogue_wave<2, Scale>, grid, dim3(256), 0, z, splits, split_stride, sv, vectors, scale, out); break;
    case 256: launch(ctx, "hadamard_epilogue", k_epilogue_wave<4, Scale>, grid, dim3(256), 0, z, splits, split_stride, sv, vectors, scale, out); break;
    case 512: launch(ctx, "hadamard_epilogue", k_epilogue_wave<8, Scale>, grid, dim3(256), 0, z, splits, split_stride, sv, vectors, scale, out); break;
    case 1024: launch(ctx, "hadamard_epilogue", k_epilogue_wave<16, Scale>, grid, dim3(256), 0, z, splits, split_stride, sv, vectors, scale, out); break;
    case 2048: launch(ctx, "hadamard_epilogue", k_epilogue_wave<32, Scale>, grid, dim3(256), 0, z, splits, split_stride, sv, vectors, scale, out); break;
    case 4096: launch(ctx, "hadamard_epilogue", k_epilogue_wave<64, Scale>, grid, dim3(256), 0, z, splits, split_stride, sv, vectors, scale, out); break;
    case 8192: launch(ctx, "hadamard_epilogue", k_epilogue_8192<Scale>, dim3(vectors), dim3(256), 0, z, splits, split_stride, sv, scale, out); break;
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

// Fills the launch geometry of `m`; returns the grid (0: nothing to do).
uint32_t plan_trellis_gemv(adi_hip_context *ctx, MoeGemv &m) {
    require(m.expert_count <= 2 && m.ne_count <= 2, "trellis GEMV: too many matrices");
    require(m.expert_count == 0 || m.expert_book != nullptr, "trellis GEMV: expert codebook missing");
    require(m.ne_count == 0 || m.ne_book != nullptr, "trellis GEMV: NE codebook missing");
    if (m.expert_count > 0) {
        const ExpertGemv &e = m.expert[0];
        require(m.max_active >= 1 && m.max_active <= kMaxSlots, "trellis GEMV: routed slots out of range");
        require(m.slot_info != nullptr || m.max_active == 1, "trellis GEMV: routed slots need a slot table");
        const uint32_t tiles = (e.rows / kTile) * (e.columns / kTile);
        m.expert_items_per_slot = ceil_div(tiles, 16u * item_groups(e.columns / kTile));
        m.item_shift = log2_of(m.expert_items_per_slot);
        for (uint32_t i = 0; i < m.expert_count; ++i) {
            ExpertGemv &x = m.expert[i];
            require(x.rows == e.rows && x.columns == e.columns,
                    "trellis GEMV: expert entries differ in shape");
            x.tile_rows = x.rows / kTile;
            x.tc_shift = log2_of(x.columns / kTile);
            x.group_shift = log2_of(item_groups(x.columns / kTile));
        }
        m.slot_capacity = m.max_active;
    } else {
        m.expert_items_per_slot = 0;
        m.slot_capacity = 0;
    }
    m.expert_items = m.expert_count * m.max_active * m.expert_items_per_slot;
    if (m.ne_count > 0) {
        const NeGemv &n = m.ne[0];
        const uint32_t tiles = (n.rows / kTile) * (n.columns / kTile);
        m.ne_items_per_matrix = ceil_div(tiles, 16u);
        for (uint32_t i = 0; i < m.ne_count; ++i) {
            NeGemv &x = m.ne[i];
            require(x.rows == n.rows && x.columns == n.columns,
                    "trellis GEMV: NE entries differ in shape");
            x.tile_rows = x.rows / kTile;
            x.tc_shift = log2_of(x.columns / kTile);
        }
    } else {
        m.ne_items_per_matrix = 0;
    }
    m.ne_items = m.ne_count * m.ne_items_per_matrix;
    m.half_items[0] = m.expert_items + (m.ne_items + 1) / 2;
    m.half_items[1] = m.expert_items + m.ne_items / 2;
    if (m.half_items[0] == 0) {
        return 0;
    }
    // persistent grid: at most one block per CU, a multiple of 16 blocks
    const uint32_t needed_workers = ceil_div(m.half_items[0], kGemvWaves);
    uint32_t blocks = 16u * ceil_div(needed_workers, 8);
    const uint32_t cap = ctx->cu_count >= 16 ? ctx->cu_count / 16 * 16 : 16u;
    return blocks < cap ? blocks : cap;
}

bool trellis_gemv_can_fuse_swiglu(adi_hip_context *ctx, MoeGemv m) {
    const uint32_t blocks = plan_trellis_gemv(ctx, m);
    return blocks > 0 && m.expert_count == 1 && m.slot_info != nullptr &&
           m.expert[0].columns == kFusedSwigluWidth &&
           (m.ne_count == 0 || m.ne[0].columns == kFusedSwigluWidth) &&
           m.expert_items <= (blocks / 2) * kGemvWaves;
}

void launch_trellis_gemv(adi_hip_context *ctx, MoeGemv &m) {
    require(m.fused_swiglu == 0 || trellis_gemv_can_fuse_swiglu(ctx, m),
            "trellis GEMV: the fused SwiGLU needs one row and one expert item per wave");
    const uint32_t blocks = plan_trellis_gemv(ctx, m);
    if (blocks == 0) {
        return;
    }
    const size_t lds = size_t(m.slot_capacity) * 16 + (m.expert_count > 0 ? kPlaneBytes : 0) +
                       (m.fused_swiglu != 0 ? size_t(1 + kGemvWaves) * kFusedSwigluWidth * 4 : 0);
    // LDS is 160 KiB; the kernel's static NE table takes 4 KiB
    constexpr size_t kMaxDynamic = 160 * 1024 - 4096;
    require(lds <= kMaxDynamic, "trellis GEMV: LDS plan exceeds 156 KiB");
    static const bool ready =
        set_lds_limit(reinterpret_cast<const void *>(&k_trellis_gemv), kMaxDynamic);
    (void)ready;
    launch(ctx, "moe_gemv", k_trellis_gemv, dim3(blocks), dim3(kGemvThreads), lds, m);
}

bool plan_moe_decode_one(adi_hip_context *ctx, MoeDecodeOne &a) {
    if (ctx->cu_count < 16 || (ctx->isa_lanes != 8 && ctx->isa_lanes != 16) || a.sync == nullptr ||
        a.experts < 8 || a.experts > kFusedMaxExperts || a.gu.expert_count != 2 || a.gu.ne_count != 2 ||
        a.dn.expert_count != 1 || a.dn.ne_count != 1 || a.gu.max_active != kFusedSlots ||
        a.dn.max_active != kFusedSlots || a.gu.ne_book != a.dn.ne_book) {
        return false;
    }
    const ExpertGemv &g = a.gu.expert[0], &d = a.dn.expert[0];
    if (g.rows != kFusedSwigluWidth || g.columns != kFusedHidden || d.rows != kFusedHidden ||
        d.columns != kFusedSwigluWidth || a.gu.ne[0].rows != kFusedSwigluWidth ||
        a.gu.ne[0].columns != kFusedHidden || a.dn.ne[0].rows != kFusedHidden ||
        a.dn.ne[0].columns != kFusedSwigluWidth) {
        return false;
    }
    const uint32_t blocks = ctx->cu_count / 16 * 16;
    if (plan_trellis_gemv(ctx, a.gu) != blocks || plan_trellis_gemv(ctx, a.dn) != blocks) {
        return false;
    }
    // one item per wave, a block's eight items in one slot, every router row
    // on some block (rows b and 2 blocks - 1 - b), every shared gate/up NE
    // item on a wave (two per block), one shared down NE item per block
    const uint32_t wave_items = (blocks / 2) * kGemvWaves;
    if (a.gu.expert_items != wave_items || a.dn.expert_items != wave_items ||
        a.gu.expert_items_per_slot % kGemvWaves != 0 || a.dn.expert_items_per_slot % kGemvWaves != 0 ||
        a.experts + 1 > 2 * blocks || a.gu.ne_items != 2 * a.gu.ne_items_per_matrix ||
        a.gu.ne_items_per_matrix > blocks || a.dn.ne_items != blocks) {
        return false;
    }
    // the slot-per-XCD assignment: eight slots on eight XCDs, each (XCD,
    // half) pair's blocks running one slot's gate and up items (half each)
    // and all of its down items
    static_assert(kFusedSlots == 8, "one routed slot per XCD");
    if (blocks % 32u != 0 || a.gu.expert_items_per_slot * 32u != blocks * kGemvWaves ||
        a.dn.expert_items_per_slot * 16u != blocks * kGemvWaves) {
        return false;
    }
    // each half of the grid runs every item once
    a.expect_slot = 2u * a.gu.expert_count * a.gu.expert_items_per_slot;
    a.expect_down = 2u * a.dn.expert_items_per_slot;
    a.down_splits = expert_splits(kFusedSwigluWidth);
    a.shared_down_splits = ne_splits(kFusedSwigluWidth);
    return true;
}

void launch_moe_decode_one(adi_hip_context *ctx, const MoeDecodeOne &a) {
    const uint32_t blocks = ctx->cu_count / 16 * 16;
    const size_t lds = kPlaneBytes + kFusedRegion;
    if (ctx->isa_lanes == 16) {
        static const bool ready =
            set_lds_limit(reinterpret_cast<const void *>(&k_moe_decode_one<16>), lds);
        (void)ready;
        launch(ctx, "moe_decode_one", k_moe_decode_one<16>, dim3(blocks), dim3(kFusedThreads), lds, a);
    } else {
        static const bool ready =
            set_lds_limit(reinterpret_cast<const void *>(&k_moe_decode_one<8>), lds);
        (void)ready;
        launch(ctx, "moe_decode_one", k_moe_decode_one<8>, dim3(blocks), dim3(kFusedThreads), lds, a);
    }
}

bool plan_moe_decode_few(adi_hip_context *ctx, MoeDecodeFew &a) {
    if (ctx->cu_count < 32 || (ctx->isa_lanes != 8 && ctx->isa_lanes != 16) || a.sync == nullptr ||
        a.error == nullptr || a.batch < 2 || a.batch > kFewMaxRows || a.experts < 8 ||
        a.experts > kFusedMaxExperts || a.gu.expert_count != 2 || a.gu.ne_count != 2 || a.dn.expert_count != 1 ||
        a.dn.ne_count != 1 || a.gu.max_active < 8 * a.batch || a.dn.max_active < 8 * a.batch ||
        a.gu.max_active > kFewMaxRoutes || a.dn.max_active > kFewMaxRoutes || a.gu.ne_book != a.dn.ne_book ||
        a.logits == nullptr || a.parts == nullptr) {
        return false;
    }
    const ExpertGemv &g = a.gu.expert[0], &d = a.dn.expert[0];
    if (g.rows != kFusedSwigluWidth || g.columns != kFusedHidden || d.rows != kFusedHidden ||
        d.columns != kFusedSwigluWidth || a.gu.ne[0].rows != kFusedSwigluWidth ||
        a.gu.ne[0].columns != kFusedHidden || a.dn.ne[0].rows != kFusedHidden ||
        a.dn.ne[0].columns != kFusedSwigluWidth || a.gu.ne[0].batch != a.batch || a.dn.ne[0].batch != a.batch) {
        return false;
    }
    const uint32_t blocks = ctx->cu_count / 32 * 32;
    plan_trellis_gemv(ctx, a.gu);
    plan_trellis_gemv(ctx, a.dn);
    // an (XCD, half) pair of blocks runs one item of every slot of its XCD
    // per wave: both gate/up entries' items, and the down entry's
    const uint32_t pair_waves = blocks / 16u * kGemvWaves;
    if (2u * a.gu.expert_items_per_slot != pair_waves || a.dn.expert_items_per_slot != pair_waves ||
        a.experts + 1 > 2 * blocks || a.gu.ne_items != 2 * a.gu.ne_items_per_matrix ||
        a.gu.ne_items_per_matrix > blocks || a.dn.ne_items != blocks || 2u * a.batch > blocks) {
        return false;
    }
    // the items' tile groups are the ones the kernel stages, and the items
    // cover each matrix exactly
    if ((1u << a.gu.expert[0].group_shift) != kFewGuGroups || (1u << a.gu.expert[1].group_shift) != kFewGuGroups ||
        (1u << d.group_shift) != kFewDnGroups ||
        (g.tile_rows << g.tc_shift) != a.gu.expert_items_per_slot * 16u * kFewGuGroups ||
        (d.tile_rows << d.tc_shift) != a.dn.expert_items_per_slot * 16u * kFewDnGroups) {
        return false;
    }
    a.expect_gu = 2u * a.gu.expert_count * a.gu.expert_items_per_slot;
    a.expect_dn = 2u * a.dn.expert_items_per_slot;
    a.down_splits = expert_splits(kFusedSwigluWidth);
    a.shared_down_splits = ne_splits(kFusedSwigluWidth);
    return true;
}

void launch_moe_decode_few(adi_hip_context *ctx, const MoeDecodeFew &a) {
    const uint32_t blocks = ctx->cu_count / 32 * 32;
    const size_t lds = kPlaneBytes + kFusedRegion;
    if (ctx->isa_lanes == 16) {
        static const bool ready =
            set_lds_limit(reinterpret_cast<const void *>(&k_moe_decode_few<16>), lds);
        (void)ready;
        launch(ctx, "moe_decode_few", k_moe_decode_few<16>, dim3(blocks), dim3(kGemvThreads), lds, a);
    } else {
        static const bool ready =
            set_lds_limit(reinterpret_cast<const void *>(&k_moe_decode_few<8>), lds);
        (void)ready;
        launch(ctx, "moe_decode_few", k_moe_decode_few<8>, dim3(blocks), dim3(kGemvThreads), lds, a);
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
    require(aligned_to(m->su, 4) && aligned_to(m->sv, 4), "Mach NE sign rows must be 4-byte aligned");
}

void ne_matmul_group(adi_hip_context *ctx, const adi_hip_ne_matrix *const *m, uint32_t count,
                     const float *inputs, uint32_t batch, float *const *outputs, const NeNormIn *in,
                     const NeNormTail *tail) {
    require(count > 0 && count <= kNeFusedJobs && batch > 0, "Mach NE batch shape mismatch");
    require(inputs != nullptr || in != nullptr, "Mach NE vector is null");
    size_t floats = 0;
    for (uint32_t j = 0; j < count; ++j) {
        validate_ne(m[j]);
        require(outputs[j] != nullptr, "Mach NE vector is null");
        floats += size_t(batch) * m[j]->rows;
    }
    if (ctx->fused_moe && batch <= kNeFusedRows) {
        auto &ws = ctx->workspace;
        ws.used = 0;
        ws.ensure(Workspace::round(floats * 4));
        float *zsum = ws.take<float>(floats);
        if (launch_ne_fused(ctx, m, count, inputs, batch, outputs, zsum, in, tail)) {
            return;
        }
    }
    if (in != nullptr) {
        launch_add_rms_norm(ctx, in->row, in->add, in->weight, m[0]->columns, batch, in->out);
        inputs = in->out;
    }
    const uint32_t columns = m[0]->columns;
    bool grouped = ctx->fused_moe && count > 1 && batch >= kNeMfmaBatch && columns >= 32 && wave_width(columns) &&
                   size_t(batch) * columns * 2u < (size_t(1) << 32) && aligned_to(inputs, 16);
    for (uint32_t j = 0; j < count; ++j) {
        grouped = grouped && m[j]->columns == columns && m[j]->rows % kTile == 0;
    }
    if (grouped) {
        // the MFMA path of adi_hip_ne_matmul for every matrix, with one
        // prologue launch for all of their x_hat and one MFMA launch for two
        // matrices of one shape and codebook (the same kernels and arithmetic)
        auto &ws = ctx->workspace;
        ws.used = 0;
        uint32_t splits[kNeFusedJobs];
        size_t bytes = 0;
        for (uint32_t j = 0; j < count; ++j) {
            splits[j] = ne_mfma_slices(m[j]->rows, columns, batch);
            bytes += Workspace::round(size_t(batch) * columns * 4) +
                     Workspace::round(size_t(splits[j]) * batch * m[j]->rows * 4);
        }
        ws.ensure(bytes);
        uint16_t *hi[kNeFusedJobs], *lo[kNeFusedJobs];
        float *z[kNeFusedJobs];
        PrologueJobs jobs{};
        jobs.segments = count;
        jobs.n = columns;
        for (uint32_t j = 0; j < count; ++j) {
            hi[j] = reinterpret_cast<uint16_t *>(ws.take<float>(size_t(batch) * columns));
            lo[j] = hi[j] + size_t(batch) * columns;
            z[j] = ws.take<float>(size_t(splits[j]) * batch * m[j]->rows);
            jobs.seg[j] = PrologueSegment{inputs, nullptr, nullptr, nullptr, m[j]->su, 0,
                                          XhatOut{nullptr, hi[j], lo[j], 1, batch}, batch};
        }
        launch_prologues(ctx, jobs);
        bool launched[kNeFusedJobs] = {};
        for (uint32_t j = 0; j < count; ++j) {
            if (launched[j]) {
                continue;
            }
            NeMfmaJobs J{};
            J.ne_book = m[j]->codebook->data;
            for (uint32_t k = j; k < count && J.ne_count < 2u; ++k) {
                if (launched[k] || m[k]->rows != m[j]->rows || m[k]->codebook->data != J.ne_book) {
                    continue;
                }
                NeMfma &n = J.ne[J.ne_count++];
                n.trellis = m[k]->trellis;
                n.weight_scale = m[k]->weight_scale;
                n.rows = m[k]->rows;
                n.columns = columns;
                n.x_hi = hi[k];
                n.x_lo = lo[k];
                n.batch = batch;
                n.z = z[k];
                launched[k] = true;
            }
            launch_ne_mfma(ctx, J);
        }
        for (uint32_t j = 0; j < count; ++j) {
            launch_epilogue_any<int8_t>(ctx, z[j], splits[j], size_t(batch) * m[j]->rows, m[j]->rows, m[j]->sv,
                                        batch, outputs[j]);
        }
    } else {
        for (uint32_t j = 0; j < count; ++j) {
            const int status = adi_hip_ne_matmul(ctx, m[j], inputs, batch, outputs[j]);
            if (status != ADI_HIP_OK) {
                fail(status, ctx->last_error());
            }
        }
    }
    if (tail != nullptr) {
        launch_add_rms_norm(ctx, tail->row, outputs[0], tail->weight, m[0]->rows, batch, tail->out);
    }
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
        const bool mfma = batch >= kExpertMfmaBatch && expert_mfma_supports(m->rows, m->columns) &&
                          wave_width(m->columns);
        const uint32_t splits = mfma ? 2u : expert_splits(m->columns);
        auto &ws = ctx->workspace;
        ws.used = 0;
        ws.ensure(Workspace::round(size_t(batch) * m->columns * 4) +
                  Workspace::round(size_t(splits) * batch * m->rows * 4));
        float *x_hat = ws.take<float>(size_t(batch) * m->columns);
        float *z = ws.take<float>(size_t(splits) * batch * m->rows);
        PrologueJobs jobs{};
        jobs.segments = 1;
        jobs.n = m->columns;
        uint16_t *hi = reinterpret_cast<uint16_t *>(x_hat);
        uint16_t *lo = hi + size_t(batch) * m->columns;
        jobs.seg[0] = PrologueSegment{inputs, nullptr, nullptr, m->su_f16, nullptr, 0,
                                      mfma ? XhatOut{nullptr, hi, lo, 2, batch}
                                           : XhatOut{x_hat, nullptr, nullptr, 0, batch},
                                      batch};
        launch_prologues(ctx, jobs);
        if (mfma) {
            ExpertMfmaJobs J{};
            ExpertMfma &e = J.expert[0];
            e.trellis = m->trellis;
            e.gamma = m->wave_gamma_f16;
            e.rows = m->rows;
            e.columns = m->columns;
            e.x_hi = hi;
            e.x_lo = lo;
            e.positions = batch;
            e.z = z;
            e.z_split_stride = size_t(batch) * m->rows;
            J.expert_count = 1;
            J.expert_book = m->codebook->data;
            J.max_active = 1;
            J.max_positions = batch;
            launch_expert_mfma(ctx, J);
            launch_epilogue_any<uint16_t>(ctx, z, splits, size_t(batch) * m->rows, m->rows,
                                          m->sv_f16, batch, outputs);
            return;
        }
        MoeGemv g{};
        ExpertGemv &e = g.expert[0];
        e.trellis = m->trellis;
        e.gamma = m->wave_gamma_f16;
        e.rows = m->rows;
        e.columns = m->columns;
        e.x_hat = x_hat;
        e.z = z;
        e.z_split_stride = size_t(batch) * m->rows;
        e.batch = batch;
        g.expert_count = 1;
        g.expert_book = m->codebook->data;
        g.max_active = 1;
        launch_trellis_gemv(ctx, g);
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
        if (ctx->fused_moe && batch <= kNeFusedRows) {
            auto &ws = ctx->workspace;
            ws.used = 0;
            ws.ensure(Workspace::round(size_t(batch) * m->rows * 4));
            float *zsum = ws.take<float>(size_t(batch) * m->rows);
            if (launch_ne_fused(ctx, &m, 1, inputs, batch, &outputs, zsum)) {
                return;
            }
        }
        const bool mfma = batch >= kNeMfmaBatch && m->columns >= 32 && wave_width(m->columns);
        const uint32_t splits = mfma ? ne_mfma_slices(m->rows, m->columns, batch) : ne_splits(m->columns);
        auto &ws = ctx->workspace;
        ws.used = 0;
        ws.ensure(Workspace::round(size_t(batch) * m->columns * 4) +
                  Workspace::round(size_t(splits) * batch * m->rows * 4));
        float *x_hat = ws.take<float>(size_t(batch) * m->columns);
        float *z = ws.take<float>(size_t(splits) * batch * m->rows);
        PrologueJobs jobs{};
        jobs.segments = 1;
        jobs.n = m->columns;
        uint16_t *hi = reinterpret_cast<uint16_t *>(x_hat);
        uint16_t *lo = hi + size_t(batch) * m->columns;
        jobs.seg[0] = PrologueSegment{inputs, nullptr, nullptr, nullptr, m->su, 0,
                                      mfma ? XhatOut{nullptr, hi, lo, 1, batch}
                                           : XhatOut{x_hat, nullptr, nullptr, 0, batch},
                                      batch};
        launch_prologues(ctx, jobs);
        if (mfma) {
            NeMfmaJobs J{};
            NeMfma &n = J.ne[0];
            n.trellis = m->trellis;
            n.weight_scale = m->weight_scale;
            n.rows = m->rows;
            n.columns = m->columns;
            n.x_hi = hi;
            n.x_lo = lo;
            n.batch = batch;
            n.z = z;
            J.ne_count = 1;
            J.ne_book = m->codebook->data;
            launch_ne_mfma(ctx, J);
            launch_epilogue_any<int8_t>(ctx, z, splits, size_t(batch) * m->rows, m->rows, m->sv,
                                        batch, outputs);
            return;
        }
        MoeGemv g{};
        NeGemv &n = g.ne[0];
        n.trellis = m->trellis;
        n.weight_scale = m->weight_scale;
        n.rows = m->rows;
        n.columns = m->columns;
        n.x_hat = x_hat;
        n.z = z;
        n.z_split_stride = size_t(batch) * m->rows;
        n.batch = batch;
        g.ne_count = 1;
        g.ne_book = m->codebook->data;
        launch_trellis_gemv(ctx, g);
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
        require(n < 512 || aligned_to(values, 16), "Hadamard vectors must be 16-byte aligned");
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
