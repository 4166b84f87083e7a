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
constexpr size_t kPlaneBytes = size_t(kExpertRows) * 8;  // one component plane
constexpr uint32_t kMaxSlots = 1024;                     // routed slots staged in LDS

// The loads of one expert wave item, issued one item ahead of its arithmetic
// so that a wave's next item is in flight while the current one computes.
struct ExpertStage {
    uint4 info;         // {matrix, first position, end position, -}; empty when end == first
    uint32_t d[4][3];   // the lane's three stream dwords in each group of 16 tiles
    float gamma[4];
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
                                                const float *x_lds = nullptr) {
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
    const uint32_t *words = reinterpret_cast<const uint32_t *>(a.trellis + st.info.x * a.trellis_stride);
    const uint16_t *gamma_row = a.gamma + st.info.x * a.gamma_stride;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        valid[g] = valid[g] && live;
        st.d[g][0] = st.d[g][1] = st.d[g][2] = 0u;
        st.gamma[g] = 0.0f;
        if (valid[g]) {
            const uint32_t *src = words + static_cast<size_t>(tile[g]) * 12u + quad * 3u;
            st.d[g][0] = __builtin_nontemporal_load(src);
            st.d[g][1] = __builtin_nontemporal_load(src + 1);
            st.d[g][2] = __builtin_nontemporal_load(src + 2);
            const uint32_t tr = tile[g] >> a.tc_shift, tc = tile[g] & (tile_columns - 1u);
            st.gamma[g] = half_bits_to_float(gamma_row[wave_slot(tr, tc, a.tile_rows, tile_columns)]);
        }
    }
    // a fused SwiGLU's x_hat sits in LDS for the item's single position
    load_x_pair(x_lds != nullptr ? x_lds : a.x_hat, a.columns, x_lds != nullptr ? 0u : st.info.y,
                column, groups, valid, st.x);
}

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
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                acc[r] = fmaf(partial[r], st.gamma[g], acc[r]);
            }
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            acc[r] = sum_over_quads(acc[r], span);
        }
        if (writer) {
            float *dst = a.z + split * a.z_split_stride + static_cast<size_t>(position) * a.rows +
                         tr * kTile + quad * 4u;
            *reinterpret_cast<float4 *>(dst) = make_float4(acc[0], acc[1], acc[2], acc[3]);
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

__device__ __forceinline__ void load_x16(const float *x_hat, uint32_t columns, uint32_t position,
                                         uint32_t column, bool valid, float (&x)[16]) {
#pragma unroll
    for (int q = 0; q < 16; ++q) {
        x[q] = 0.0f;
    }
    if (valid) {
        const float4 *src =
            reinterpret_cast<const float4 *>(x_hat + static_cast<size_t>(position) * columns + column);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float4 v = src[q];
            x[4 * q] = v.x;
            x[4 * q + 1] = v.y;
            x[4 * q + 2] = v.z;
            x[4 * q + 3] = v.w;
        }
    }
}

__device__ __forceinline__ void ne_prefetch(const MoeGemv &m, uint32_t k, uint32_t lane,
                                            NeStage &st, const float *x_lds = nullptr) {
    const uint2 it = ne_item_of(m, k);
    const NeGemv &a = m.ne[it.x];
    uint32_t tile, column;
    bool valid;
    ne_tile(a, it.y, lane, tile, valid, column);
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    u32x4 lo = {0u, 0u, 0u, 0u}, hi = {0u, 0u, 0u, 0u};
    if (valid) {
        const u32x4 *src = reinterpret_cast<const u32x4 *>(a.trellis) +
                           static_cast<size_t>(tile) * 8u + (lane & 3u) * 2u;
        lo = __builtin_nontemporal_load(src);
        hi = __builtin_nontemporal_load(src + 1);
    }
    st.d[0] = lo.x; st.d[1] = lo.y; st.d[2] = lo.z; st.d[3] = lo.w;
    st.d[4] = hi.x; st.d[5] = hi.y; st.d[6] = hi.z; st.d[7] = hi.w;
    load_x16(x_lds != nullptr ? x_lds : a.x_hat, a.columns, 0, column, valid && a.batch > 0, st.x);
}

// Row sums over all 16 columns of each tile with the signed table in LDS,
// scaled by Wscale once after the tile sums.
__device__ __forceinline__ void ne_compute(const MoeGemv &m, uint32_t k, const uint32_t *table,
                                           uint32_t lane, NeStage &st) {
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
    float (&x)[16] = st.x;  // position 0's, then reloaded per position
    for (uint32_t position = 0; position < a.batch; ++position) {
        if (position != 0) {
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
            *reinterpret_cast<float4 *>(dst) =
                make_float4(acc[0] * a.weight_scale, acc[1] * a.weight_scale,
                            acc[2] * a.weight_scale, acc[3] * a.weight_scale);
        }
    }
}

// One row's SwiGLU into x_hat (width 512, the wave layout), as the MoE's
// swiglu launch computes it (src/executor.cpp:300-312): the routed row of
// grouped position `row` with expert `expert`'s f16 scales, or the shared
// expert's with its signs. Split in two so that the scale and first four
// slice loads go out before the codebook plane's (loads return in order).
struct SwigluInputs {
    float sa[kFusedSwigluWidth / 64], sb[kFusedSwigluWidth / 64], sc[kFusedSwigluWidth / 64];
    float g[4][kFusedSwigluWidth / 64], u[4][kFusedSwigluWidth / 64];
};

__device__ __forceinline__ void swiglu_issue(const GemvSwiglu &f, bool shared, uint32_t row,
                                             uint32_t expert, uint32_t lane, SwigluInputs &in) {
    constexpr int VPL = kFusedSwigluWidth / 64;
    constexpr uint32_t n = kFusedSwigluWidth;
    const float *zg = shared ? f.shared_z_gate : f.z_gate + static_cast<size_t>(row) * n;
    const float *zu = shared ? f.shared_z_up : f.z_up + static_cast<size_t>(row) * n;
    const size_t stride = shared ? f.shared_split_stride : f.split_stride;
    const uint32_t splits = shared ? f.shared_splits : f.splits;
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
#pragma unroll
    for (uint32_t s = 0; s < 4; ++s) {
        const uint32_t at = s < splits ? s : splits - 1u;  // a missing slice reloads the last
        load_wave<VPL>(zg + at * stride, lane, in.g[s]);
        load_wave<VPL>(zu + at * stride, lane, in.u[s]);
    }
}

__device__ __forceinline__ void swiglu_finish(const GemvSwiglu &f, bool shared, uint32_t row,
                                              uint32_t lane, SwigluInputs &in,
                                              float (&out)[kFusedSwigluWidth / 64]) {
#pragma clang fp contract(off)
    constexpr int VPL = kFusedSwigluWidth / 64;
    constexpr uint32_t n = kFusedSwigluWidth;
    const float *zg = shared ? f.shared_z_gate : f.z_gate + static_cast<size_t>(row) * n;
    const float *zu = shared ? f.shared_z_up : f.z_up + static_cast<size_t>(row) * n;
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
    for (uint32_t s = 4; s < splits; ++s) {
        float a[VPL], c[VPL];
        load_wave<VPL>(zg + s * stride, lane, a);
        load_wave<VPL>(zu + s * stride, lane, c);
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
        const uint32_t *src = static_cast<const uint32_t *>(m.ne_book);
        for (uint32_t i = threadIdx.x; i < 1024u; i += kGemvThreads) {
            ne_table[i] = src[i];
        }
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

}  // namespace

// ---- launchers -------------------------------------------------------------

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

}  // namespace adi_hip

using namespace adi_hip;

extern "C" {

int adi_hip_expert_matmul(adi_hip_context *ctx, const adi_hip_expert_matrix *m,
                          const float *inputs, uint32_t batch, float *outputs) {
    return guarded(ctx, [&] {
        validate_expert(m);
        require(batch > 0, "Mach expert batch shape mismatch");
        require(inputs != nullptr && outputs != nullptr, "Mach expert vector is null");
        const bool mfma = batch >= kMfmaBatch && expert_mfma_supports(m->rows, m->columns) &&
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
        const bool mfma = batch >= kMfmaBatch && m->columns >= 32 && wave_width(m->columns);
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
