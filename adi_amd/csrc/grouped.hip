// grouped.hip -- MFMA grouped GEMMs for prefill microbatches
// (src/kernels.cpp:491-593, 703-800 with the batch kernels of
// src/expert_batch_impl.hpp and src/ne_batch_impl.hpp): the codes are decoded
// straight into the A operand of v_mfma_f32_16x16x32_f16, x_hat is the B
// operand as f16 hi/lo pairs, accumulation is fp32.
//
// Expert codec. In 16x16x32 the lane l holds A[l % 16][8 * (l / 16) + 0..7]:
// eight consecutive K values of one row. With the K axis laid out as the
// eight columns a codebook plane covers in each tile (XhatOut planes 2), those
// eight values are the two half-states of row l % 16 of one tile: exactly two
// gathers from the block's LDS plane. The wave gamma of a tile is folded into
// A in f16: hi = f16(gamma * V), lo = f16(gamma * V - hi) (one packed f16
// multiply and one packed f16 fma; gamma and V are f16, so the product has at
// most 22 significant bits and hi + lo holds it). Three MFMA passes,
// hi*hi + hi*lo + lo*hi, keep the error near fp32 rounding.
//
// NE codec. The 4 KiB signed table gives V exactly in f16 (Wscale is applied
// to the fp32 row sums); two passes, V*hi + V*lo.
//
// A wave item is 4 tile rows x 16*NT positions x the full K. Its next K step's
// trellis words, gammas and B fragments are loaded before the current step's
// MFMAs.
#include "grouped.hpp"

namespace adi_hip {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr uint32_t kMfmaThreads = 256;                   // NE GEMM blocks
constexpr uint32_t kMfmaWaves = kMfmaThreads / kWave;
constexpr uint32_t kRowTiles = 4;                         // NE GEMM: tile rows per item
// expert GEMM shape: positions 16 * kExpertNT, tile rows kExpertRT per item,
// kExpertThreads per block (one block per CU)
constexpr int kExpertNT = 2;
constexpr int kExpertRT = 4;
constexpr int kExpertThreads = 512;
constexpr uint32_t kPlaneRows16 = kExpertRows * 8 / 16;   // 16-byte rows of a plane
constexpr uint32_t kSlotCapacity = 1024;

__device__ __forceinline__ half8 load_half8(const uint16_t *p) {
    return __builtin_bit_cast(half8, *reinterpret_cast<const u32x4 *>(p));
}

__device__ __forceinline__ half8 zero_half8() {
    return __builtin_bit_cast(half8, u32x4{0u, 0u, 0u, 0u});
}

// The 16-bit window at bit r (r <= 48) of the 64-bit string of u16 words
// w0 w1 w2 w3, each read most-significant bit first, where d0 = w0 | w1 << 16
// and d1 = w2 | w3 << 16 (src/expert_trellis.hpp:81-105).
__device__ __forceinline__ uint32_t window64(uint32_t d0, uint32_t d1, uint32_t r) {
    const uint64_t bits = (static_cast<uint64_t>(d0 & 0xFFFFu) << 48) |
                          (static_cast<uint64_t>(d0 >> 16) << 32) |
                          (static_cast<uint64_t>(d1 & 0xFFFFu) << 16) | (d1 >> 16);
    return static_cast<uint32_t>(bits >> (48u - r)) & 0xFFFFu;
}

__device__ __forceinline__ f32x4 mfma(half8 a, half8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// ---- expert ---------------------------------------------------------------

template <int NT, int RT>
struct ExpertStep {
    half8 bh[NT], bl[NT];
    uint32_t d0[RT], d1[RT];
    uint32_t gamma[RT];  // f16 bits
};

// A buffer resource over `bytes` bytes at `base`: loads past the end return 0.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_over(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, bytes, 0x00020000);
}

// Everything about an item that does not change along K: buffer resources,
// per-lane byte offsets (the K step advances the scalar offset only) and the
// lane's window shifts.
template <int NT, int RT>
struct ExpertItem {
    __amdgpu_buffer_rsrc_t xh, xl, words, gamma;
    uint32_t xoff[NT];     // B fragment of position tile j at K step 0
    uint32_t woff[RT];     // the lane's first stream dword of tile row t at K step 0
    uint32_t wnext[RT];    // and its second (row 15 wraps to word 0)
    uint32_t dgamma[RT];   // tr + tile column at K step 0
    uint32_t gamma_top;    // R_t + C_t - 1
    uint32_t tile_columns;
    uint32_t sh0, sh1;     // shifts of the lane's two windows in the 64-bit string
    uint32_t end, p0, tr0;
};

template <int NT, int RT>
__device__ __forceinline__ void expert_load(const ExpertItem<NT, RT> &it, uint32_t kc,
                                            ExpertStep<NT, RT> &s) {
    const uint32_t kx = kc * 64u;   // 32 f16 of B per K step
    const uint32_t kw = kc * 192u;  // 4 tiles of 48 bytes per K step
#pragma unroll
    for (int j = 0; j < NT; ++j) {
        s.bh[j] = __builtin_bit_cast(half8, __builtin_amdgcn_raw_buffer_load_b128(it.xh, it.xoff[j], kx, 0));
        s.bl[j] = __builtin_bit_cast(half8, __builtin_amdgcn_raw_buffer_load_b128(it.xl, it.xoff[j], kx, 0));
    }
#pragma unroll
    for (int t = 0; t < RT; ++t) {
        s.d0[t] = __builtin_amdgcn_raw_buffer_load_b32(it.words, it.woff[t], kw, 0);
        s.d1[t] = __builtin_amdgcn_raw_buffer_load_b32(it.words, it.wnext[t], kw, 0);
        // wave slot of (tr, tc): R_t + C_t - 1 - d, one less past the main
        // anti-diagonal (src/codec_cache.cpp:117-147)
        const uint32_t d = it.dgamma[t] + 4u * kc;
        const uint32_t slot = it.gamma_top - d - (d >= it.tile_columns ? 1u : 0u);
        s.gamma[t] = __builtin_amdgcn_raw_buffer_load_b16(it.gamma, slot * 2u, 0, 0);
    }
}

template <int NT, int RT>
__device__ __forceinline__ void expert_compute(const ExpertItem<NT, RT> &it, uint32_t sign_mask,
                                               const uint2 *plane, const ExpertStep<NT, RT> &s,
                                               f32x4 (&acc)[RT][NT]) {
#pragma clang fp contract(off)
#pragma unroll
    for (int t = 0; t < RT; ++t) {
        // the lane's four stream words, most significant bit first
        const uint64_t bits = (static_cast<uint64_t>(__builtin_amdgcn_alignbit(s.d0[t], s.d0[t], 16)) << 32) |
                              __builtin_amdgcn_alignbit(s.d1[t], s.d1[t], 16);
        const uint32_t w0 = static_cast<uint32_t>(bits >> it.sh0) & 0xFFFFu;
        const uint32_t w1 = static_cast<uint32_t>(bits >> it.sh1) & 0xFFFFu;
        const uint32_t p0 = state_product(w0);
        const uint32_t p1 = state_product(w1);
        uint2 e0 = plane[(p0 >> 1) & 0x3FFFu];
        uint2 e1 = plane[(p1 >> 1) & 0x3FFFu];
        e0.x ^= p0 & sign_mask;
        e1.x ^= p1 & sign_mask;
        const half8 v = __builtin_bit_cast(half8, u32x4{e0.x, e0.y, e1.x, e1.y});
        const _Float16 g = __builtin_bit_cast(_Float16, static_cast<uint16_t>(s.gamma[t]));
        const half8 gv = {g, g, g, g, g, g, g, g};
        const half8 hi = gv * v;
        const half8 lo = __builtin_elementwise_fma(gv, v, -hi);
        // positions past the slot carry another slot's x_hat: their output
        // columns are computed and never stored
#pragma unroll
        for (int j = 0; j < NT; ++j) {
            acc[t][j] = mfma(hi, s.bh[j], acc[t][j]);
        }
#pragma unroll
        for (int j = 0; j < NT; ++j) {
            acc[t][j] = mfma(hi, s.bl[j], acc[t][j]);
        }
#pragma unroll
        for (int j = 0; j < NT; ++j) {
            acc[t][j] = mfma(lo, s.bh[j], acc[t][j]);
        }
    }
}

// Block b serves codebook plane (b / 8) % 2 as worker ((b / 16) * 8 + b % 8)
// (the two blocks that walk the same tiles share an XCD). Each block counts
// the items of every routed slot (position groups x row groups) and scans the
// counts in LDS, so the waves walk only real items, evenly. Items are numbered
// (entry, slot, position group, row group), row group fastest, so the waves of
// a block share B fragments in L1.
template <int NT, int RT, int THREADS>
__global__ __launch_bounds__(THREADS) void k_expert_mfma(ExpertMfmaJobs J) {
    constexpr uint32_t kExpertThreads = THREADS;
    constexpr uint32_t kExpertWaves = THREADS / kWave;
    extern __shared__ uint4 lds_dynamic[];  // [kSlotCapacity] slots, item starts, plane
    uint4 *slots = lds_dynamic;
    uint32_t *starts = reinterpret_cast<uint32_t *>(lds_dynamic + kSlotCapacity);  // [kSlotCapacity + 1]
    uint4 *plane_lds = lds_dynamic + kSlotCapacity + (kSlotCapacity + 16) / 4;
    __shared__ uint32_t wave_sums[kExpertWaves];
    const uint32_t b = blockIdx.x;
    const uint32_t half = (b >> 3) & 1u;
    const uint32_t worker = ((b >> 4) << 3) | (b & 7u);
    const uint32_t workers = gridDim.x >> 1;
    {
        const uint4 *src = static_cast<const uint4 *>(J.expert_book) + half * kPlaneRows16;
        // indexes past the plane are clamped: those threads reload and rewrite
        // its last row, so no load is guarded
        constexpr uint32_t kPer = (kPlaneRows16 + kExpertThreads - 1) / kExpertThreads;
        uint4 v[kPer];
#pragma unroll
        for (uint32_t u = 0; u < kPer; ++u) {
            v[u] = src[min(u * kExpertThreads + threadIdx.x, kPlaneRows16 - 1u)];
        }
        // item counts per slot: each thread owns two consecutive slots
        const uint32_t group = 16u * NT;
        uint32_t count[2];
#pragma unroll
        for (uint32_t k = 0; k < 2; ++k) {
            const uint32_t s = 2u * threadIdx.x + k;
            uint4 info = make_uint4(0u, 0u, 0u, 0u);
            if (s < J.max_active) {
                info = J.slot_info != nullptr ? J.slot_info[s]
                                              : make_uint4(0u, 0u, s == 0 ? J.max_positions : 0u, 0u);
                slots[s] = info;
            }
            count[k] = info.z > info.y ? (info.z - info.y + group - 1u) / group * J.row_groups : 0u;
        }
        // block-wide exclusive scan of the counts (slot order)
        const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
        const uint32_t own = count[0] + count[1];
        uint32_t inclusive = own;
#pragma unroll
        for (int offset = 1; offset < 64; offset <<= 1) {
            const uint32_t other = static_cast<uint32_t>(__shfl_up(static_cast<int>(inclusive), offset));
            if (lane >= static_cast<uint32_t>(offset)) {
                inclusive += other;
            }
        }
        if (lane == 63u) {
            wave_sums[wave] = inclusive;
        }
#pragma unroll
        for (uint32_t u = 0; u < kPer; ++u) {
            plane_lds[min(u * kExpertThreads + threadIdx.x, kPlaneRows16 - 1u)] = v[u];
        }
        __syncthreads();
        uint32_t before = 0;
        for (uint32_t w = 0; w < wave; ++w) {
            before += wave_sums[w];
        }
        const uint32_t exclusive = before + inclusive - own;
        if (2u * threadIdx.x < kSlotCapacity) {
            starts[2u * threadIdx.x] = exclusive;
            starts[2u * threadIdx.x + 1u] = exclusive + count[0];
        }
        if (threadIdx.x == kExpertThreads - 1u) {
            starts[kSlotCapacity] = before + inclusive;  // items per entry
        }
    }
    __syncthreads();
    const uint32_t lane = threadIdx.x & 63u;
    const uint2 *plane = reinterpret_cast<const uint2 *>(plane_lds);
    const uint32_t per_entry = starts[kSlotCapacity];
    const uint32_t total = per_entry * J.expert_count;
    const uint32_t stride = workers * kExpertWaves;
    for (uint32_t i = worker * kExpertWaves + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
         i < total; i += stride) {
        const uint32_t which = i / per_entry;
        const uint32_t local = i - which * per_entry;
        // the slot whose item range holds `local`: last s with starts[s] <= local
        uint32_t lo = 0, hi = J.max_active;
        while (hi - lo > 1u) {
            const uint32_t mid = (lo + hi) >> 1;
            if (starts[mid] <= local) {
                lo = mid;
            } else {
                hi = mid;
            }
        }
        const uint32_t slot = __builtin_amdgcn_readfirstlane(lo);
        const uint32_t within = local - starts[slot];
        const uint32_t rg = within % J.row_groups;
        const uint32_t pg = within / J.row_groups;
        const uint4 info = slots[slot];
        const uint32_t first = __builtin_amdgcn_readfirstlane(info.y);
        const uint32_t mat = __builtin_amdgcn_readfirstlane(info.x);
        const ExpertMfma &a = J.expert[which];
        ExpertItem<NT, RT> it;
        it.end = __builtin_amdgcn_readfirstlane(info.z);
        it.p0 = first + pg * 16u * NT;
        it.tr0 = rg * RT;
        const uint32_t m = lane & 15u, kq = lane >> 4;
        const uint32_t half_columns = a.columns >> 1;
        const uint32_t tile_columns = 1u << a.tc_shift;
        const size_t plane_elems = static_cast<size_t>(a.positions) * half_columns;
        const uint32_t x_bytes = static_cast<uint32_t>(plane_elems * 2u);
        it.xh = buffer_over(a.x_hi + half * plane_elems, x_bytes);
        it.xl = buffer_over(a.x_lo + half * plane_elems, x_bytes);
        const uint32_t tiles = a.tile_rows << a.tc_shift;
        it.words = buffer_over(a.trellis + mat * a.trellis_stride, tiles * 48u);
        it.gamma = buffer_over(a.gamma + mat * a.gamma_stride, (a.tile_rows + tile_columns) * 2u);
#pragma unroll
        for (int j = 0; j < NT; ++j) {
            const uint32_t p = it.p0 + 16u * j + m;
            const uint32_t pc = p < it.end ? p : it.p0;  // clamped: a real, finite row
            it.xoff[j] = (pc * half_columns + kq * 8u) * 2u;
        }
        const uint32_t dw = (24u * m) >> 5;
        const uint32_t dn = dw == 11u ? 0u : dw + 1u;  // row 15 wraps to word 0 (src/expert_trellis.hpp:79-80)
#pragma unroll
        for (int t = 0; t < RT; ++t) {
            const uint32_t tr = min(it.tr0 + t, a.tile_rows - 1u);
            const uint32_t tile = (tr << a.tc_shift) + kq;
            it.woff[t] = (tile * 12u + dw) * 4u;
            it.wnext[t] = (tile * 12u + dn) * 4u;
            it.dgamma[t] = tr + kq;
        }
        it.gamma_top = a.tile_rows + tile_columns - 1u;
        it.tile_columns = tile_columns;
        const uint32_t pos = (24u * m) & 31u;  // bit of state 2m in the loaded words
        it.sh0 = 48u - pos;
        it.sh1 = 36u - pos;
        f32x4 acc[RT][NT];
#pragma unroll
        for (int t = 0; t < RT; ++t) {
#pragma unroll
            for (int j = 0; j < NT; ++j) {
                acc[t][j] = f32x4{0.f, 0.f, 0.f, 0.f};
            }
        }
        const uint32_t steps = tile_columns / 4u;  // a power of two
        const uint32_t sign_mask = half == 0 ? 0x8000u : 0u;
        ExpertStep<NT, RT> s0, s1;
        expert_load<NT, RT>(it, 0, s0);
        if (steps == 1) {
            expert_compute<NT, RT>(it, sign_mask, plane, s0, acc);
        } else {
            // no branch inside the body, so the compiler's wait counts see
            // that only the other stage's loads are outstanding; the last
            // iteration reloads the final step (in bounds, unused)
            for (uint32_t kc = 0; kc < steps; kc += 2) {
                expert_load<NT, RT>(it, kc + 1, s1);
                expert_compute<NT, RT>(it, sign_mask, plane, s0, acc);
                expert_load<NT, RT>(it, min(kc + 2, steps - 1), s0);
                expert_compute<NT, RT>(it, sign_mask, plane, s1, acc);
            }
        }
        float *z = a.z + half * a.z_split_stride;
#pragma unroll
        for (uint32_t t = 0; t < RT; ++t) {
            const uint32_t tr = it.tr0 + t;
            if (tr >= a.tile_rows) {
                continue;
            }
#pragma unroll
            for (int j = 0; j < NT; ++j) {
                const uint32_t p = it.p0 + 16u * j + m;
                if (p < it.end) {
                    *reinterpret_cast<f32x4 *>(z + static_cast<size_t>(p) * a.rows + tr * kTile +
                                               kq * 4u) = acc[t][j];
                }
            }
        }
    }
}

// ---- NE -------------------------------------------------------------------

template <int NT>
struct NeStep {
    half8 bh[NT], bl[NT];
    uint32_t d0[kRowTiles], d1[kRowTiles];
};

template <int NT>
__device__ __forceinline__ void ne_load(const NeMfma &a, uint32_t tr0, uint32_t p0, uint32_t kc,
                                        uint32_t lane, NeStep<NT> &s) {
    const uint32_t m = lane & 15u, kq = lane >> 4;
#pragma unroll
    for (int j = 0; j < NT; ++j) {
        const uint32_t p = p0 + 16u * j + m;
        const uint32_t pc = p < a.batch ? p : p0;
        const size_t at = static_cast<size_t>(pc) * a.columns + kc * 32u + kq * 8u;
        s.bh[j] = load_half8(a.x_hi + at);
        s.bl[j] = load_half8(a.x_lo + at);
    }
    // lane: tile column 2kc + kq/2, columns 8*(kq%2)..+7 of row m = NE states
    // 8m + 4(kq%2) + 0..3, the windows at bits 32*(2m + kq%2) + 8i
    const uint32_t tc = kc * 2u + (kq >> 1);
    const uint32_t dw = 2u * m + (kq & 1u);
    const uint32_t dn = dw == 31u ? 0u : dw + 1u;  // row 15 wraps (src/ne_trellis.hpp:196-200)
    const uint32_t *words = reinterpret_cast<const uint32_t *>(a.trellis);
#pragma unroll
    for (uint32_t t = 0; t < kRowTiles; ++t) {
        const uint32_t tr = min(tr0 + t, a.tile_rows - 1u);
        const size_t tile = (static_cast<size_t>(tr) << a.tc_shift) + tc;
        s.d0[t] = __builtin_nontemporal_load(words + tile * 32u + dw);
        s.d1[t] = __builtin_nontemporal_load(words + tile * 32u + dn);
    }
}

template <int NT>
__device__ __forceinline__ void ne_compute(const NeMfma &a, uint32_t p0, const uint32_t *table,
                                           uint32_t lane, const NeStep<NT> &s,
                                           f32x4 (&acc)[kRowTiles][NT]) {
    const uint32_t m = lane & 15u;
    half8 bh[NT], bl[NT];
#pragma unroll
    for (int j = 0; j < NT; ++j) {
        const bool ok = p0 + 16u * j + m < a.batch;
        bh[j] = ok ? s.bh[j] : zero_half8();
        bl[j] = ok ? s.bl[j] : zero_half8();
    }
#pragma unroll
    for (uint32_t t = 0; t < kRowTiles; ++t) {
        uint32_t v[4];
#pragma unroll
        for (uint32_t q = 0; q < 4; ++q) {
            v[q] = table[(state_product(window64(s.d0[t], s.d1[t], 8u * q)) >> 6) & 0x3FFu];
        }
        const half8 w = __builtin_bit_cast(half8, u32x4{v[0], v[1], v[2], v[3]});
#pragma unroll
        for (int j = 0; j < NT; ++j) {
            acc[t][j] = mfma(w, bh[j], acc[t][j]);
        }
#pragma unroll
        for (int j = 0; j < NT; ++j) {
            acc[t][j] = mfma(w, bl[j], acc[t][j]);
        }
    }
}

template <int NT>
__global__ __launch_bounds__(kMfmaThreads) void k_ne_mfma(NeMfmaJobs J) {
    __shared__ uint32_t table[1024];
    const uint32_t *src = static_cast<const uint32_t *>(J.ne_book);
    for (uint32_t i = threadIdx.x; i < 1024u; i += kMfmaThreads) {
        table[i] = src[i];
    }
    __syncthreads();
    const uint32_t i = blockIdx.x * kMfmaWaves + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (i >= J.items) {
        return;
    }
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t rg = i % J.row_groups;
    uint32_t rest = i / J.row_groups;
    const uint32_t ks = rest % J.k_slices;
    rest /= J.k_slices;
    const uint32_t pg = rest % J.position_groups;
    const uint32_t which = rest / J.position_groups;
    const NeMfma &a = J.ne[which];
    const uint32_t p0 = pg * 16u * NT;
    const uint32_t tr0 = rg * kRowTiles;
    f32x4 acc[kRowTiles][NT];
#pragma unroll
    for (uint32_t t = 0; t < kRowTiles; ++t) {
#pragma unroll
        for (int j = 0; j < NT; ++j) {
            acc[t][j] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
    }
    const uint32_t steps = a.columns / 32u / J.k_slices;  // a power of two
    const uint32_t k0 = ks * steps;
    NeStep<NT> s0, s1;
    ne_load<NT>(a, tr0, p0, k0, lane, s0);
    if (steps == 1) {
        ne_compute<NT>(a, p0, table, lane, s0, acc);
    } else {
        for (uint32_t kc = 0; kc < steps; kc += 2) {
            ne_load<NT>(a, tr0, p0, k0 + kc + 1, lane, s1);
            ne_compute<NT>(a, p0, table, lane, s0, acc);
            ne_load<NT>(a, tr0, p0, k0 + min(kc + 2, steps - 1), lane, s0);
            ne_compute<NT>(a, p0, table, lane, s1, acc);
        }
    }
    float *z = a.z + static_cast<size_t>(ks) * a.batch * a.rows;
    const uint32_t m = lane & 15u, kq = lane >> 4;
#pragma unroll
    for (uint32_t t = 0; t < kRowTiles; ++t) {
        const uint32_t tr = tr0 + t;
        if (tr >= a.tile_rows) {
            continue;
        }
#pragma unroll
        for (int j = 0; j < NT; ++j) {
            const uint32_t p = p0 + 16u * j + m;
            if (p < a.batch) {
                const f32x4 r = acc[t][j] * a.weight_scale;
                *reinterpret_cast<f32x4 *>(z + static_cast<size_t>(p) * a.rows + tr * kTile +
                                           kq * 4u) = r;
            }
        }
    }
}

}  // namespace

uint32_t mfma_position_tiles(uint32_t batch) {
    return batch >= 256u ? 4u : (batch >= 64u ? 2u : 1u);
}

uint32_t ne_mfma_slices(uint32_t rows, uint32_t columns, uint32_t batch) {
    const uint32_t nt = mfma_position_tiles(batch);
    const uint32_t items = ceil_div(rows / kTile, kRowTiles) * ceil_div(batch, 16u * nt);
    uint32_t slices = 1;
    // at least about 2048 wave items, each with at least four K steps
    while (items * slices < 2048u && columns / 32u / (slices * 2u) >= 4u) {
        slices *= 2u;
    }
    return slices;
}

void launch_expert_mfma(adi_hip_context *ctx, ExpertMfmaJobs &J) {
    require(J.expert_count >= 1 && J.expert_count <= 2, "MFMA GEMM: one or two expert entries");
    require(J.expert_book != nullptr, "MFMA GEMM: expert codebook missing");
    require(J.max_active >= 1 && J.max_active <= kSlotCapacity, "MFMA GEMM: routed slots out of range");
    require(J.slot_info != nullptr || J.max_active == 1, "MFMA GEMM: routed slots need a slot table");
    const ExpertMfma &e = J.expert[0];
    require(e.columns >= 64 && e.rows >= 16, "MFMA GEMM: expert matrix below 16 x 64");
    for (uint32_t i = 0; i < J.expert_count; ++i) {
        ExpertMfma &x = J.expert[i];
        require(x.rows == e.rows && x.columns == e.columns, "MFMA GEMM: expert entries differ in shape");
        x.tile_rows = x.rows / kTile;
        x.tc_shift = log2_of(x.columns / kTile);
    }
    J.row_groups = ceil_div(e.rows / kTile, kExpertRT);
    J.position_groups = ceil_div(J.max_positions, 16u * kExpertNT);
    J.items = J.expert_count * J.max_active * J.position_groups * J.row_groups;  // upper bound
    const uint32_t cap = ctx->cu_count >= 16 ? ctx->cu_count / 16 * 16 : 16u;
    const uint32_t needed = 16u * ceil_div(ceil_div(J.items, kExpertThreads / kWave), 8);
    const uint32_t blocks = needed < cap ? needed : cap;
    const size_t lds = size_t(kSlotCapacity) * 16 + size_t(kSlotCapacity + 16) * 4 +
                       size_t(kPlaneRows16) * 16;
    auto kernel = k_expert_mfma<kExpertNT, kExpertRT, kExpertThreads>;
    static const bool ready = set_lds_limit(reinterpret_cast<const void *>(kernel), lds);
    (void)ready;
    launch(ctx, "expert_mfma", kernel, dim3(blocks), dim3(kExpertThreads), lds, J);
}

void launch_ne_mfma(adi_hip_context *ctx, NeMfmaJobs &J) {
    require(J.ne_count >= 1 && J.ne_count <= 2, "MFMA GEMM: one or two NE entries");
    require(J.ne_book != nullptr, "MFMA GEMM: NE codebook missing");
    const NeMfma &n = J.ne[0];
    require(n.columns >= 32 && n.rows >= 16, "MFMA GEMM: NE matrix below 16 x 32");
    for (uint32_t i = 0; i < J.ne_count; ++i) {
        NeMfma &x = J.ne[i];
        require(x.rows == n.rows && x.columns == n.columns && x.batch == n.batch,
                "MFMA GEMM: NE entries differ in shape");
        x.tile_rows = x.rows / kTile;
        x.tc_shift = log2_of(x.columns / kTile);
    }
    const uint32_t nt = mfma_position_tiles(n.batch);
    J.row_groups = ceil_div(n.rows / kTile, kRowTiles);
    J.position_groups = ceil_div(n.batch, 16u * nt);
    J.k_slices = ne_mfma_slices(n.rows, n.columns, n.batch);
    J.items = J.ne_count * J.position_groups * J.row_groups * J.k_slices;
    const dim3 grid(ceil_div(J.items, kMfmaWaves));
    switch (nt) {
    case 1: launch(ctx, "ne_mfma", k_ne_mfma<1>, grid, dim3(kMfmaThreads), 0, J); break;
    case 2: launch(ctx, "ne_mfma", k_ne_mfma<2>, grid, dim3(kMfmaThreads), 0, J); break;
    default: launch(ctx, "ne_mfma", k_ne_mfma<4>, grid, dim3(kMfmaThreads), 0, J);
    }
}

}  // namespace adi_hip
