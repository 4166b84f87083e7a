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
constexpr uint32_t kExpertThreads = 512;                 // expert GEMM: 2 waves per SIMD
constexpr uint32_t kExpertWaves = kExpertThreads / kWave;
constexpr uint32_t kRowTiles = 4;                         // tile rows per item
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

template <int NT>
struct ExpertStep {
    half8 bh[NT], bl[NT];
    uint32_t d0[kRowTiles], d1[kRowTiles];
    uint32_t gamma[kRowTiles];  // f16 bits
};

struct ExpertItem {
    const ExpertMfma *a;
    const uint32_t *words;      // the matrix's trellis as dwords
    const uint16_t *gamma_row;
    const uint16_t *xh, *xl;    // this plane's x_hat pairs
    uint32_t first, end, p0;    // slot positions and this item's first
    uint32_t tr0;
};

template <int NT>
__device__ __forceinline__ void expert_load(const ExpertItem &it, uint32_t kc, uint32_t lane,
                                            ExpertStep<NT> &s) {
    const ExpertMfma &a = *it.a;
    const uint32_t m = lane & 15u, kq = lane >> 4;
    const uint32_t half_columns = a.columns >> 1;
#pragma unroll
    for (int j = 0; j < NT; ++j) {
        const uint32_t p = it.p0 + 16u * j + m;
        const uint32_t pc = p < it.end ? p : it.p0;
        const size_t at = static_cast<size_t>(pc) * half_columns + kc * 32u + kq * 8u;
        s.bh[j] = load_half8(it.xh + at);
        s.bl[j] = load_half8(it.xl + at);
    }
    const uint32_t tile_columns = 1u << a.tc_shift;
    const uint32_t tc = kc * 4u + kq;
    const uint32_t dw = (24u * m) >> 5;
    const uint32_t dn = dw == 11u ? 0u : dw + 1u;  // row 15 wraps to word 0 (src/expert_trellis.hpp:79-80)
#pragma unroll
    for (uint32_t t = 0; t < kRowTiles; ++t) {
        const uint32_t tr = min(it.tr0 + t, a.tile_rows - 1u);
        const size_t tile = (static_cast<size_t>(tr) << a.tc_shift) + tc;
        s.d0[t] = __builtin_nontemporal_load(it.words + tile * 12u + dw);
        s.d1[t] = __builtin_nontemporal_load(it.words + tile * 12u + dn);
        s.gamma[t] = it.gamma_row[wave_slot(tr, tc, a.tile_rows, tile_columns)];
    }
}

template <int NT>
__device__ __forceinline__ void expert_compute(const ExpertItem &it, uint32_t half,
                                               const uint2 *plane, uint32_t lane,
                                               const ExpertStep<NT> &s, f32x4 (&acc)[kRowTiles][NT]) {
#pragma clang fp contract(off)
    const uint32_t m = lane & 15u, kq = lane >> 4;
    const uint32_t pos = ((24u * m) & 31u);  // bit of state 2m in the loaded words
    const uint32_t sign_mask = half == 0 ? 0x8000u : 0u;
    // zero the decoded values of masked lanes' invalid positions: B is clamped,
    // so only positions past the slot need zeroing
    half8 bh[NT], bl[NT];
#pragma unroll
    for (int j = 0; j < NT; ++j) {
        const bool ok = it.p0 + 16u * j + m < it.end;
        bh[j] = ok ? s.bh[j] : zero_half8();
        bl[j] = ok ? s.bl[j] : zero_half8();
    }
    (void)kq;
#pragma unroll
    for (uint32_t t = 0; t < kRowTiles; ++t) {
        const uint32_t p0 = state_product(window64(s.d0[t], s.d1[t], pos));
        const uint32_t p1 = state_product(window64(s.d0[t], s.d1[t], pos + 12u));
        uint2 e0 = plane[(p0 >> 1) & 0x3FFFu];
        uint2 e1 = plane[(p1 >> 1) & 0x3FFFu];
        e0.x ^= p0 & sign_mask;
        e1.x ^= p1 & sign_mask;
        const half8 v = __builtin_bit_cast(half8, u32x4{e0.x, e0.y, e1.x, e1.y});
        const _Float16 g = __builtin_bit_cast(_Float16, static_cast<uint16_t>(s.gamma[t]));
        const half8 gv = {g, g, g, g, g, g, g, g};
        const half8 hi = gv * v;
        const half8 lo = __builtin_elementwise_fma(gv, v, -hi);
#pragma unroll
        for (int j = 0; j < NT; ++j) {
            acc[t][j] = mfma(hi, bh[j], acc[t][j]);
        }
#pragma unroll
        for (int j = 0; j < NT; ++j) {
            acc[t][j] = mfma(hi, bl[j], acc[t][j]);
        }
#pragma unroll
        for (int j = 0; j < NT; ++j) {
            acc[t][j] = mfma(lo, bh[j], acc[t][j]);
        }
    }
}

// Block b serves codebook plane (b / 8) % 2 as worker ((b / 16) * 8 + b % 8)
// (the two blocks that walk the same tiles share an XCD). Each block counts
// the items of every routed slot (position groups x row groups) and scans the
// counts in LDS, so the waves walk only real items, evenly. Items are numbered
// (entry, slot, position group, row group), row group fastest, so the waves of
// a block share B fragments in L1.
template <int NT>
__global__ __launch_bounds__(kExpertThreads) void k_expert_mfma(ExpertMfmaJobs J) {
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
        constexpr uint32_t kPer = kPlaneRows16 / kExpertThreads;  // 16
        uint4 v[kPer];
#pragma unroll
        for (uint32_t u = 0; u < kPer; ++u) {
            v[u] = src[u * kExpertThreads + threadIdx.x];
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
            plane_lds[u * kExpertThreads + threadIdx.x] = v[u];
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
        ExpertItem it;
        it.first = __builtin_amdgcn_readfirstlane(info.y);
        it.end = __builtin_amdgcn_readfirstlane(info.z);
        it.p0 = it.first + pg * 16u * NT;
        const uint32_t mat = __builtin_amdgcn_readfirstlane(info.x);
        it.a = &J.expert[which];
        const ExpertMfma &a = *it.a;
        it.words = reinterpret_cast<const uint32_t *>(a.trellis + mat * a.trellis_stride);
        it.gamma_row = a.gamma + mat * a.gamma_stride;
        const size_t plane_stride = static_cast<size_t>(a.positions) * (a.columns >> 1);
        it.xh = a.x_hi + half * plane_stride;
        it.xl = a.x_lo + half * plane_stride;
        it.tr0 = rg * kRowTiles;
        f32x4 acc[kRowTiles][NT];
#pragma unroll
        for (uint32_t t = 0; t < kRowTiles; ++t) {
#pragma unroll
            for (int j = 0; j < NT; ++j) {
                acc[t][j] = f32x4{0.f, 0.f, 0.f, 0.f};
            }
        }
        const uint32_t steps = (1u << a.tc_shift) / 4u;  // a power of two
        ExpertStep<NT> s0, s1;
        expert_load<NT>(it, 0, lane, s0);
        if (steps == 1) {
            expert_compute<NT>(it, half, plane, lane, s0, acc);
        } else {
            // no branch inside the body, so the compiler's wait counts see
            // that only the other stage's loads are outstanding; the last
            // iteration reloads the final step (in bounds, unused)
            for (uint32_t kc = 0; kc < steps; kc += 2) {
                expert_load<NT>(it, kc + 1, lane, s1);
                expert_compute<NT>(it, half, plane, lane, s0, acc);
                expert_load<NT>(it, min(kc + 2, steps - 1), lane, s0);
                expert_compute<NT>(it, half, plane, lane, s1, acc);
            }
        }
        const uint32_t m = lane & 15u, kq = lane >> 4;
        float *z = a.z + half * a.z_split_stride;
#pragma unroll
        for (uint32_t t = 0; t < kRowTiles; ++t) {
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
    // 32 positions per item: two waves per SIMD fit in the registers
    J.row_groups = ceil_div(e.rows / kTile, kRowTiles);
    J.position_groups = ceil_div(J.max_positions, 32u);
    J.items = J.expert_count * J.max_active * J.position_groups * J.row_groups;  // upper bound
    const uint32_t cap = ctx->cu_count >= 16 ? ctx->cu_count / 16 * 16 : 16u;
    const uint32_t needed = 16u * ceil_div(ceil_div(J.items, kExpertWaves), 8);
    const uint32_t blocks = needed < cap ? needed : cap;
    const size_t lds = size_t(kSlotCapacity) * 16 + size_t(kSlotCapacity + 16) * 4 +
                       size_t(kPlaneRows16) * 16;
    static const bool ready = set_lds_limit(reinterpret_cast<const void *>(&k_expert_mfma<2>), lds);
    (void)ready;
    launch(ctx, "expert_mfma", k_expert_mfma<2>, dim3(blocks), dim3(kExpertThreads), lds, J);
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
