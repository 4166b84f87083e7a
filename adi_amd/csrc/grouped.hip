// grouped.hip -- MFMA grouped GEMMs for prefill microbatches
// (src/kernels.cpp:491-593, 703-800 with the batch kernels of
// src/expert_batch_impl.hpp and src/ne_batch_impl.hpp): the codes are decoded
// straight into the A operand of v_mfma_f32_32x32x16_f16, x_hat is the B
// operand as f16 hi/lo pairs staged once per block in LDS, accumulation is
// fp32.
//
// Expert codec. The K axis is laid out as the eight columns a codebook plane
// covers in each tile (XhatOut planes 2), so a lane's eight K values are the
// two half-states of one tile row: two gathers from the block's LDS plane.
// The wave gamma of a tile is folded into A in f16: hi = f16(gamma * V),
// lo = f16(gamma * V - hi) (one packed f16 multiply and one packed f16 fma;
// gamma and V are f16, so the product has at most 22 significant bits and
// hi + lo holds it). Three MFMA passes, hi*hi + hi*lo + lo*hi, keep the error
// near fp32 rounding.
//
// NE codec. The 4 KiB signed table gives V exactly in f16 (Wscale is applied
// to the fp32 row sums); two passes, V*hi + V*lo.
#include "grouped.hpp"

#include <type_traits>

namespace adi_hip {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// expert GEMM shape: 32 positions per item, tile rows kExpertRT per wave,
// 512 * kExpertGroups threads per block (one block per CU), MFMA passes per
// product (hi*hi + hi*lo + lo*hi)
constexpr int kExpertRT = 4;
constexpr int kExpertCB = 2;      // blocks of 32 positions per item (the later one may be empty)
constexpr int kExpertGroups = 1;  // wave groups of eight per block, each on its own item
constexpr int kExpertPasses = 3;
constexpr uint32_t kPlaneRows16 = kExpertRows * 8 / 16;   // 16-byte rows of a plane
constexpr uint32_t kSlotCapacity = 1024;

// The 16-bit window at bit r (r <= 48) of the 64-bit string of u16 words
// w0 w1 w2 w3, each read most-significant bit first, where d0 = w0 | w1 << 16
// and d1 = w2 | w3 << 16 (src/expert_trellis.hpp:81-105).
__device__ __forceinline__ uint32_t window64(uint32_t d0, uint32_t d1, uint32_t r) {
    const uint64_t bits = (static_cast<uint64_t>(d0 & 0xFFFFu) << 48) |
                          (static_cast<uint64_t>(d0 >> 16) << 32) |
                          (static_cast<uint64_t>(d1 & 0xFFFFu) << 16) | (d1 >> 16);
    return static_cast<uint32_t>(bits >> (48u - r)) & 0xFFFFu;
}

// w (w + 1) mod 2^16 in bits 0..15 for any 32-bit w whose low 16 bits are
// the state: v_mad_u32_u24 reads 24 bits of each factor, and the bits above
// bit 15 only add multiples of 2^16 (the compiler would otherwise pick the
// quarter-rate v_mad_u64_u32 for the unmasked product).
__device__ __forceinline__ uint32_t state_hash_low16(uint32_t w) {
    uint32_t p;
    asm("v_mad_u32_u24 %0, %1, %1, %1" : "=v"(p) : "v"(w));
    return p;
}

// ---- expert ---------------------------------------------------------------
//
// v_mfma_f32_32x32x16_f16 (on the box 1.6x the f16 rate of 16x16x32): lane l
// holds A[l % 32][8 (l / 32) .. + 7], B[8 (l / 32) .. + 7][l % 32], and D
// column l % 32, rows (r % 4) + 8 (r / 4) + 4 (l / 32) of register r.
//
// An item is one routed slot's 32 positions times 32 tile rows of one entry.
// A block runs kExpertGroups wave groups of eight, each on its own item; wave
// w of a group takes tile rows 4w .. 4w + 3 of it as two 32-row blocks. Lane
// l holds row l % 16 of tile row 2 rb + (l % 32) / 16 of its block rb, and of
// K pair c at K step kc the tile column 4 kc + 2 c + l / 32: its eight K
// values (in the codebook-plane order of XhatOut planes 2) are the two
// half-states of that row, two gathers from the LDS plane. A group loads each
// K step's x_hat hi and lo of its positions once into its LDS ring that its
// eight waves read; the block takes one barrier per K step (all items of a
// launch have the same K). Each wave loads its own trellis words, four K
// steps ahead.

constexpr uint32_t kBlockTileRows = kExpertRT * 8;  // tile rows of an item (a wave group's share)
constexpr uint32_t kBRowPitch = 80;  // bytes per B row in LDS: 64 of data, 16 of pad (no bank conflicts)
constexpr uint32_t kGammaRow = kMaxTileColumns + kBlockTileRows;  // halves per gamma row
constexpr int kFragments = 4;  // A fragments per K step: (row block, K pair)

typedef float f32x16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ f32x16 mfma32(half8 a, half8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// A buffer resource over `bytes` bytes at `base`: loads past the end return 0.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_over(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, bytes, 0x00020000);
}

// The trellis words of the lane's four tiles (fragment f = 2 rb + c) at one K
// step: its two stream dwords (row 15: dwords 10 and 11).
struct ExpertWords {
    uint2 w[kFragments];
};

// Everything about a wave's share of an item that does not change along K:
// per-lane byte offsets (a K step advances the scalar offset only), the
// lane's window shifts and its gamma row in LDS.
struct ExpertWave {
    __amdgpu_buffer_rsrc_t words;
    uint32_t woff[kFragments];  // the lane's stream dword pair of fragment f at K step 0
    const uint2 *gammas;        // gamma row tsub + kh of the item, at the wave's first tile row
    uint32_t sh0, sh1;          // shifts of the lane's two windows in the 64-bit string
    bool row15;                 // the lane holds tile row 15, whose last window wraps
};

__device__ __forceinline__ void expert_words(const ExpertWave &wv, uint32_t kc, ExpertWords &s) {
    const uint32_t kw = kc * 192u;  // 4 tiles of 48 bytes per K step
#pragma unroll
    for (int f = 0; f < kFragments; ++f) {
        s.w[f] = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(wv.words, wv.woff[f], kw, 0));
    }
}

// The lane's A fragments at one K step: hi = f16(gamma * V) and
// lo = f16(gamma * V - hi).
struct ExpertA {
    half8 hi[kFragments], lo[kFragments];
};

// Decodes the lane's A fragments at K step kc (lo only when PASSES is 3).
template <int PASSES>
__device__ __forceinline__ void expert_decode(const ExpertWave &wv, uint32_t kc, uint32_t sign_mask,
                                              const uint2 *plane, const ExpertWords &s, ExpertA &a) {
#pragma clang fp contract(off)
    // gammas of the lane's tiles: fragment (rb, c) sits 2 rb + 2 c anti-diagonals
    // past the lane's first, so offsets 0, 2, 2, 4 of the lane's gamma row
    const uint2 g03 = wv.gammas[kc];
    const uint2 g47 = wv.gammas[kc + 1];
    const uint32_t gbits[kFragments] = {g03.x & 0xFFFFu, g03.y & 0xFFFFu, g03.y & 0xFFFFu, g47.x & 0xFFFFu};
#pragma unroll
    for (int f = 0; f < kFragments; ++f) {
        // row 15's second dword is dword 0 of its tile, which lane 0 of the
        // same 16-lane row (the same tile) loaded first (row_ror:15 reads
        // lane (i + 1) mod 16)
        const uint32_t wrap = __builtin_amdgcn_update_dpp(0u, s.w[f].x, 0x12F, 0xF, 0xF, false);
        const uint32_t d0 = wv.row15 ? s.w[f].y : s.w[f].x;
        const uint32_t d1 = wv.row15 ? wrap : s.w[f].y;
        // the lane's four stream words, most significant bit first
        const uint64_t bits = (static_cast<uint64_t>(__builtin_amdgcn_alignbit(d0, d0, 16)) << 32) |
                              __builtin_amdgcn_alignbit(d1, d1, 16);
        const uint32_t p0 = state_hash_low16(static_cast<uint32_t>(bits >> wv.sh0));
        const uint32_t p1 = state_hash_low16(static_cast<uint32_t>(bits >> wv.sh1));
        uint2 e0 = plane[(p0 >> 1) & 0x3FFFu];
        uint2 e1 = plane[(p1 >> 1) & 0x3FFFu];
        e0.x ^= p0 & sign_mask;
        e1.x ^= p1 & sign_mask;
        const half8 v = __builtin_bit_cast(half8, u32x4{e0.x, e0.y, e1.x, e1.y});
        const _Float16 g = __builtin_bit_cast(_Float16, static_cast<uint16_t>(gbits[f]));
        const half8 gv = {g, g, g, g, g, g, g, g};
        a.hi[f] = gv * v;
        if constexpr (PASSES == 3) {
            a.lo[f] = __builtin_elementwise_fma(gv, v, -a.hi[f]);
        }
    }
}

// acc[rb][cb] += hi * bh + hi * bl + lo * bh over the two K pairs, for the
// item's first LIVE of its CB blocks of 32 positions (lo only when PASSES is
// 3). Positions past the slot in a live block carry another slot's x_hat:
// their output columns are computed and never stored.
template <int CB, int LIVE, int PASSES>
__device__ __forceinline__ void expert_multiply(const ExpertA &a, const half8 (&bh)[CB][2],
                                                const half8 (&bl)[CB][2], f32x16 (&acc)[2][CB]) {
    static_assert(LIVE >= 1 && LIVE <= CB, "live blocks of an item");
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
#pragma unroll
        for (int cb = 0; cb < LIVE; ++cb) {
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                acc[rb][cb] = mfma32(a.hi[2 * rb + c], bh[cb][c], acc[rb][cb]);
            }
        }
    }
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
#pragma unroll
        for (int cb = 0; cb < LIVE; ++cb) {
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                acc[rb][cb] = mfma32(a.hi[2 * rb + c], bl[cb][c], acc[rb][cb]);
            }
        }
    }
    if constexpr (PASSES == 3) {
#pragma unroll
        for (int rb = 0; rb < 2; ++rb) {
#pragma unroll
            for (int cb = 0; cb < LIVE; ++cb) {
#pragma unroll
                for (int c = 0; c < 2; ++c) {
                    acc[rb][cb] = mfma32(a.lo[2 * rb + c], bh[cb][c], acc[rb][cb]);
                }
            }
        }
    }
}

// Block b serves codebook plane (b / 8) % 2 as worker ((b / 16) * 8 + b % 8)
// (the two blocks that walk the same tiles share an XCD). Each block counts
// the items of every routed slot (position groups x row quarters) and scans
// the counts in LDS, so the blocks walk only real items, evenly. Items are
// numbered (entry, slot, position group, row quarter); a block takes them
// kExpertGroups at a time, and a group past the last item runs a copy of the
// last one without storing it.
template <int CB, int GROUPS, int PASSES>
__global__ __launch_bounds__(512 * GROUPS) void k_expert_mfma(ExpertMfmaJobs J) {
    static_assert(CB == 1 || CB == 2, "items of 32 or 64 positions");
    constexpr uint32_t kExpertThreads = 512 * GROUPS;
    constexpr uint32_t kExpertGroups = GROUPS;
    constexpr uint32_t kPositions = 32 * CB;              // per item
    // a thread's share of a K step's B rows: 8 bytes (32 positions) or 16 (64)
    using BChunk = std::conditional_t<CB == 1, uint2, uint4>;
    constexpr uint32_t kThreadsPerRow = CB == 1 ? 8u : 4u;
    constexpr uint32_t kChunkBytes = 64u / kThreadsPerRow;
    constexpr uint32_t kWaves = kExpertThreads / kWave;
    constexpr uint32_t kGroupThreads = 512;
    constexpr uint32_t kBRows = 2u * kPositions;          // (hi/lo, position) rows of B
    constexpr uint32_t kBSlot = kBRows * kBRowPitch;      // bytes per K step in the ring
    constexpr int kDepth = 4;                             // K steps of loads in flight
    // static LDS with the plane first: its address is a compile-time
    // constant, so a gather's address is the masked row offset alone
    __shared__ uint4 plane_lds[kPlaneRows16];
    __shared__ uint32_t starts[kSlotCapacity + 1];
    __shared__ uint32_t wave_sums[kWaves];
    // gamma rows of an item: row q entry i = gamma of the tile at
    // anti-diagonal tr_block + i + q; lane (w, tsub, kh) reads its tiles'
    // gammas at K step kc from row tsub + kh at entries 4w + 4kc .. + 7
    __shared__ uint2 gamma_rows[kExpertGroups][4][kGammaRow / 4];
    __shared__ uint4 b_ring[kExpertGroups][2][kBSlot / 16];
    const uint32_t b = blockIdx.x;
    const uint32_t half = (b >> 3) & 1u;
    const uint32_t worker = ((b >> 4) << 3) | (b & 7u);
    const uint32_t workers = gridDim.x >> 1;
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t group = wave >> 3, gwave = wave & 7u;
    const uint32_t gthread = threadIdx.x & (kGroupThreads - 1u);
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
        const uint32_t quarters = J.row_groups;
        uint32_t count[2];
#pragma unroll
        for (uint32_t k = 0; k < 2; ++k) {
            const uint32_t s = 2u * threadIdx.x + k;
            uint4 info = make_uint4(0u, 0u, 0u, 0u);
            if (s < J.max_active) {
                info = J.slot_info != nullptr ? J.slot_info[s]
                                              : make_uint4(0u, 0u, s == 0 ? J.max_positions : 0u, 0u);
            }
            count[k] = info.z > info.y ? (info.z - info.y + kPositions - 1u) / kPositions * quarters : 0u;
        }
        // block-wide exclusive scan of the counts (slot order)
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
    const uint2 *plane = reinterpret_cast<const uint2 *>(plane_lds);
    const uint32_t per_entry = starts[kSlotCapacity];
    const uint32_t total = per_entry * J.expert_count;
    const uint32_t m = lane & 31u, kh = lane >> 5;   // MFMA row / column and K half
    const uint32_t trow = m & 15u, tsub = m >> 4;    // row within the tile, tile row within the block
    const uint32_t sign_mask = half == 0 ? 0x8000u : 0u;
    // the thread's share of its group's B loads: one chunk of one B row (B
    // rows are (hi/lo, position); wave w of the group loads rows
    // (64 / kThreadsPerRow) w .., so the hi/lo plane is wave-uniform: derived
    // from `gwave`, the buffer resource stays scalar)
    const uint32_t b_row = gthread / kThreadsPerRow, b_chunk = gthread % kThreadsPerRow;
    const uint32_t b_lo = gwave >> 2, b_n = b_row & (kPositions - 1u);
    char *ring = reinterpret_cast<char *>(b_ring[group]);
    const uint32_t b_store = b_row * kBRowPitch + b_chunk * kChunkBytes;
    auto load_b = [](__amdgpu_buffer_rsrc_t src, uint32_t off, uint32_t soff) {
        if constexpr (CB == 1) {
            return __builtin_bit_cast(BChunk, __builtin_amdgcn_raw_buffer_load_b64(src, off, soff, 0));
        } else {
            return __builtin_bit_cast(BChunk, __builtin_amdgcn_raw_buffer_load_b128(src, off, soff, 0));
        }
    };
    const uint32_t rounds = (total + kExpertGroups - 1u) / kExpertGroups;
    for (uint32_t round = worker; round < rounds; round += workers) {
        const uint32_t item_any = round * kExpertGroups + group;
        const bool live = item_any < total;
        const uint32_t item = live ? item_any : total - 1u;
        const uint32_t which = item / per_entry;
        const uint32_t local = item - which * per_entry;
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
        const uint32_t rq = within % J.row_groups;
        const uint32_t pg = within / J.row_groups;
        // the slot is uniform: its entry comes through the scalar cache
        const uint4 info = J.slot_info != nullptr ? J.slot_info[slot]
                                                  : make_uint4(0u, 0u, J.max_positions, 0u);
        const uint32_t first = __builtin_amdgcn_readfirstlane(info.y);
        const uint32_t mat = __builtin_amdgcn_readfirstlane(info.x);
        const uint32_t end = __builtin_amdgcn_readfirstlane(info.z);
        const ExpertMfma &a = J.expert[which];
        const uint32_t p0 = first + pg * kPositions;
        const uint32_t tr_block = rq * kBlockTileRows;
        const uint32_t tr0 = tr_block + gwave * kExpertRT;
        const uint32_t half_columns = a.columns >> 1;
        const uint32_t tile_columns = 1u << a.tc_shift;
        const uint32_t steps = tile_columns / 4u;  // a power of two
        const uint32_t last = steps - 1u;
        // this thread's B row: position p0 + b_n (clamped to a real row past
        // the slot), hi or lo plane
        const size_t plane_elems = static_cast<size_t>(a.positions) * half_columns;
        const uint32_t x_bytes = static_cast<uint32_t>(plane_elems * 2u);
        const __amdgpu_buffer_rsrc_t xsrc =
            buffer_over((b_lo ? a.x_lo : a.x_hi) + half * plane_elems, x_bytes);
        const uint32_t bp = p0 + b_n;
        const uint32_t b_off = ((bp < end ? bp : p0) * half_columns + b_chunk * (kChunkBytes / 2u)) * 2u;
        ExpertWave wv;
        const uint32_t tiles = a.tile_rows << a.tc_shift;
        wv.words = buffer_over(a.trellis + mat * a.trellis_stride, tiles * 48u);
        // the lane's states 2 trow, 2 trow + 1 start in dword dw = 24 trow / 32;
        // row 15's second window wraps to dword 0 of its tile
        // (src/expert_trellis.hpp:79-80), so that lane loads dwords 10 and 11
        // and takes dword 0 from lane 0 of its 16-lane row
        const uint32_t dw = (24u * trow) >> 5;
        wv.row15 = trow == 15u;
        const uint32_t dpair = wv.row15 ? 10u : dw;
#pragma unroll
        for (int f = 0; f < kFragments; ++f) {
            const uint32_t rb = f >> 1, c = f & 1;
            const uint32_t tr = min(tr0 + 2u * rb + tsub, a.tile_rows - 1u);
            const uint32_t tile = (tr << a.tc_shift) + 2u * c + kh;
            wv.woff[f] = (tile * 12u + dpair) * 4u;
        }
        wv.gammas = gamma_rows[group][tsub + kh] + gwave;  // entry 4 * gwave
        const uint32_t pos = (24u * trow) & 31u;  // bit of state 2 trow in dword dw
        wv.sh0 = 48u - pos;
        wv.sh1 = 36u - pos;

        // the previous item's readers of the gamma rows and the ring are done
        __syncthreads();
        {
            // gamma of the tile at anti-diagonal d = tr_block + e sits in wave
            // slot R_t + C_t - 1 - d, one less past the main anti-diagonal
            // (src/codec_cache.cpp:117-147); slots past the matrix read 0 and
            // belong to tiles that are never stored
            const __amdgpu_buffer_rsrc_t gbuf =
                buffer_over(a.gamma + mat * a.gamma_stride, (a.tile_rows + tile_columns) * 2u);
            const uint32_t top = a.tile_rows + tile_columns - 1u;
            uint16_t *rows = reinterpret_cast<uint16_t *>(gamma_rows[group]);
            const uint32_t e = gthread;  // tile_columns + 35 <= 512
            const uint32_t d = tr_block + e;
            const uint32_t gslot = top - d - (d >= tile_columns ? 1u : 0u);
            const uint16_t g = __builtin_amdgcn_raw_buffer_load_b16(gbuf, gslot * 2u, 0, 0);
            if (e < tile_columns + kBlockTileRows + 3u) {
#pragma unroll
                for (uint32_t q = 0; q < 4u; ++q) {
                    const uint32_t i = e - q;  // wraps past zero: then out of range
                    if (i < kGammaRow) {
                        rows[q * kGammaRow + i] = g;
                    }
                }
            }
        }
        f32x16 acc[2][CB];
#pragma unroll
        for (int rb = 0; rb < 2; ++rb) {
#pragma unroll
            for (int cb = 0; cb < CB; ++cb) {
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    acc[rb][cb][r] = 0.0f;
                }
            }
        }
        // B of K step kc, as the MFMA operands of position block cb, K pair c
        // (the item's first LIVE blocks)
        auto read_b = [&]<int LIVE>(uint32_t ring_slot, half8 (&bh)[CB][2], half8 (&bl)[CB][2]) {
            const char *base = ring + ring_slot * kBSlot + m * kBRowPitch + kh * 16u;
#pragma unroll
            for (int cb = 0; cb < LIVE; ++cb) {
#pragma unroll
                for (int c = 0; c < 2; ++c) {
                    bh[cb][c] = *reinterpret_cast<const half8 *>(base + cb * 32u * kBRowPitch + c * 32u);
                    bl[cb][c] = *reinterpret_cast<const half8 *>(base + (kPositions + cb * 32u) * kBRowPitch + c * 32u);
                }
            }
        };
        // the K loop for an item whose first LIVE blocks of 32 positions hold
        // positions of its slot: each K step's A fragments are decoded once
        // and multiplied with every live block (the slot's later blocks skip
        // their MFMAs, not the decode)
        auto k_loop = [&]<int LIVE>() {
            if (steps % kDepth != 0) {
                // short K (under 4 steps): one step at a time
                for (uint32_t kc = 0; kc < steps; ++kc) {
                    const BChunk bv = load_b(xsrc, b_off, kc * 64u);
                    ExpertWords ws;
                    expert_words(wv, kc, ws);
                    *reinterpret_cast<BChunk *>(ring + b_store) = bv;
                    __syncthreads();
                    half8 bh[CB][2], bl[CB][2];
                    read_b.template operator()<LIVE>(0, bh, bl);
                    ExpertA fa;
                    expert_decode<PASSES>(wv, kc, sign_mask, plane, ws, fa);
                    expert_multiply<CB, LIVE, PASSES>(fa, bh, bl, acc);
                    __syncthreads();
                }
            } else {
                // B of step s waits in bv[s % 4] (registers) until step s - 1
                // writes it to ring slot s % 2; the words of step s wait in
                // ws[s % 4]. Loads past the last step reload it (in bounds,
                // unused), so the loop body has no branch.
                BChunk bv[kDepth];
                ExpertWords ws[kDepth];
#pragma unroll
                for (int u = 0; u < kDepth; ++u) {
                    __builtin_amdgcn_sched_barrier(0);
                    bv[u] = load_b(xsrc, b_off, u * 64u);
                    if (u < kDepth - 1) {
                        expert_words(wv, u, ws[u]);
                    }
                }
                __builtin_amdgcn_sched_barrier(0);
                *reinterpret_cast<BChunk *>(ring + b_store) = bv[0];
                bv[0] = load_b(xsrc, b_off, min(static_cast<uint32_t>(kDepth), last) * 64u);
                __syncthreads();
                for (uint32_t kc = 0; kc < steps; kc += kDepth) {
#pragma unroll
                    for (int u = 0; u < kDepth; ++u) {
                        const uint32_t step = kc + u;
                        __builtin_amdgcn_sched_barrier(0);
                        // hand B of the next step to the ring and refill its registers
                        *reinterpret_cast<BChunk *>(ring + ((u + 1) & 1) * kBSlot + b_store) = bv[(u + 1) % kDepth];
                        bv[(u + 1) % kDepth] = load_b(xsrc, b_off, min(step + 1u + kDepth, last) * 64u);
                        expert_words(wv, min(step + kDepth - 1u, last), ws[(u + kDepth - 1) % kDepth]);
                        __builtin_amdgcn_sched_barrier(0);
                        half8 bh[CB][2], bl[CB][2];
                        read_b.template operator()<LIVE>(u & 1, bh, bl);
                        ExpertA fa;
                        expert_decode<PASSES>(wv, step, sign_mask, plane, ws[u], fa);
                        expert_multiply<CB, LIVE, PASSES>(fa, bh, bl, acc);
                        __syncthreads();
                    }
                }
            }
        };
        if constexpr (CB == 2) {
            if (p0 + 32u < end) {
                k_loop.template operator()<2>();
            } else {
                k_loop.template operator()<1>();
            }
        } else {
            k_loop.template operator()<1>();
        }
        // D register r of lane l: position 32 cb + l % 32, block row
        // (r % 4) + 8 (r / 4) + 4 kh
        float *z = a.z + half * a.z_split_stride;
#pragma unroll
        for (int cb = 0; cb < CB; ++cb) {
            const uint32_t p = p0 + 32u * cb + m;
            if (live && p < end) {
#pragma unroll
                for (int rb = 0; rb < 2; ++rb) {
#pragma unroll
                    for (int g = 0; g < 4; ++g) {
                        const uint32_t row = (tr0 + 2u * rb) * kTile + 8u * g + 4u * kh;
                        if (row < a.rows) {
                            *reinterpret_cast<f32x4 *>(z + static_cast<size_t>(p) * a.rows + row) =
                                f32x4{acc[rb][cb][4 * g], acc[rb][cb][4 * g + 1], acc[rb][cb][4 * g + 2],
                                      acc[rb][cb][4 * g + 3]};
                        }
                    }
                }
            }
        }
    }
}

// ---- NE -------------------------------------------------------------------
//
// Also on v_mfma_f32_32x32x16_f16. A block of eight waves takes one item: 32
// positions x 16 tile rows (256 rows) of one NE entry over one K slice; wave w
// takes tile rows 2w, 2w + 1 as one 32-row block. Lane l holds row l % 16 of
// tile row 2w + (l % 32) / 16 and, of K pair c at K step kc, columns
// 8 (l / 32) .. + 7 of tile column 2 kc + c: NE states 8 (l % 16) +
// 4 (l / 32) + 0..3, four lookups of the signed table (two f16 each). The
// block loads each K step's x_hat hi and lo of its 32 positions once into an
// LDS ring (one barrier per K step); each wave loads its trellis words four K
// steps ahead.

constexpr uint32_t kNeThreads = 512;
constexpr uint32_t kNeWaves = kNeThreads / kWave;
constexpr uint32_t kNeItemTileRows = 2 * kNeWaves;   // 256 rows per item
constexpr uint32_t kNeBSlot = 64 * kBRowPitch;      // (hi/lo, position) rows of one K step

// The lane's trellis dwords of its two fragments (K pair c) at one K step.
struct NeWords {
    uint32_t d0[2], d1[2];
};

__global__ __launch_bounds__(kNeThreads) void k_ne_mfma(NeMfmaJobs J) {
    __shared__ uint32_t table[1024];
    __shared__ uint4 b_ring[2][kNeBSlot / 16];
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // item (row group, K slice, position group, entry), fastest first
    uint32_t rest = blockIdx.x;
    const uint32_t rg = rest % J.row_groups;
    rest /= J.row_groups;
    const uint32_t ks = rest % J.k_slices;
    rest /= J.k_slices;
    const uint32_t pg = rest % J.position_groups;
    const uint32_t which = rest / J.position_groups;
    const NeMfma &a = J.ne[which];
    const uint32_t steps = (a.columns >> 5) / J.k_slices;  // K steps of 32 columns, a power of two
    const uint32_t k0 = ks * steps;
    const uint32_t last = steps - 1u;
    const uint32_t p0 = pg * 32u;
    // the table: eight bytes per thread, stored once the first loads are out
    const uint2 tv = reinterpret_cast<const uint2 *>(J.ne_book)[threadIdx.x];
    // B staging: thread t copies 8 bytes of B row t / 8 (rows 0..31 hi, 32..63
    // lo, so the plane is wave-uniform); positions past the batch repeat p0
    const uint32_t b_row = threadIdx.x >> 3, b_chunk = threadIdx.x & 7u;
    const uint32_t bp = p0 + (b_row & 31u);
    const uint32_t b_pos = bp < a.batch ? bp : p0;
    const __amdgpu_buffer_rsrc_t xsrc =
        buffer_over(wave >= 4u ? a.x_lo : a.x_hi, a.batch * a.columns * 2u);
    const uint32_t b_off = (b_pos * a.columns + b_chunk * 4u) * 2u + k0 * 64u;
    char *ring = reinterpret_cast<char *>(b_ring);
    const uint32_t b_store = b_row * kBRowPitch + b_chunk * 8u;
    auto load_b = [&](uint32_t kc) {
        return __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(xsrc, b_off, kc * 64u, 0));
    };
    // the lane's trellis words: row trow of tile row tr, dwords dw and dw + 1
    // (row 15's second wraps to dword 0, src/ne_trellis.hpp:196-200)
    const uint32_t m = lane & 31u, kh = lane >> 5;
    const uint32_t trow = m & 15u;
    const uint32_t tr_block = rg * kNeItemTileRows + 2u * wave;
    const uint32_t tr = min(tr_block + (m >> 4), a.tile_rows - 1u);
    const uint32_t dw = 2u * trow + kh, dn = dw == 31u ? 0u : dw + 1u;
    const __amdgpu_buffer_rsrc_t wsrc = buffer_over(a.trellis, (a.tile_rows << a.tc_shift) * 128u);
    const uint32_t w0 = ((tr << a.tc_shift) * 32u + dw) * 4u;
    const uint32_t w1 = ((tr << a.tc_shift) * 32u + dn) * 4u;
    auto load_words = [&](uint32_t kc, NeWords &w) {
#pragma unroll
        for (uint32_t c = 0; c < 2; ++c) {
            const uint32_t soff = (2u * (k0 + kc) + c) * 128u;  // tile column 2 kc + c
            w.d0[c] = __builtin_amdgcn_raw_buffer_load_b32(wsrc, w0, soff, 0);
            w.d1[c] = __builtin_amdgcn_raw_buffer_load_b32(wsrc, w1, soff, 0);
        }
    };
    f32x16 acc;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        acc[r] = 0.0f;
    }
    // one K step: the two A fragments from the table, B from ring slot `slot`
    auto multiply = [&](uint32_t slot, const NeWords &w) {
        const char *base = ring + slot * kNeBSlot + m * kBRowPitch + kh * 16u;
#pragma unroll
        for (uint32_t c = 0; c < 2; ++c) {
            const half8 bh = *reinterpret_cast<const half8 *>(base + c * 32u);
            const half8 bl = *reinterpret_cast<const half8 *>(base + 32u * kBRowPitch + c * 32u);
            uint32_t v[4];
#pragma unroll
            for (uint32_t q = 0; q < 4; ++q) {
                // state hash in v_mad_u32_u24: the window's bits above bit 15
                // only add multiples of 2^16
                v[q] = table[(state_hash_low16(window64(w.d0[c], w.d1[c], 8u * q)) >> 6) & 0x3FFu];
            }
            const half8 av = __builtin_bit_cast(half8, u32x4{v[0], v[1], v[2], v[3]});
            acc = mfma32(av, bh, acc);
            acc = mfma32(av, bl, acc);
        }
    };
    constexpr uint32_t kDepth = 4;
    if (steps % kDepth != 0) {
        // short K (under 4 steps): one step at a time
        table[threadIdx.x * 2u] = tv.x;
        table[threadIdx.x * 2u + 1u] = tv.y;
        for (uint32_t kc = 0; kc < steps; ++kc) {
            const uint2 bv = load_b(kc);
            NeWords w;
            load_words(kc, w);
            *reinterpret_cast<uint2 *>(ring + b_store) = bv;
            __syncthreads();
            multiply(0, w);
            __syncthreads();
        }
    } else {
        // B of step s waits in bv[s % 4] until step s - 1 writes it to ring
        // slot s % 2; the words of step s wait in ws[s % 4]. Loads past the
        // last step reload it (in bounds, unused).
        uint2 bv[kDepth];
        NeWords ws[kDepth];
#pragma unroll
        for (uint32_t u = 0; u < kDepth; ++u) {
            bv[u] = load_b(u);
            if (u < kDepth - 1) {
                load_words(u, ws[u]);
            }
        }
        table[threadIdx.x * 2u] = tv.x;
        table[threadIdx.x * 2u + 1u] = tv.y;
        *reinterpret_cast<uint2 *>(ring + b_store) = bv[0];
        bv[0] = load_b(min(kDepth, last));
        __syncthreads();
        for (uint32_t kc = 0; kc < steps; kc += kDepth) {
#pragma unroll
            for (uint32_t u = 0; u < kDepth; ++u) {
                const uint32_t step = kc + u;
                __builtin_amdgcn_sched_barrier(0);
                *reinterpret_cast<uint2 *>(ring + ((u + 1) & 1) * kNeBSlot + b_store) = bv[(u + 1) % kDepth];
                bv[(u + 1) % kDepth] = load_b(min(step + 1u + kDepth, last));
                load_words(min(step + kDepth - 1u, last), ws[(u + kDepth - 1) % kDepth]);
                __builtin_amdgcn_sched_barrier(0);
                multiply(u & 1, ws[u]);
                __syncthreads();
            }
        }
    }
    // D register r of lane l: position l % 32, row (r % 4) + 8 (r / 4) + 4 kh
    // of the wave's 32-row block
    const uint32_t p = p0 + m;
    if (p < a.batch) {
        float *z = a.z + static_cast<size_t>(ks) * a.batch * a.rows + static_cast<size_t>(p) * a.rows;
#pragma unroll
        for (uint32_t g = 0; g < 4; ++g) {
            const uint32_t row = tr_block * kTile + 8u * g + 4u * kh;
            if (row < a.rows) {
                *reinterpret_cast<f32x4 *>(z + row) =
                    f32x4{acc[4 * g], acc[4 * g + 1], acc[4 * g + 2], acc[4 * g + 3]} * a.weight_scale;
            }
        }
    }
}

}  // namespace

uint32_t ne_mfma_slices(uint32_t rows, uint32_t columns, uint32_t batch) {
    const uint32_t items = ceil_div(rows, kNeItemTileRows * kTile) * ceil_div(batch, 32u);
    uint32_t slices = 1;
    // about one block per CU, each with at least four K steps of 32 columns
    while (items * slices < 256u && columns / 32u / (slices * 2u) >= 4u) {
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
    require(expert_mfma_supports(e.rows, e.columns), "MFMA GEMM: expert matrix shape out of range");
    for (uint32_t i = 0; i < J.expert_count; ++i) {
        ExpertMfma &x = J.expert[i];
        require(x.rows == e.rows && x.columns == e.columns, "MFMA GEMM: expert entries differ in shape");
        x.tile_rows = x.rows / kTile;
        x.tc_shift = log2_of(x.columns / kTile);
    }
    J.row_groups = ceil_div(e.rows / kTile, kBlockTileRows);  // row quarters of an item
    J.position_groups = ceil_div(J.max_positions, 32u * kExpertCB);
    J.items = J.expert_count * J.max_active * J.position_groups * J.row_groups;  // upper bound
    const uint32_t cap = ctx->cu_count >= 16 ? ctx->cu_count / 16 * 16 : 16u;
    const uint32_t needed = 16u * ceil_div(ceil_div(J.items, kExpertGroups), 8u);
    const uint32_t blocks = needed < cap ? needed : cap;
    auto kernel = k_expert_mfma<kExpertCB, kExpertGroups, kExpertPasses>;
    launch(ctx, "expert_mfma", kernel, dim3(blocks), dim3(512 * kExpertGroups), 0, J);
}

void launch_ne_mfma(adi_hip_context *ctx, NeMfmaJobs &J) {
    require(J.ne_count >= 1 && J.ne_count <= 2, "MFMA GEMM: one or two NE entries");
    require(J.ne_book != nullptr, "MFMA GEMM: NE codebook missing");
    const NeMfma &n = J.ne[0];
    require(n.columns >= 32 && n.rows >= 16, "MFMA GEMM: NE matrix below 16 x 32");
    require(is_power_of_two(n.columns) && n.rows % kTile == 0,
            "MFMA GEMM: NE columns must be a power of two and rows whole tiles");
    require(size_t(n.batch) * n.columns * 2u < (size_t(1) << 32) &&
                size_t(n.rows / kTile) * (n.columns / kTile) * 128u < (size_t(1) << 32),
            "MFMA GEMM: NE operands beyond 4 GiB");
    for (uint32_t i = 0; i < J.ne_count; ++i) {
        NeMfma &x = J.ne[i];
        require(x.rows == n.rows && x.columns == n.columns && x.batch == n.batch,
                "MFMA GEMM: NE entries differ in shape");
        require(aligned_to(x.x_hi, 16) && aligned_to(x.x_lo, 16) && aligned_to(x.z, 16),
                "MFMA GEMM: NE x_hat and Z must be 16-byte aligned");
        x.tile_rows = x.rows / kTile;
        x.tc_shift = log2_of(x.columns / kTile);
    }
    J.row_groups = ceil_div(n.rows / kTile, kNeItemTileRows);
    J.position_groups = ceil_div(n.batch, 32u);
    J.k_slices = ne_mfma_slices(n.rows, n.columns, n.batch);
    J.items = J.ne_count * J.position_groups * J.row_groups * J.k_slices;
    launch(ctx, "ne_mfma", k_ne_mfma, dim3(J.items), dim3(kNeThreads), 0, J);
}

}  // namespace adi_hip
