// dense.hip -- bf16 dense products in the CPU's reduction order, RMS norm,
// top_experts and the stable counting sort of the MoE dispatch.
//
// Routing must be bit-identical with the CPU path, so the router logits are
// computed in exactly the order of the CPU ISA the host build selects
// (src/simd.cpp:88-96, src/simd_x86_avx2.cpp:172-193,
// src/simd_x86_avx512.cpp:109-130): `lanes` independent sums, lane j taking
// columns j, j+lanes, ..., then the lane sums added 0..lanes-1 from 0.0f, then
// any trailing columns. The AVX-512 build of the reference fuses each lane's
// multiply-add (GCC contracts the intrinsics' mul+add), the AVX2 and scalar
// builds do not. Contraction is switched off in this file and the fused form
// is written as fmaf.
#include "dense.hpp"
#include "route.hpp"

namespace adi_hip {
namespace {

constexpr uint32_t kTokensPerThread = 4;

template <int LANES, bool FUSED>
__device__ __forceinline__ float lane_step(float acc, float w, float x) {
#pragma clang fp contract(off)
    if constexpr (FUSED) {
        return fmaf(w, x, acc);
    } else {
        return acc + w * x;
    }
}

// Block of 256 threads = 256/LANES rows x LANES lanes; each thread carries
// kTokensPerThread tokens.
template <int LANES, bool FUSED>
__global__ __launch_bounds__(256) void k_bf16_ordered(
    const uint16_t *__restrict__ w, uint32_t rows, uint32_t columns,
    const float *__restrict__ x, uint32_t batch, float *__restrict__ out) {
#pragma clang fp contract(off)
    constexpr uint32_t rows_per_block = 256 / LANES;
    __shared__ float lanes[kTokensPerThread][256];
    const uint32_t lane = threadIdx.x % LANES;
    const uint32_t local_row = threadIdx.x / LANES;
    const uint32_t row = blockIdx.x * rows_per_block + local_row;
    const uint32_t t0 = blockIdx.y * kTokensPerThread;
    const bool row_ok = row < rows;
    const uint32_t full = columns / LANES * LANES;

    float acc[kTokensPerThread];
#pragma unroll
    for (uint32_t t = 0; t < kTokensPerThread; ++t) {
        acc[t] = 0.0f;
    }
    if (row_ok) {
        const uint16_t *wr = w + static_cast<size_t>(row) * columns;
        for (uint32_t base = 0; base < full; base += LANES) {
            const uint32_t k = base + lane;
            const float wk = bf16_bits_to_float(wr[k]);
#pragma unroll
            for (uint32_t t = 0; t < kTokensPerThread; ++t) {
                if (t0 + t < batch) {
                    acc[t] = lane_step<LANES, FUSED>(acc[t], wk,
                                                     x[static_cast<size_t>(t0 + t) * columns + k]);
                }
            }
        }
    }
#pragma unroll
    for (uint32_t t = 0; t < kTokensPerThread; ++t) {
        lanes[t][threadIdx.x] = acc[t];
    }
    __syncthreads();
    if (!row_ok || lane >= kTokensPerThread) {
        return;
    }
    // Lane t of the row finishes token t0 + t: ordered lane sum, then tail.
    const uint32_t t = lane;
    if (t0 + t >= batch) {
        return;
    }
    float sum = 0.0f;
    for (uint32_t j = 0; j < LANES; ++j) {
        sum = sum + lanes[t][local_row * LANES + j];
    }
    const uint16_t *wr = w + static_cast<size_t>(row) * columns;
    const float *xr = x + static_cast<size_t>(t0 + t) * columns;
    for (uint32_t k = full; k < columns; ++k) {
        sum = lane_step<LANES, FUSED>(sum, bf16_bits_to_float(wr[k]), xr[k]);
    }
    out[static_cast<size_t>(t0 + t) * rows + row] = sum;
}

// Faster form of the same order for widths up to 4096: one wave per block
// holding 64/LANES rows x LANES lanes; the block's weight rows and its
// kTokensPerThread tokens are first staged in LDS with wide coalesced loads,
// so the lanes' strictly sequential multiply-add chains read only LDS. An
// optional extra row (the shared-expert gate) is appended after `rows` and
// written to `out_extra`.
// The chains of one thread for the first NT tokens: lane `lane` of a row
// accumulates columns lane, lane + LANES, ... in order (operands of kUnroll
// steps are read from LDS first, then the chains advance).
template <int LANES, bool FUSED, int NT>
__device__ __forceinline__ void bf16_chains(const uint16_t *wr, const float *xs, uint32_t columns,
                                            uint32_t full, uint32_t lane,
                                            float (&acc)[kTokensPerThread]) {
#pragma clang fp contract(off)
    constexpr uint32_t kUnroll = 8;
    uint32_t base = 0;
    for (; base + kUnroll * LANES <= full; base += kUnroll * LANES) {
        float wk[kUnroll], xk[NT][kUnroll];
#pragma unroll
        for (uint32_t u = 0; u < kUnroll; ++u) {
            const uint32_t k = base + u * LANES + lane;
            wk[u] = bf16_bits_to_float(wr[k]);
#pragma unroll
            for (uint32_t t = 0; t < NT; ++t) {
                xk[t][u] = xs[t * columns + k];
            }
        }
#pragma unroll
        for (uint32_t u = 0; u < kUnroll; ++u) {
#pragma unroll
            for (uint32_t t = 0; t < NT; ++t) {
                acc[t] = lane_step<LANES, FUSED>(acc[t], wk[u], xk[t][u]);
            }
        }
    }
    for (; base < full; base += LANES) {
        const uint32_t k = base + lane;
        const float wk = bf16_bits_to_float(wr[k]);
#pragma unroll
        for (uint32_t t = 0; t < NT; ++t) {
            acc[t] = lane_step<LANES, FUSED>(acc[t], wk, xs[t * columns + k]);
        }
    }
}

// One wave per block: registers for a whole staging round (16 + XB 16-byte
// loads in flight) matter more than occupancy.
template <int LANES, bool FUSED, uint32_t XB>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(1, 2))) void k_bf16_lds(
    const uint16_t *__restrict__ w, uint32_t rows, const uint16_t *__restrict__ w_extra, uint32_t extra_rows,
    uint32_t columns, const float *__restrict__ x, uint32_t batch, float *__restrict__ out,
    float *__restrict__ out_extra) {
#pragma clang fp contract(off)
    constexpr uint32_t rows_per_block = 64 / LANES;
    extern __shared__ float xs[];  // [tokens][columns] then [rows_per_block][columns] bf16
    const uint32_t t0 = blockIdx.y * kTokensPerThread;
    const uint32_t tokens = batch - t0 < kTokensPerThread ? batch - t0 : kTokensPerThread;
    uint16_t *ws = reinterpret_cast<uint16_t *>(xs + static_cast<size_t>(kTokensPerThread) * columns);
    const uint32_t total_rows = rows + (w_extra != nullptr ? extra_rows : 0u);
    const uint32_t row0 = blockIdx.x * rows_per_block;
    const uint32_t rows_here =
        total_rows - row0 < rows_per_block ? total_rows - row0 : rows_per_block;
    const uintptr_t addresses = reinterpret_cast<uintptr_t>(w) | reinterpret_cast<uintptr_t>(x) |
                                reinterpret_cast<uintptr_t>(w_extra);
    if ((columns % 8u) == 0 && (addresses & 15u) == 0) {
        // 16-byte staging in rounds: every load of a round (16 of the
        // weight rows, XB of the tokens: 8 for one token, 32 for four; one
        // round for a 4 x 2048 block) is issued before the first LDS store,
        // so the block waits for memory once per round (with 8 token loads a
        // round, four tokens took four rounds: 257 x 2048 at 4 tokens
        // 10.6 -> 6.8 us, at 16 tokens 10.7 -> 7.0). Indexes past the end
        // are clamped to the last element: those lanes load it and store the
        // same value again, so nothing is guarded.
        constexpr uint32_t kWBatch = 16, kXBatch = XB;
        const uint32_t w_per_row = columns / 8u;
        const uint32_t w_total = rows_here * w_per_row;
        const uint32_t x_per_row = columns / 4u;
        const uint32_t x_total = tokens * x_per_row;
        const float4 *xsrc = reinterpret_cast<const float4 *>(x + static_cast<size_t>(t0) * columns);
        for (uint32_t round = 0;; ++round) {
            const uint32_t wf0 = round * 64u * kWBatch, xf0 = round * 64u * kXBatch;
            if (wf0 >= w_total && xf0 >= x_total) {
                break;
            }
            uint4 wv[kWBatch];
            float4 xv[kXBatch];
            uint32_t wat[kWBatch], xat[kXBatch];
#pragma unroll
            for (uint32_t u = 0; u < kWBatch; ++u) {
                wat[u] = min(wf0 + u * 64u + threadIdx.x, w_total - 1u);
                const uint32_t r = wat[u] / w_per_row, k = wat[u] - r * w_per_row;
                const uint32_t row = row0 + r;
                const uint16_t *src = row < rows ? w + static_cast<size_t>(row) * columns
                                                 : w_extra + static_cast<size_t>(row - rows) * columns;
                wv[u] = reinterpret_cast<const uint4 *>(src)[k];
            }
#pragma unroll
            for (uint32_t u = 0; u < kXBatch; ++u) {
                xat[u] = min(xf0 + u * 64u + threadIdx.x, x_total - 1u);
                xv[u] = xsrc[xat[u]];
            }
#pragma unroll
            for (uint32_t u = 0; u < kWBatch; ++u) {
                reinterpret_cast<uint4 *>(ws)[wat[u]] = wv[u];
            }
#pragma unroll
            for (uint32_t u = 0; u < kXBatch; ++u) {
                reinterpret_cast<float4 *>(xs)[xat[u]] = xv[u];
            }
        }
    } else {
        for (uint32_t t = 0; t < tokens; ++t) {
            const float *src = x + static_cast<size_t>(t0 + t) * columns;
            for (uint32_t k = threadIdx.x; k < columns; k += 64u) {
                xs[t * columns + k] = src[k];
            }
        }
        for (uint32_t r = 0; r < rows_here; ++r) {
            const uint32_t row = row0 + r;
            const uint16_t *src = row < rows ? w + static_cast<size_t>(row) * columns
                                             : w_extra + static_cast<size_t>(row - rows) * columns;
            for (uint32_t k = threadIdx.x; k < columns; k += 64u) {
                ws[r * columns + k] = src[k];
            }
        }
    }
    __syncthreads();
    const uint32_t lane = threadIdx.x % LANES;
    const uint32_t local_row = threadIdx.x / LANES;
    const uint32_t row = row0 + local_row;
    const bool row_ok = row < total_rows;
    const uint16_t *wr = ws + local_row * columns;
    const uint32_t full = columns / LANES * LANES;
    // chains of the block's tokens only (rows of xs past `tokens` are not
    // staged; the sums of those chains are never read)
    float acc[kTokensPerThread] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (row_ok) {
        static_assert(kTokensPerThread == 4, "one case per token count");
        switch (tokens) {
        case 1: bf16_chains<LANES, FUSED, 1>(wr, xs, columns, full, lane, acc); break;
        case 2: bf16_chains<LANES, FUSED, 2>(wr, xs, columns, full, lane, acc); break;
        case 3: bf16_chains<LANES, FUSED, 3>(wr, xs, columns, full, lane, acc); break;
        default: bf16_chains<LANES, FUSED, 4>(wr, xs, columns, full, lane, acc); break;
        }
    }
    // ordered lane sums through LDS: lane t of each row finishes token t
    __shared__ float lane_sums[kTokensPerThread][64];
#pragma unroll
    for (uint32_t t = 0; t < kTokensPerThread; ++t) {
        lane_sums[t][threadIdx.x] = acc[t];
    }
    __syncthreads();
    if (!row_ok || lane >= tokens) {
        return;
    }
    float sum = 0.0f;
    for (uint32_t j = 0; j < LANES; ++j) {
        sum = sum + lane_sums[lane][local_row * LANES + j];
    }
    for (uint32_t k = full; k < columns; ++k) {
        sum = lane_step<LANES, FUSED>(sum, bf16_bits_to_float(wr[k]), xs[lane * columns + k]);
    }
    if (row < rows) {
        out[static_cast<size_t>(t0 + lane) * rows + row] = sum;
    } else {
        out_extra[static_cast<size_t>(t0 + lane) * extra_rows + (row - rows)] = sum;
    }
}

// Register-tiled form of the same order for batches of many tokens: a block
// of THREADS threads holds BLOCK tokens x BLOCK rows (16, or 8 where 16 would
// leave most CUs idle); thread (lane l, tile group)
// carries the chains of lane l for T tokens x R rows, so each operand read
// from LDS feeds T or R multiply-adds. K is staged 256 columns at a time,
// transposed to [token or row][lane][step] with a padded pitch, so a thread
// reads four consecutive steps of its lane with one 16-byte read and the 16
// (or 8) lanes of a read hit distinct banks. The lane sums are then added in
// lane order from 0.0f, exactly as above. Needs columns % 256 == 0 and
// 16-byte aligned operands.
constexpr uint32_t kTiledChunk = 256;
constexpr uint32_t kTiledLargeThreads = 256;  // threads of a 16 x 16 tile block

template <int LANES, uint32_t BLOCK, uint32_t THREADS>
struct TiledShape {
    static constexpr uint32_t groups = THREADS / LANES;                // tile groups per lane
    static constexpr uint32_t row_groups = 4;
    static constexpr uint32_t token_groups = groups / row_groups;
    static constexpr uint32_t T = BLOCK / token_groups;                // tokens per thread
    static constexpr uint32_t R = BLOCK / row_groups;                  // rows per thread
    static constexpr uint32_t steps = kTiledChunk / LANES;             // chunk steps per lane
    static constexpr uint32_t pitch = steps + 4;                       // floats per [.][lane] row
};

template <int LANES, bool FUSED, uint32_t BLOCK, uint32_t THREADS>
__global__ __launch_bounds__(THREADS) void k_bf16_tiled(
    const uint16_t *__restrict__ w, uint32_t rows, const uint16_t *__restrict__ w_extra,
    uint32_t extra_rows, uint32_t columns, const float *__restrict__ x, uint32_t batch,
    float *__restrict__ out, float *__restrict__ out_extra) {
#pragma clang fp contract(off)
    using S = TiledShape<LANES, BLOCK, THREADS>;
    static_assert(S::T >= 1 && S::R >= 1 && S::T * S::token_groups == BLOCK, "tile shape");
    __shared__ float xs[BLOCK][LANES][S::pitch];
    __shared__ float ws[BLOCK][LANES][S::pitch];
    const uint32_t total_rows = rows + (w_extra != nullptr ? extra_rows : 0u);
    // XCD-aware tiles: blocks are dealt to the eight XCDs round robin, so
    // block id goes to XCD id % 8. With at least eight token tiles XCD x
    // takes token tiles x, x + 8, ... with every row tile, and its L2 holds
    // only its own tokens (and the weights, which every XCD needs); with
    // fewer it takes row tiles x, x + 8, ... with every token tile, so no
    // XCD idles and each reads an eighth of the weights
    const uint32_t row_tiles = (total_rows + BLOCK - 1u) / BLOCK;
    const uint32_t token_tiles = (batch + BLOCK - 1u) / BLOCK;
    const uint32_t xcd = blockIdx.x & 7u, k = blockIdx.x >> 3;
    uint32_t token_tile, row_tile;
    if (token_tiles >= 8u) {
        token_tile = xcd + 8u * (k / row_tiles);
        row_tile = k % row_tiles;
    } else {
        row_tile = xcd + 8u * (k / token_tiles);
        token_tile = k % token_tiles;
    }
    if (token_tile >= token_tiles || row_tile >= row_tiles) {
        return;  // the whole block, before any barrier
    }
    const uint32_t row0 = row_tile * BLOCK;
    const uint32_t t0 = token_tile * BLOCK;
    const uint32_t lane = threadIdx.x % LANES;
    const uint32_t group = threadIdx.x / LANES;
    const uint32_t tg = group / S::row_groups, rg = group % S::row_groups;
    // staging: thread tid copies float4 number u * 128 + tid of the chunk's
    // 16 x 256 x-block and uint4 (8 bf16) number u * 128 + tid of the
    // w-block; rows and tokens past the ends are clamped to real ones (never
    // stored)
    float acc[S::T][S::R];
#pragma unroll
    for (uint32_t t = 0; t < S::T; ++t) {
#pragma unroll
        for (uint32_t r = 0; r < S::R; ++r) {
            acc[t][r] = 0.0f;
        }
    }
    // chunk c + 1 is loaded into registers while chunk c is multiplied
    constexpr uint32_t kXU = BLOCK * 64u / THREADS, kWU = BLOCK * 32u / THREADS;
    static_assert(kXU >= 1 && kWU >= 1, "staging shares");
    float4 xv[kXU];
    uint4 wv[kWU];
    auto load_chunk = [&](uint32_t c0) {
#pragma unroll
        for (uint32_t u = 0; u < kXU; ++u) {
            const uint32_t idx = u * THREADS + threadIdx.x;  // tokens x 64 float4
            const uint32_t t = idx >> 6, k = (idx & 63u) * 4u;
            const uint32_t tok = min(t0 + t, batch - 1u);
            xv[u] = *reinterpret_cast<const float4 *>(x + static_cast<size_t>(tok) * columns + c0 + k);
        }
#pragma unroll
        for (uint32_t u = 0; u < kWU; ++u) {
            const uint32_t idx = u * THREADS + threadIdx.x;  // rows x 32 uint4
            const uint32_t r = idx >> 5, k = (idx & 31u) * 8u;
            const uint32_t row = min(row0 + r, total_rows - 1u);
            const uint16_t *src = row < rows ? w + static_cast<size_t>(row) * columns
                                             : w_extra + static_cast<size_t>(row - rows) * columns;
            wv[u] = *reinterpret_cast<const uint4 *>(src + c0 + k);
        }
    };
    auto store_chunk = [&]() {
#pragma unroll
        for (uint32_t u = 0; u < kXU; ++u) {
            const uint32_t idx = u * THREADS + threadIdx.x;
            const uint32_t t = idx >> 6, k = (idx & 63u) * 4u;
            const float e[4] = {xv[u].x, xv[u].y, xv[u].z, xv[u].w};
#pragma unroll
            for (uint32_t q = 0; q < 4; ++q) {
                xs[t][(k + q) % LANES][(k + q) / LANES] = e[q];
            }
        }
#pragma unroll
        for (uint32_t u = 0; u < kWU; ++u) {
            const uint32_t idx = u * THREADS + threadIdx.x;
            const uint32_t r = idx >> 5, k = (idx & 31u) * 8u;
            const uint32_t e[4] = {wv[u].x, wv[u].y, wv[u].z, wv[u].w};
#pragma unroll
            for (uint32_t q = 0; q < 8; ++q) {
                const uint32_t bits = q & 1u ? e[q / 2] >> 16 : e[q / 2] & 0xFFFFu;
                ws[r][(k + q) % LANES][(k + q) / LANES] = bf16_bits_to_float(static_cast<uint16_t>(bits));
            }
        }
    };
    load_chunk(0);
    store_chunk();
    __syncthreads();
    for (uint32_t c0 = 0; c0 < columns; c0 += kTiledChunk) {
        // the last chunk reloads itself (in bounds, never staged)
        load_chunk(c0 + kTiledChunk < columns ? c0 + kTiledChunk : c0);
#pragma unroll 2
        for (uint32_t i = 0; i < S::steps; i += 4) {
            float4 xk[S::T], wk[S::R];
#pragma unroll
            for (uint32_t t = 0; t < S::T; ++t) {
                xk[t] = *reinterpret_cast<const float4 *>(&xs[tg * S::T + t][lane][i]);
            }
#pragma unroll
            for (uint32_t r = 0; r < S::R; ++r) {
                wk[r] = *reinterpret_cast<const float4 *>(&ws[rg * S::R + r][lane][i]);
            }
#pragma unroll
            for (uint32_t q = 0; q < 4; ++q) {
#pragma unroll
                for (uint32_t t = 0; t < S::T; ++t) {
#pragma unroll
                    for (uint32_t r = 0; r < S::R; ++r) {
                        acc[t][r] = lane_step<LANES, FUSED>(acc[t][r], wk[r][q], xk[t][q]);
                    }
                }
            }
        }
        if (c0 + kTiledChunk < columns) {
            __syncthreads();  // every reader of this chunk is done
            store_chunk();
            __syncthreads();
        }
    }
    // ordered lane sums: the chains go to LDS (reusing xs), then each of the
    // block's kOut outputs is finished by one thread
    constexpr uint32_t kOut = BLOCK * BLOCK;
    static_assert(kOut <= BLOCK * S::pitch, "lane sums must fit the x staging");
    __syncthreads();
    float *sums = &xs[0][0][0];  // [LANES][kOut]
#pragma unroll
    for (uint32_t t = 0; t < S::T; ++t) {
#pragma unroll
        for (uint32_t r = 0; r < S::R; ++r) {
            sums[lane * kOut + (tg * S::T + t) * BLOCK + rg * S::R + r] = acc[t][r];
        }
    }
    __syncthreads();
#pragma unroll
    for (uint32_t o = threadIdx.x; o < kOut; o += THREADS) {
        const uint32_t t = o / BLOCK, r = o % BLOCK;
        const uint32_t tok = t0 + t, row = row0 + r;
        if (tok < batch && row < total_rows) {
            float sum = 0.0f;
            for (uint32_t j = 0; j < LANES; ++j) {
                sum = sum + sums[j * kOut + o];
            }
            if (row < rows) {
                out[static_cast<size_t>(tok) * rows + row] = sum;
            } else {
                out_extra[static_cast<size_t>(tok) * extra_rows + (row - rows)] = sum;
            }
        }
    }
}

// The scalar order has one lane per row; its "lane sum" is 0 + the row sum,
// so the generic kernel with LANES = 1 would need four lanes to finish four
// tokens. This variant gives each thread one (row, token).
__global__ __launch_bounds__(256) void k_bf16_scalar(
    const uint16_t *__restrict__ w, uint32_t rows, uint32_t columns,
    const float *__restrict__ x, uint32_t batch, float *__restrict__ out) {
#pragma clang fp contract(off)
    const uint32_t row = blockIdx.x * 256u + threadIdx.x;
    const uint32_t t = blockIdx.y;
    if (row >= rows || t >= batch) {
        return;
    }
    const uint16_t *wr = w + static_cast<size_t>(row) * columns;
    const float *xr = x + static_cast<size_t>(t) * columns;
    float sum = 0.0f;
    for (uint32_t k = 0; k < columns; ++k) {
        sum = sum + bf16_bits_to_float(wr[k]) * xr[k];
    }
    out[static_cast<size_t>(t) * rows + row] = sum;
}

// rms_norm (src/kernels.cpp:1052-1073): scale = 1 / sqrt(sum(x^2) / n +
// epsilon), then x * scale * (offset + w), each product rounded as written.
// One block of 256 per row; the sum of squares runs as a tree (each thread
// its strided share, then the wave and block sums) rather than the CPU's
// left-to-right loop, so the scale agrees to float rounding (a sequential
// sum on one lane costs ~20 us for 2048 values).
// With ADD the row is first replaced by row + residual (the residual add of
// a decoder layer), and the norm is taken of that sum: the same values as a
// separate add and norm.
template <bool ADD>
__global__ __launch_bounds__(256) void k_rms_norm(
    float *__restrict__ x, const float *__restrict__ residual, const uint16_t *__restrict__ weight,
    uint32_t count, float offset, float epsilon, float *__restrict__ out) {
#pragma clang fp contract(off)
    __shared__ float scale_shared;
    __shared__ float wave_sums[4];
    float *row = x + static_cast<size_t>(blockIdx.x) * count;
    const float *add = ADD ? residual + static_cast<size_t>(blockIdx.x) * count : nullptr;
    float *dst = out + static_cast<size_t>(blockIdx.x) * count;
    // up to 8 values a thread: the row and the weights are loaded at once
    // and kept in registers for the output (same sums, same products)
    if (count <= 8u * blockDim.x) {
        block_rms_norm(
            [&](uint32_t i) {
                if constexpr (ADD) {
                    return row[i] + add[i];
                } else {
                    return row[i];
                }
            },
            [&](uint32_t i, float v) {
                if constexpr (ADD) {
                    row[i] = v;
                }
            },
            weight, count, offset, epsilon, dst, wave_sums, &scale_shared, threadIdx.x);
        return;
    }
    float squares = 0.0f;
    for (uint32_t i = threadIdx.x; i < count; i += blockDim.x) {
        float value = row[i];
        if constexpr (ADD) {
            value = value + add[i];
            row[i] = value;
        }
        squares += value * value;
    }
    squares += lane_xor<1>(squares);
    squares += lane_xor<2>(squares);
    squares += lane_xor<4>(squares);
    squares += lane_xor<8>(squares);
    squares += lane_xor<16>(squares);
    squares += lane_xor<32>(squares);
    if ((threadIdx.x & 63u) == 0) {
        wave_sums[threadIdx.x >> 6] = squares;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        const float total = (wave_sums[0] + wave_sums[1]) + (wave_sums[2] + wave_sums[3]);
        scale_shared = 1.0f / sqrtf(total / static_cast<float>(count) + epsilon);
    }
    __syncthreads();
    const float scale = scale_shared;
    for (uint32_t i = threadIdx.x; i < count; i += blockDim.x) {
        dst[i] = row[i] * scale * (offset + bf16_bits_to_float(weight[i]));
    }
}

// One wave per row, four rows per block.
template <int SLOTS>
__global__ __launch_bounds__(256) void k_top_experts(
    const float *__restrict__ logits, const float *__restrict__ bias, uint32_t batch,
    uint32_t experts, uint32_t *__restrict__ route_expert, float *__restrict__ route_weight) {
    const uint32_t row = blockIdx.x * 4u + (threadIdx.x >> 6);
    if (row >= batch) {
        return;
    }
    top8_wave<SLOTS>(logits + static_cast<size_t>(row) * experts, bias, experts,
                     threadIdx.x & 63u, route_expert + row * 8u, route_weight + row * 8u);
}

// ---- multi-block sort ---------------------------------------------------------

constexpr uint32_t kChunk = 64;             // route positions per histogram chunk
constexpr uint32_t kFinalizeBases = 16384;  // chunk x expert bases held in LDS

// Exclusive scan of one value per thread over a block of up to 1024 threads
// (16 waves); `sums` holds 16 words. Ends with a barrier.
__device__ __forceinline__ uint32_t block_exclusive_scan(uint32_t value, uint32_t *sums,
                                                         uint32_t &block_total) {
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    uint32_t inclusive = value;
#pragma unroll
    for (int offset = 1; offset < 64; offset <<= 1) {
        const uint32_t other = static_cast<uint32_t>(__shfl_up(static_cast<int>(inclusive), offset));
        if (lane >= static_cast<uint32_t>(offset)) {
            inclusive += other;
        }
    }
    if (lane == 63u) {
        sums[wave] = inclusive;
    }
    __syncthreads();
    uint32_t before = 0, total = 0;
    const uint32_t waves = blockDim.x >> 6;
    for (uint32_t w = 0; w < waves; ++w) {
        before += w < wave ? sums[w] : 0u;
        total += sums[w];
    }
    __syncthreads();
    block_total = total;
    return before + inclusive - value;
}

// One wave over chunk c of 64 route positions (expert of position c * 64 +
// lane in `e`): the rank of each position among the chunk's earlier positions
// with the same expert (ballot match on the expert bits) and the chunk's
// per-expert counts, built in `h` (zeroed by the caller, visible to this wave).
__device__ __forceinline__ void chunk_hist_wave(const RouteSort &a, uint32_t c, uint32_t lane,
                                                bool valid, uint32_t e, uint32_t *h) {
    const uint32_t i = c * kChunk + lane;
    uint64_t peers = __ballot(valid);
    if (!valid) {
        peers = ~peers;
    }
    for (uint32_t bit = 0; bit < 10u; ++bit) {
        const bool set = (e >> bit) & 1u;
        const uint64_t vote = __ballot(set);
        peers &= set ? vote : ~vote;
    }
    const uint32_t rank = __popcll(peers & ((1ull << lane) - 1ull));
    if (valid) {
        a.position_rank[i] = rank;
        if (rank == 0) {
            h[e] = __popcll(peers);
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_wave_barrier();
    for (uint32_t x = lane; x < a.experts; x += 64u) {
        a.chunk_hist[static_cast<size_t>(c) * a.experts + x] = h[x];
    }
}

// One wave per chunk of 64 route positions (routes from a.route_expert).
__global__ __launch_bounds__(256) void k_route_hist(RouteSort a, uint32_t chunks) {
    extern __shared__ uint32_t hist[];  // [4][experts]
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t c = blockIdx.x * 4u + wave;
    if (c >= chunks) {
        return;  // wave-uniform; no block barrier follows
    }
    uint32_t *h = hist + wave * a.experts;
    for (uint32_t e = lane; e < a.experts; e += 64u) {
        h[e] = 0u;
    }
    const uint32_t i = c * kChunk + lane;
    const bool valid = i < a.positions;
    // LDS operations of one wave complete in order: the zeroing lands first
    chunk_hist_wave(a, c, lane, valid, valid ? a.route_expert[i] : 0u, h);
}

// top_experts for the 8 rows of one chunk (one wave per row), then the
// chunk's ranks and counts from the routes kept in LDS: block b is chunk b.
template <int SLOTS>
__global__ __launch_bounds__(512) void k_top_experts_hist(
    const float *__restrict__ logits, const float *__restrict__ bias, uint32_t batch,
    uint32_t *__restrict__ route_expert, float *__restrict__ route_weight, RouteSort a) {
    static_assert(kChunk == 64, "a chunk is the 8 routes of 8 rows");
    __shared__ uint32_t local[kChunk];
    __shared__ uint32_t hist[kMaxExperts];
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t row = blockIdx.x * 8u + wave;
    for (uint32_t e = threadIdx.x; e < a.experts; e += blockDim.x) {
        hist[e] = 0u;
    }
    if (row < batch) {
        top8_wave<SLOTS>(logits + static_cast<size_t>(row) * a.experts, bias, a.experts, lane,
                         route_expert + row * 8u, route_weight + row * 8u, local + wave * 8u);
    }
    __syncthreads();
    if (wave == 0) {
        const uint32_t i = blockIdx.x * kChunk + lane;
        const bool valid = i < a.positions;
        chunk_hist_wave(a, blockIdx.x, lane, valid, valid ? local[lane] : 0u, hist);
    }
}

// One block: per-expert totals and offsets, the ascending active list and
// slot table, each chunk's first grouped index per expert (in LDS), and then
// the grouped index of every position, stable in (token, route) order: its
// chunk's first index for its expert plus its rank within the chunk. The chunk
// counts are staged in LDS with coalesced loads and each expert's scan over
// the chunks is split into up to four ranges scanned by separate threads.
__global__ __launch_bounds__(1024) void k_route_finalize(RouteSort a, uint32_t chunks) {
    extern __shared__ uint32_t base[];  // [chunks][experts]
    __shared__ uint32_t start[kMaxExperts];
    __shared__ uint32_t part[4][kMaxExperts];
    __shared__ uint32_t sums[16];
    const uint32_t t = threadIdx.x;
    const uint32_t E = a.experts;
    const uint32_t cells = chunks * E;
    // kStage loads in flight per thread before their LDS stores
    constexpr uint32_t kStage = 8;
    for (uint32_t i0 = t; i0 < cells; i0 += kStage * blockDim.x) {
        uint32_t v[kStage];
#pragma unroll
        for (uint32_t u = 0; u < kStage; ++u) {
            const uint32_t i = i0 + u * blockDim.x;
            v[u] = i < cells ? a.chunk_hist[i] : 0u;
        }
#pragma unroll
        for (uint32_t u = 0; u < kStage; ++u) {
            const uint32_t i = i0 + u * blockDim.x;
            if (i < cells) {
                base[i] = v[u];
            }
        }
    }
    __syncthreads();
    // thread (q, e) = (t / E, t % E) scans chunks [q * per, (q + 1) * per)
    const uint32_t ranges = E <= blockDim.x / 4u ? 4u : (E <= blockDim.x / 2u ? 2u : 1u);
    const uint32_t per = (chunks + ranges - 1u) / ranges;
    const uint32_t q = t / E, e_scan = t - q * E;
    const bool scanner = q < ranges;
    const uint32_t c_begin = scanner ? min(q * per, chunks) : 0u;
    const uint32_t c_end = scanner ? min(c_begin + per, chunks) : 0u;
    if (scanner) {
        uint32_t running = 0;
        // eight chunks' counts are read before any is overwritten
        for (uint32_t c0 = c_begin; c0 < c_end; c0 += 8u) {
            uint32_t v[8];
#pragma unroll
            for (uint32_t u = 0; u < 8u; ++u) {
                v[u] = c0 + u < c_end ? base[(c0 + u) * E + e_scan] : 0u;
            }
#pragma unroll
            for (uint32_t u = 0; u < 8u; ++u) {
                if (c0 + u < c_end) {
                    base[(c0 + u) * E + e_scan] = running;
                }
                running += v[u];
            }
        }
        part[q][e_scan] = running;
    }
    __syncthreads();
    if (scanner && q > 0) {
        uint32_t offset = 0;
        for (uint32_t r = 0; r < q; ++r) {
            offset += part[r][e_scan];
        }
        for (uint32_t c = c_begin; c < c_end; ++c) {
            base[c * E + e_scan] += offset;
        }
    }
    const bool mine = t < E;
    uint32_t total = 0;
    if (mine) {
        for (uint32_t r = 0; r < ranges; ++r) {
            total += part[r][t];
        }
    }
    uint32_t all = 0;
    const uint32_t offset = block_exclusive_scan(mine ? total : 0u, sums, all);
    uint32_t active_total = 0;
    const uint32_t slot = block_exclusive_scan(mine && total != 0u ? 1u : 0u, sums, active_total);
    if (mine) {
        start[t] = offset;
        a.counts[t] = total;
        a.offsets[t] = offset;
        if (total != 0u) {
            if (a.active != nullptr) {
                a.active[slot] = t;
            }
            if (a.slot_info != nullptr) {
                a.slot_info[slot] = make_uint4(t, offset, offset + total, 0u);
            }
        }
    }
    if (t == 0) {
        a.offsets[E] = all;
        if (a.active_count != nullptr) {
            *a.active_count = active_total;
        }
    }
    if (a.slot_info != nullptr) {
        for (uint32_t s = active_total + t; s < E; s += blockDim.x) {
            a.slot_info[s] = make_uint4(0u, 0u, 0u, 0u);
        }
    }
    __syncthreads();
    // kPlace positions per thread at a time: every load of a batch is issued
    // before its stores (the outputs may alias the inputs as far as the
    // compiler knows, so it would not move later loads above them)
    constexpr uint32_t kPlace = 4;
    for (uint32_t i0 = t; i0 < a.positions; i0 += kPlace * blockDim.x) {
        uint32_t e[kPlace], rank[kPlace];
#pragma unroll
        for (uint32_t u = 0; u < kPlace; ++u) {
            const uint32_t i = i0 + u * blockDim.x;
            const bool valid = i < a.positions;
            e[u] = valid ? a.route_expert[i] : 0u;
            rank[u] = valid ? a.position_rank[i] : 0u;
        }
#pragma unroll
        for (uint32_t u = 0; u < kPlace; ++u) {
            const uint32_t i = i0 + u * blockDim.x;
            if (i < a.positions) {
                const uint32_t g = start[e[u]] + base[(i / kChunk) * E + e[u]] + rank[u];
                a.grouped_batch[g] = i / 8u;
                a.route_to_grouped[i] = g;
                if (a.position_expert != nullptr) {
                    a.position_expert[g] = e[u];
                }
            }
        }
    }
}

__global__ __launch_bounds__(64) void k_route_sort(RouteSort a) {
    __shared__ uint32_t counts[kMaxExperts];
    __shared__ uint32_t cursor[kMaxExperts];
    route_sort_block(a, a.route_expert, counts, cursor);
}

// Routing of a whole batch of at most kRouteBatch rows in one block:
// top_experts for every row (one wave per row), then the stable counting sort
// reading the routes back from LDS.
template <int SLOTS>
__global__ __launch_bounds__(1024) void k_route(const float *__restrict__ logits,
                                               const float *__restrict__ bias, uint32_t batch,
                                               uint32_t *__restrict__ route_expert,
                                               float *__restrict__ route_weight, RouteSort a) {
    __shared__ uint32_t counts[kMaxExperts];
    __shared__ uint32_t cursor[kMaxExperts];
    __shared__ uint32_t local_expert[kRouteBatch * 8];
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    for (uint32_t t = wave; t < batch; t += blockDim.x / 64u) {
        top8_wave<SLOTS>(logits + static_cast<size_t>(t) * a.experts, bias, a.experts, lane,
                         route_expert + t * 8u, route_weight + t * 8u, local_expert + t * 8u);
    }
    __syncthreads();
    route_sort_block(a, local_expert, counts, cursor);
}

}  // namespace

void launch_bf16_ordered(adi_hip_context *ctx, const uint16_t *w, uint32_t rows,
                         uint32_t columns, const float *x, uint32_t batch,
                         float *out, uint32_t lanes) {
    launch_bf16_ordered_extra(ctx, w, rows, nullptr, columns, x, batch, out, nullptr, lanes);
}

void launch_bf16_ordered_extra(adi_hip_context *ctx, const uint16_t *w, uint32_t rows,
                               const uint16_t *w_extra, uint32_t columns, const float *x,
                               uint32_t batch, float *out, float *out_extra, uint32_t lanes) {
    const uint32_t total = rows + (w_extra != nullptr ? 1u : 0u);
    const uintptr_t addresses = reinterpret_cast<uintptr_t>(w) | reinterpret_cast<uintptr_t>(x) |
                                reinterpret_cast<uintptr_t>(w_extra);
    if ((lanes == 8 || lanes == 16) && batch >= kTiledBatch && columns % kTiledChunk == 0 &&
        (addresses & 15u) == 0) {
        // one dimension: the kernel maps block ids to (row tile, token tile)
        // per XCD. 8 x 8 tiles of 128 threads up to kTiledSmallBatch tokens
        // (257 x 2048 router: 16.2 -> 8.0 us at 32 and 64 tokens, 9.5 us at
        // 128, 12.6 at 256), 16 x 16 tiles of 256 threads above (21.3 us at
        // 512 tokens with 128 threads, 17.4 with 256; 8 x 8: 20.7)
        const bool small = batch <= kTiledSmallBatch;
        const uint32_t block = small ? 8u : 16u;
        const uint32_t token_tiles = ceil_div(batch, block), row_tiles = ceil_div(total, block);
        const dim3 grid(token_tiles >= 8u ? 8u * ceil_div(token_tiles, 8u) * row_tiles
                                          : 8u * ceil_div(row_tiles, 8u) * token_tiles);
        const uint32_t threads = small ? 128u : kTiledLargeThreads;
        if (lanes == 8) {
            launch(ctx, "router", small ? k_bf16_tiled<8, false, 8, 128> : k_bf16_tiled<8, false, 16, kTiledLargeThreads>,
                   grid, dim3(threads), 0, w, rows, w_extra, 1u, columns, x, batch, out, out_extra);
        } else {
            launch(ctx, "router", small ? k_bf16_tiled<16, true, 8, 128> : k_bf16_tiled<16, true, 16, kTiledLargeThreads>,
                   grid, dim3(threads), 0, w, rows, w_extra, 1u, columns, x, batch, out, out_extra);
        }
        return;
    }
    const dim3 tokens(ceil_div(batch, kTokensPerThread));
    const uint32_t rpb = lanes == 1 ? 1 : 64 / lanes;
    const size_t lds = size_t(kTokensPerThread) * columns * sizeof(float) +
                       size_t(rpb) * columns * sizeof(uint16_t);
    // dynamic plus the kernel's static 1 KiB must fit the 64 KiB default
    if (lanes != 1 && lds + 1024 <= 65536) {
        if (lanes == 8) {
            launch(ctx, "router", batch == 1 ? k_bf16_lds<8, false, 8> : k_bf16_lds<8, false, 32>,
                   dim3(ceil_div(total, rpb), tokens.x),
                   dim3(64), lds, w, rows, w_extra, 1u, columns, x, batch, out, out_extra);
        } else {
            launch(ctx, "router", batch == 1 ? k_bf16_lds<16, true, 8> : k_bf16_lds<16, true, 32>,
                   dim3(ceil_div(total, rpb), tokens.x),
                   dim3(64), lds, w, rows, w_extra, 1u, columns, x, batch, out, out_extra);
        }
        return;
    }
    if (w_extra != nullptr) {
        launch_bf16_ordered_plain(ctx, w_extra, 1, columns, x, batch, out_extra, lanes);
    }
    launch_bf16_ordered_plain(ctx, w, rows, columns, x, batch, out, lanes);
}

void launch_bf16_pair(adi_hip_context *ctx, const uint16_t *w0, uint32_t rows0, const uint16_t *w1,
                      uint32_t rows1, uint32_t columns, const float *x, uint32_t batch, float *out0,
                      float *out1, uint32_t lanes) {
    const uintptr_t addresses = reinterpret_cast<uintptr_t>(w0) | reinterpret_cast<uintptr_t>(w1) |
                                reinterpret_cast<uintptr_t>(x);
    const uint32_t rpb = 64 / (lanes == 1 ? 64 : lanes);
    const size_t lds = size_t(kTokensPerThread) * columns * sizeof(float) + size_t(rpb) * columns * sizeof(uint16_t);
    if ((lanes == 8 || lanes == 16) && batch < kTiledBatch && lds + 1024 <= 65536 && (addresses & 15u) == 0) {
        // both matrices' rows in one launch of the small-batch kernel
        const dim3 grid(ceil_div(rows0 + rows1, rpb), ceil_div(batch, kTokensPerThread));
        if (lanes == 8) {
            launch(ctx, "bf16_pair", batch == 1 ? k_bf16_lds<8, false, 8> : k_bf16_lds<8, false, 32>, grid,
                   dim3(64), lds, w0, rows0, w1, rows1, columns, x, batch, out0, out1);
        } else {
            launch(ctx, "bf16_pair", batch == 1 ? k_bf16_lds<16, true, 8> : k_bf16_lds<16, true, 32>, grid,
                   dim3(64), lds, w0, rows0, w1, rows1, columns, x, batch, out0, out1);
        }
        return;
    }
    if ((lanes == 8 || lanes == 16) && batch >= kTiledBatch && columns % kTiledChunk == 0 &&
        (addresses & 15u) == 0) {
        // both matrices' rows in one launch of the register-tiled kernel
        const bool small = batch <= kTiledSmallBatch;
        const uint32_t block = small ? 8u : 16u;
        const uint32_t token_tiles = ceil_div(batch, block), row_tiles = ceil_div(rows0 + rows1, block);
        const dim3 grid(token_tiles >= 8u ? 8u * ceil_div(token_tiles, 8u) * row_tiles
                                          : 8u * ceil_div(row_tiles, 8u) * token_tiles);
        const uint32_t threads = small ? 128u : kTiledLargeThreads;
        if (lanes == 8) {
            launch(ctx, "bf16_pair", small ? k_bf16_tiled<8, false, 8, 128> : k_bf16_tiled<8, false, 16, kTiledLargeThreads>,
                   grid, dim3(threads), 0, w0, rows0, w1, rows1, columns, x, batch, out0, out1);
        } else {
            launch(ctx, "bf16_pair", small ? k_bf16_tiled<16, true, 8, 128> : k_bf16_tiled<16, true, 16, kTiledLargeThreads>,
                   grid, dim3(threads), 0, w0, rows0, w1, rows1, columns, x, batch, out0, out1);
        }
        return;
    }
    launch_bf16_ordered(ctx, w0, rows0, columns, x, batch, out0, lanes);
    launch_bf16_ordered(ctx, w1, rows1, columns, x, batch, out1, lanes);
}

void launch_bf16_ordered_plain(adi_hip_context *ctx, const uint16_t *w, uint32_t rows,
                               uint32_t columns, const float *x, uint32_t batch, float *out,
                               uint32_t lanes) {
    switch (lanes) {
    case 1:
        launch(ctx, "bf16_ordered", k_bf16_scalar, dim3(ceil_div(rows, 256), batch), dim3(256), 0,
               w, rows, columns, x, batch, out);
        break;
    case 8:
        launch(ctx, "bf16_ordered", k_bf16_ordered<8, false>,
               dim3(ceil_div(rows, 256 / 8), ceil_div(batch, kTokensPerThread)), dim3(256), 0, w,
               rows, columns, x, batch, out);
        break;
    default:
        launch(ctx, "bf16_ordered", k_bf16_ordered<16, true>,
               dim3(ceil_div(rows, 256 / 16), ceil_div(batch, kTokensPerThread)), dim3(256), 0, w,
               rows, columns, x, batch, out);
        break;
    }
}

void launch_top_experts(adi_hip_context *ctx, const float *logits, const float *bias,
                        uint32_t batch, uint32_t experts, uint32_t *route_expert,
                        float *route_weight) {
    const dim3 grid(ceil_div(batch, 4));
    const uint32_t slots = ceil_div(experts, 64);
    if (slots <= 1) {
        launch(ctx, "top_experts", k_top_experts<1>, grid, dim3(256), 0, logits, bias, batch, experts, route_expert, route_weight);
    } else if (slots <= 2) {
        launch(ctx, "top_experts", k_top_experts<2>, grid, dim3(256), 0, logits, bias, batch, experts, route_expert, route_weight);
    } else if (slots <= 4) {
        launch(ctx, "top_experts", k_top_experts<4>, grid, dim3(256), 0, logits, bias, batch, experts, route_expert, route_weight);
    } else if (slots <= 8) {
        launch(ctx, "top_experts", k_top_experts<8>, grid, dim3(256), 0, logits, bias, batch, experts, route_expert, route_weight);
    } else {
        launch(ctx, "top_experts", k_top_experts<16>, grid, dim3(256), 0, logits, bias, batch, experts, route_expert, route_weight);
    }
}

void launch_route_sort(adi_hip_context *ctx, const RouteSort &args) {
    const uint32_t chunks = ceil_div(args.positions, kChunk);
    if (args.position_rank != nullptr && args.chunk_hist != nullptr &&
        size_t(chunks) * args.experts <= kFinalizeBases) {
        launch(ctx, "route_hist", k_route_hist, dim3(ceil_div(chunks, 4)), dim3(256),
               size_t(4) * args.experts * sizeof(uint32_t), args, chunks);
        const size_t lds = size_t(chunks) * args.experts * sizeof(uint32_t);
        static const bool ready = set_lds_limit(reinterpret_cast<const void *>(&k_route_finalize),
                                                size_t(kFinalizeBases) * sizeof(uint32_t));
        (void)ready;
        launch(ctx, "route_sort", k_route_finalize, dim3(1), dim3(1024), lds, args, chunks);
        return;
    }
    launch(ctx, "route_sort", k_route_sort, dim3(1), dim3(64), 0, args);
}

// top_experts with the chunk histograms in the same launch, then the one-block
// finalize: two launches for batches whose chunk bases fit the finalize's LDS.
bool launch_route_fused(adi_hip_context *ctx, const float *logits, const float *bias,
                        uint32_t batch, uint32_t *route_expert, float *route_weight,
                        const RouteSort &args) {
    const uint32_t chunks = ceil_div(args.positions, kChunk);
    if (args.position_rank == nullptr || args.chunk_hist == nullptr ||
        args.positions != batch * 8u || size_t(chunks) * args.experts > kFinalizeBases) {
        return false;
    }
    const uint32_t slots = ceil_div(args.experts, 64);
    const dim3 grid(chunks);
    if (slots <= 1) {
        launch(ctx, "top_experts", k_top_experts_hist<1>, grid, dim3(512), 0, logits, bias, batch, route_expert, route_weight, args);
    } else if (slots <= 2) {
        launch(ctx, "top_experts", k_top_experts_hist<2>, grid, dim3(512), 0, logits, bias, batch, route_expert, route_weight, args);
    } else if (slots <= 4) {
        launch(ctx, "top_experts", k_top_experts_hist<4>, grid, dim3(512), 0, logits, bias, batch, route_expert, route_weight, args);
    } else if (slots <= 8) {
        launch(ctx, "top_experts", k_top_experts_hist<8>, grid, dim3(512), 0, logits, bias, batch, route_expert, route_weight, args);
    } else {
        launch(ctx, "top_experts", k_top_experts_hist<16>, grid, dim3(512), 0, logits, bias, batch, route_expert, route_weight, args);
    }
    const size_t lds = size_t(chunks) * args.experts * sizeof(uint32_t);
    static const bool ready = set_lds_limit(reinterpret_cast<const void *>(&k_route_finalize),
                                            size_t(kFinalizeBases) * sizeof(uint32_t));
    (void)ready;
    launch(ctx, "route_sort", k_route_finalize, dim3(1), dim3(1024), lds, args, chunks);
    return true;
}

void launch_route(adi_hip_context *ctx, const float *logits, const float *bias, uint32_t batch,
                  uint32_t *route_expert, float *route_weight, const RouteSort &args) {
    const uint32_t slots = ceil_div(args.experts, 64);
    if (batch > kRouteBatch) {
        // many rows: top_experts over a grid, then the one-block sort
        if (launch_route_fused(ctx, logits, bias, batch, route_expert, route_weight, args)) {
            return;
        }
        launch_top_experts(ctx, logits, bias, batch, args.experts, route_expert, route_weight);
        launch_route_sort(ctx, args);
        return;
    }
    if (slots <= 1) {
        launch(ctx, "route", k_route<1>, dim3(1), dim3(64 * batch), 0, logits, bias, batch, route_expert, route_weight, args);
    } else if (slots <= 2) {
        launch(ctx, "route", k_route<2>, dim3(1), dim3(64 * batch), 0, logits, bias, batch, route_expert, route_weight, args);
    } else if (slots <= 4) {
        launch(ctx, "route", k_route<4>, dim3(1), dim3(64 * batch), 0, logits, bias, batch, route_expert, route_weight, args);
    } else if (slots <= 8) {
        launch(ctx, "route", k_route<8>, dim3(1), dim3(64 * batch), 0, logits, bias, batch, route_expert, route_weight, args);
    } else {
        launch(ctx, "route", k_route<16>, dim3(1), dim3(64 * batch), 0, logits, bias, batch, route_expert, route_weight, args);
    }
}

void launch_add_rms_norm(adi_hip_context *ctx, float *rows_in_out, const float *residual,
                         const uint16_t *weight, uint32_t count, uint32_t rows, float *out) {
    require(count > 0 && rows > 0 && rows_in_out != nullptr && weight != nullptr && out != nullptr,
            "RMS norm shape mismatch");
    if (residual != nullptr) {
        launch(ctx, "add_rms_norm", k_rms_norm<true>, dim3(rows), dim3(256), 0, rows_in_out,
               residual, weight, count, 1.0f, 1.0e-6f, out);
    } else {
        launch(ctx, "rms_norm", k_rms_norm<false>, dim3(rows), dim3(256), 0, rows_in_out,
               residual, weight, count, 1.0f, 1.0e-6f, out);
    }
}

}  // namespace adi_hip

using namespace adi_hip;

extern "C" {

int adi_hip_bf16_matmul(adi_hip_context *ctx, const adi_hip_bf16_matrix *m,
                        const float *inputs, uint32_t batch, float *outputs) {
    return guarded(ctx, [&] {
        require(m != nullptr && m->values != nullptr, "BF16 matrix is null");
        require(batch > 0 && m->rows > 0 && m->columns > 0, "BF16 matrix batch shape mismatch");
        require(inputs != nullptr && outputs != nullptr, "BF16 vector is null");
        launch_bf16_ordered(ctx, m->values, m->rows, m->columns, inputs, batch, outputs,
                            ctx->isa_lanes);
    });
}

int adi_hip_bf16_matvec(adi_hip_context *ctx, const adi_hip_bf16_matrix *m,
                        const float *input, float *output) {
    return adi_hip_bf16_matmul(ctx, m, input, 1, output);
}

int adi_hip_rms_norm(adi_hip_context *ctx, const float *input, const uint16_t *weight_bf16,
                     uint32_t count, uint32_t rows, float weight_offset, float epsilon,
                     float *output) {
    return guarded(ctx, [&] {
        require(count > 0 && rows > 0, "RMS norm shape mismatch");
        require(input != nullptr && weight_bf16 != nullptr && output != nullptr,
                "RMS norm vector is null");
        launch(ctx, "rms_norm", k_rms_norm<false>, dim3(rows), dim3(256), 0,
               const_cast<float *>(input), static_cast<const float *>(nullptr), weight_bf16, count,
               weight_offset, epsilon, output);
    });
}

int adi_hip_top_experts(adi_hip_context *ctx, const float *logits, uint32_t batch,
                        uint32_t experts, uint32_t *route_expert, float *route_weight) {
    return guarded(ctx, [&] {
        require(experts >= 8, "MoE routing requires at least eight experts");
        require(experts <= kMaxExperts, "MoE routing supports at most 1024 experts");
        require(batch > 0 && logits != nullptr && route_expert != nullptr &&
                    route_weight != nullptr,
                "MoE routing shape mismatch");
        launch_top_experts(ctx, logits, nullptr, batch, experts, route_expert, route_weight);
    });
}

int adi_hip_moe_route(adi_hip_context *ctx, const float *logits, const float *logit_bias,
                      uint32_t batch, uint32_t experts, uint32_t *route_expert,
                      float *route_weight, uint32_t *counts, uint32_t *offsets,
                      uint32_t *grouped_batch, uint32_t *route_to_grouped) {
    return guarded(ctx, [&] {
        require(experts >= 8, "MoE routing requires at least eight experts");
        require(experts <= kMaxExperts, "MoE routing supports at most 1024 experts");
        require(batch > 0 && logits != nullptr && route_expert != nullptr &&
                    route_weight != nullptr && counts != nullptr && offsets != nullptr &&
                    grouped_batch != nullptr && route_to_grouped != nullptr,
                "MoE routing shape mismatch");
        launch_top_experts(ctx, logits, logit_bias, batch, experts, route_expert, route_weight);
        RouteSort s{};
        s.route_expert = route_expert;
        s.positions = batch * 8u;
        s.experts = experts;
        s.counts = counts;
        s.offsets = offsets;
        s.grouped_batch = grouped_batch;
        s.route_to_grouped = route_to_grouped;
        auto &ws = ctx->workspace;
        ws.used = 0;
        ws.ensure(Workspace::round(route_sort_scratch(s.positions, experts) * 4) + 256);
        s.position_rank = ws.take<uint32_t>(s.positions);
        s.chunk_hist = ws.take<uint32_t>(route_sort_scratch(s.positions, experts) - s.positions);
        launch_route_sort(ctx, s);
    });
}

}  // extern "C"
