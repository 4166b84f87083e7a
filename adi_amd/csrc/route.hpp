// route.hpp -- top_experts and the one-block counting sort of the MoE
// routing as device functions, shared by the routing kernels and the fused
// batch-1 routing + prologue launch.
#pragma once

#include "dense.hpp"

namespace adi_hip {

// Order of route values: the float's bits mapped to an unsigned order, larger
// floats to larger words, with -0 folded into +0 (which compares equal to it).
__device__ __forceinline__ uint32_t route_order(float value) {
    const uint32_t bits = __float_as_uint(value + 0.0f);
    return (bits & 0x80000000u) ? ~bits : (bits | 0x80000000u);
}

__device__ __forceinline__ float route_order_value(uint32_t ordered) {
    return __uint_as_float((ordered & 0x80000000u) ? (ordered & 0x7FFFFFFFu) : ~ordered);
}

// One wave per logit row. Lane l holds experts l, l+64, ...; eight rounds of
// a wave-wide maximum of the ordered values, each followed by ballots for the
// lowest expert holding it, pick the routes in the order of the comparator of
// top_experts: larger logit first, lower index on ties (src/executor.cpp:
// 202-211). Order 0 marks an empty or chosen slot; a live value's order is at
// least 1 (only the negative NaNs 0xFFFFFFFF and 0xFFFFFFFE share order 1). The softmax over the eight then runs on lane 0 in the reference's
// order (src/executor.cpp:213-227) when route_expert is set. `chosen` (when
// set) receives the eight experts in every lane.
template <int SLOTS>
__device__ __forceinline__ void top8_wave(const float *__restrict__ row,
                                          const float *__restrict__ bias, uint32_t experts,
                                          uint32_t lane, uint32_t *__restrict__ route_expert,
                                          float *__restrict__ route_weight,
                                          uint32_t *local_expert = nullptr,
                                          uint32_t *chosen = nullptr) {
#pragma clang fp contract(off)
    float value[SLOTS], offset[SLOTS];
    // unguarded loads of clamped indexes, so all of them are in flight at once
#pragma unroll
    for (uint32_t i = 0; i < SLOTS; ++i) {
        const uint32_t e = min(lane + 64u * i, experts - 1u);
        value[i] = row[e];
        offset[i] = bias != nullptr ? bias[e] : 0.0f;
    }
    uint32_t order[SLOTS];
#pragma unroll
    for (uint32_t i = 0; i < SLOTS; ++i) {
        const float v = bias != nullptr ? value[i] + offset[i] : value[i];
        order[i] = lane + 64u * i < experts ? max(route_order(v), 1u) : 0u;
    }
    float chosen_value[8];
    uint32_t chosen_index[8];
    for (int round = 0; round < 8; ++round) {
        uint32_t best = order[0];
#pragma unroll
        for (uint32_t i = 1; i < SLOTS; ++i) {
            best = max(best, order[i]);
        }
        best = max(best, lane_xor_bits<1>(best));
        best = max(best, lane_xor_bits<2>(best));
        best = max(best, lane_xor_bits<4>(best));
        best = max(best, lane_xor_bits<8>(best));
        best = max(best, lane_xor_bits<16>(best));
        best = max(best, lane_xor_bits<32>(best));
        best = __builtin_amdgcn_readfirstlane(best);
        // the lowest expert holding the maximum: slot i covers experts
        // 64i .. 64i + 63, so the last slot with a vote, counting down, decides
        uint64_t votes[SLOTS];
#pragma unroll
        for (uint32_t i = 0; i < SLOTS; ++i) {
            votes[i] = __ballot(order[i] == best);
        }
        uint32_t index = 0u;
#pragma unroll
        for (int i = SLOTS - 1; i >= 0; --i) {
            index = votes[i] != 0ull ? 64u * i + static_cast<uint32_t>(__builtin_ctzll(votes[i])) : index;
        }
        chosen_value[round] = route_order_value(best);
        chosen_index[round] = index;
#pragma unroll
        for (uint32_t i = 0; i < SLOTS; ++i) {
            order[i] = lane + 64u * i == index ? 0u : order[i];
        }
    }
    if (chosen != nullptr) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            chosen[i] = chosen_index[i];
        }
    }
    if (lane == 0 && route_expert != nullptr) {
        const float maximum = chosen_value[0];
        float selected[8];
        float sum = 0.0f;
        for (int i = 0; i < 8; ++i) {
            selected[i] = expf(chosen_value[i] - maximum);
            sum = sum + selected[i];
        }
        sum = fmaxf(sum, 6.103515625e-5f);
        for (int i = 0; i < 8; ++i) {
            route_expert[i] = chosen_index[i];
            route_weight[i] = selected[i] / sum;
            if (local_expert != nullptr) {
                local_expert[i] = chosen_index[i];
            }
        }
    }
}

// Counting sort of moe_forward_batch (src/executor.cpp:1235-1258) in one
// wave: counts by LDS integer atomics, an exclusive scan for offsets, then the
// (token, route) slots are placed 64 at a time in order; lanes that share an
// expert in a chunk find their rank among earlier lanes with ballots, so each
// expert's cursor advances exactly as the sequential loop's does.
// `route_expert` is a.route_expert or a copy of it in LDS.
__device__ __forceinline__ void route_sort_block(const RouteSort &a,
                                                 const uint32_t *route_expert,
                                                 uint32_t *counts, uint32_t *cursor) {
    for (uint32_t e = threadIdx.x; e < a.experts; e += blockDim.x) {
        counts[e] = 0u;
    }
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < a.positions; i += blockDim.x) {
        atomicAdd(&counts[route_expert[i]], 1u);
    }
    __syncthreads();
    if (threadIdx.x >= 64) {
        return;  // the scan and the ordered scatter run on wave 0
    }
    const uint32_t lane = threadIdx.x;
    // exclusive scan over experts: each lane owns a contiguous run
    const uint32_t per_lane = (a.experts + 63u) / 64u;
    const uint32_t first = lane * per_lane;
    uint32_t local = 0;
    for (uint32_t e = first; e < first + per_lane && e < a.experts; ++e) {
        local += counts[e];
    }
    uint32_t inclusive = local;
    for (int offset = 1; offset < 64; offset <<= 1) {
        const uint32_t other = static_cast<uint32_t>(__shfl_up(static_cast<int>(inclusive), offset));
        if (lane >= static_cast<uint32_t>(offset)) {
            inclusive += other;
        }
    }
    uint32_t running = inclusive - local;
    for (uint32_t e = first; e < first + per_lane && e < a.experts; ++e) {
        cursor[e] = running;
        a.offsets[e] = running;
        a.counts[e] = counts[e];
        if (a.position_expert != nullptr) {
            for (uint32_t p = running; p < running + counts[e]; ++p) {
                a.position_expert[p] = e;
            }
        }
        running += counts[e];
    }
    if (lane == 63) {
        a.offsets[a.experts] = inclusive;
    }
    // ascending list of active experts
    if (a.active != nullptr) {
        uint32_t base = 0;
        for (uint32_t e0 = 0; e0 < a.experts; e0 += 64u) {
            const uint32_t e = e0 + lane;
            const bool on = e < a.experts && counts[e] != 0u;
            const uint64_t mask = __ballot(on);
            if (on) {
                const uint32_t s = base + __popcll(mask & ((1ull << lane) - 1ull));
                a.active[s] = e;
                if (a.slot_info != nullptr) {
                    a.slot_info[s] = make_uint4(e, cursor[e], cursor[e] + counts[e], 0u);
                }
            }
            base += __popcll(mask);
        }
        if (a.slot_info != nullptr) {
            for (uint32_t s = base + lane; s < a.experts; s += 64u) {
                a.slot_info[s] = make_uint4(0u, 0u, 0u, 0u);
            }
        }
        if (lane == 0 && a.active_count != nullptr) {
            *a.active_count = base;
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_wave_barrier();
    const uint64_t below = (1ull << lane) - 1ull;
    for (uint32_t c = 0; c < a.positions; c += 64u) {
        const uint32_t i = c + lane;
        const bool valid = i < a.positions;
        const uint32_t e = valid ? route_expert[i] : 0u;
        uint64_t peers = __ballot(valid);
        if (!valid) {
            peers = ~peers;
        }
        for (uint32_t bit = 0; bit < 10u; ++bit) {
            const bool set = (e >> bit) & 1u;
            const uint64_t vote = __ballot(set);
            peers &= set ? vote : ~vote;
        }
        const uint32_t rank = __popcll(peers & below);
        const uint32_t total = __popcll(peers);
        uint32_t position = 0;
        if (valid) {
            position = cursor[e] + rank;
        }
        // every lane has read its cursor before any lane advances one
        __builtin_amdgcn_wave_barrier();
        if (valid) {
            a.grouped_batch[position] = i / 8u;
            a.route_to_grouped[i] = position;
            if (rank == 0) {
                cursor[e] += total;
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        __builtin_amdgcn_wave_barrier();
    }
}

}  // namespace adi_hip
