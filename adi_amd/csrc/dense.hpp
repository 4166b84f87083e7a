// dense.hpp -- ISA-ordered bf16 matmul and routing launchers.
#pragma once

#include "context.hpp"

namespace adi_hip {

// out[b][r] = bf16 row r . x[b] in the CPU reduction order `lanes`.
// `bias` (nullable, [rows]) is added to each result afterwards in fp32.
void launch_bf16_ordered(adi_hip_context *ctx, const uint16_t *w, uint32_t rows,
                         uint32_t columns, const float *x, uint32_t batch,
                         float *out, uint32_t lanes);

// The same with an optional extra row appended (written to out_extra [batch]).
void launch_bf16_ordered_extra(adi_hip_context *ctx, const uint16_t *w, uint32_t rows,
                               const uint16_t *w_extra, uint32_t columns, const float *x,
                               uint32_t batch, float *out, float *out_extra, uint32_t lanes);
// Two bf16 matrices of the same width over the same rows in one launch of the
// small-batch kernel (each row's chain and sum as launch_bf16_ordered forms
// them), else one launch each.
void launch_bf16_pair(adi_hip_context *ctx, const uint16_t *w0, uint32_t rows0, const uint16_t *w1,
                      uint32_t rows1, uint32_t columns, const float *x, uint32_t batch, float *out0,
                      float *out1, uint32_t lanes);
void launch_bf16_ordered_plain(adi_hip_context *ctx, const uint16_t *w, uint32_t rows,
                               uint32_t columns, const float *x, uint32_t batch, float *out,
                               uint32_t lanes);

// Top-8 routes per logit row (bias nullable, [experts]).
void launch_top_experts(adi_hip_context *ctx, const float *logits,
                        const float *bias, uint32_t batch, uint32_t experts,
                        uint32_t *route_expert, float *route_weight);

// Stable counting sort of the batch's routes (one block).
struct RouteSort {
    const uint32_t *route_expert; // [positions]
    uint32_t positions;           // batch * 8
    uint32_t experts;
    uint32_t *counts;             // [experts]
    uint32_t *offsets;            // [experts + 1]
    uint32_t *active;             // [experts] active experts ascending (nullable)
    uint32_t *active_count;       // [1] (nullable)
    uint4 *slot_info;             // [experts] {expert, first, end, 0} per active slot,
                                  // zero past the active count (nullable)
    uint32_t *position_expert;    // [positions] (nullable)
    uint32_t *grouped_batch;      // [positions]
    uint32_t *route_to_grouped;   // [positions]
    // scratch for the multi-block sort (both nullable: one block sorts)
    uint32_t *position_rank;      // [positions]
    uint32_t *chunk_hist;         // [ceil(positions / 64)][experts]
};

// Scratch words the multi-block sort needs for `positions` and `experts`.
inline size_t route_sort_scratch(size_t positions, size_t experts) {
    return positions + (positions + 63) / 64 * experts;
}
void launch_route_sort(adi_hip_context *ctx, const RouteSort &args);

// top_experts for every row plus the counting sort: one launch up to
// kRouteBatch rows, else top_experts with the chunk histograms and a one-block
// finalize that also places the positions. route_expert must be
// args.route_expert.
void launch_route(adi_hip_context *ctx, const float *logits, const float *bias, uint32_t batch,
                  uint32_t *route_expert, float *route_weight, const RouteSort &args);

// The decoder layers' norm (weight offset 1, epsilon 1e-6) of `rows` rows of
// `count`: with `residual` (nullable) each row first becomes row + residual
// in place, the residual add before the norm in one launch.
void launch_add_rms_norm(adi_hip_context *ctx, float *rows_in_out, const float *residual,
                         const uint16_t *weight, uint32_t count, uint32_t rows, float *out);

constexpr uint32_t kMaxExperts = 1024;
constexpr uint32_t kTiledBatch = 32;  // batches from which the bf16 products run register-tiled
constexpr uint32_t kTiledSmallBatch = 256;  // and up to which with 8 x 8 tiles
constexpr uint32_t kRouteBatch = 16;  // largest batch launch_route handles in one block

}  // namespace adi_hip
