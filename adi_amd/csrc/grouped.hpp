// grouped.hpp -- MFMA grouped GEMMs over expert-sorted positions (prefill
// microbatches): the trellis codes are decoded into the MFMA A operand in
// registers and multiplied with x_hat held as f16 hi/lo pairs.
#pragma once

#include "context.hpp"

namespace adi_hip {

// Batches from which the MoE block runs its projections as MFMA GEMMs
// instead of the decode-GEMV (the 256-expert layer at 8 rows: 111 against
// 122 us, at 16 rows 154 against 189, at 32 rows 203 against 308), and from
// which a single expert or NE projection does: an NE matrix from 8 rows
// (MFMA 2048 x 2048: 22.8 us at 8 rows and 22.9 at 16, against 30.3 and 31.4
// for the GEMV, which decodes per row), an expert matrix from 16 (512 x
// 2048: 35.8 against 39.8 us; 27.0 against 35.3 at 8).
constexpr uint32_t kMfmaBatch = 8;
constexpr uint32_t kNeMfmaBatch = 8;
constexpr uint32_t kExpertMfmaBatch = 16;

// Widest expert matrix the MFMA GEMM takes, in 16-column tiles (its per-wave
// gamma rows live in LDS).
constexpr uint32_t kMaxTileColumns = 256;

inline bool expert_mfma_supports(uint32_t rows, uint32_t columns) {
    return rows >= 16 && columns >= 64 && columns / 16 <= kMaxTileColumns;
}

// One expert projection over the routed slots: Z[plane][p][r] for the
// positions p of each active slot (x_hat in the codebook-plane order of
// XhatOut, planes 2).
struct ExpertMfma {
    const uint16_t *trellis;  // matrix e at e * trellis_stride words
    size_t trellis_stride;
    const uint16_t *gamma;    // f16 wave gammas, matrix e at e * gamma_stride
    uint32_t gamma_stride;
    uint32_t rows;
    uint32_t columns;
    const uint16_t *x_hi;     // [2][positions][columns/2] f16
    const uint16_t *x_lo;
    uint32_t positions;
    float *z;                 // [2][positions][rows]
    size_t z_split_stride;    // positions * rows
    // geometry, set by the launcher
    uint32_t tile_rows;
    uint32_t tc_shift;
};

// One NE projection: Z[p][r] for p < batch (x_hat in column order, planes 1).
struct NeMfma {
    const uint16_t *trellis;
    float weight_scale;
    uint32_t rows;
    uint32_t columns;
    const uint16_t *x_hi;  // [batch][columns] f16
    const uint16_t *x_lo;
    uint32_t batch;
    float *z;              // [k_slices][batch][rows]
    // geometry, set by the launcher
    uint32_t tile_rows;
    uint32_t tc_shift;
};

// Up to two expert projections (same shape, routing and codebook) in one
// persistent launch.
struct ExpertMfmaJobs {
    ExpertMfma expert[2];
    uint32_t expert_count;
    const void *expert_book;   // codebook planes
    const uint4 *slot_info;    // [max_active] {expert, first, end, 0}
    uint32_t max_active;
    uint32_t max_positions;    // bound on the positions of one slot (the batch)
    // set by the launcher
    uint32_t row_groups;
    uint32_t position_groups;
    uint32_t items;            // per plane
};

struct NeMfmaJobs {
    NeMfma ne[2];
    uint32_t ne_count;
    const void *ne_book;  // NE signed table
    // set by the launcher
    uint32_t row_groups;
    uint32_t position_groups;
    uint32_t k_slices;    // the K range is cut into this many slices of Z
    uint32_t items;
};

// Z slices the NE MFMA GEMM writes for a projection of `rows` x `columns` at
// `batch` positions (enough items to fill the GPU; the consumer adds them).
uint32_t ne_mfma_slices(uint32_t rows, uint32_t columns, uint32_t batch);

void launch_expert_mfma(adi_hip_context *ctx, ExpertMfmaJobs &jobs);
void launch_ne_mfma(adi_hip_context *ctx, NeMfmaJobs &jobs);

}  // namespace adi_hip
