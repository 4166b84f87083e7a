// attention.hpp -- the decoder layer for the model-level entry points.
#pragma once

#include "context.hpp"

namespace adi_hip {

// One decode token of each of `rows` sequences through one decoder layer on
// hidden[rows][moe.hidden]: row r is at positions[r] of the sequence whose
// state for this layer is states[r] (decode_batch's layer step,
// src/executor.cpp:1620-1811). The kernels read the positions from
// device_positions (the same values); the launches cover positions below
// `span` (0: the largest positions[r] + 1), so a captured step replays
// correctly at any positions below it. `pending` (nullable) holds the
// previous layer's MoE rows, added to hidden first; this layer's MoE rows go
// to moe_out (may be `pending`), left for the next layer's first norm or the
// final norm to add.
void decoder_rows(adi_hip_context *ctx, const adi_hip_decoder_layer *L, uint32_t rows,
                  float *hidden, const float *pending, float *moe_out,
                  const adi_hip_layer_state *const *states, const uint32_t *positions,
                  const uint32_t *device_positions, uint32_t span);

// `count` consecutive tokens of one sequence at positions position ..
// position + count - 1 through one decoder layer (the layer step of prefill,
// src/executor.cpp:1869-2058) on hidden[count][moe.hidden], pending and
// moe_out as decoder_rows'.
void prefill_chunk(adi_hip_context *ctx, const adi_hip_decoder_layer *L, uint32_t position,
                   uint32_t count, float *hidden, const float *pending, float *moe_out,
                   const adi_hip_layer_state *state);

}  // namespace adi_hip
