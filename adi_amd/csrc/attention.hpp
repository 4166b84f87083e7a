// attention.hpp -- the decoder layer for the model-level entry points.
#pragma once

#include "context.hpp"

namespace adi_hip {

// One decode token of each of `rows` sequences through one decoder layer, in
// place on hidden[rows][moe.hidden]: row r is at positions[r] of the sequence
// whose state for this layer is states[r] (decode_batch's layer step,
// src/executor.cpp:1620-1811).
void decoder_rows(adi_hip_context *ctx, const adi_hip_decoder_layer *L, uint32_t rows,
                  float *hidden, const adi_hip_layer_state *const *states,
                  const uint32_t *positions);

// `count` consecutive tokens of one sequence at positions position ..
// position + count - 1 through one decoder layer (the layer step of prefill,
// src/executor.cpp:1869-2058), in place on hidden[count][moe.hidden].
void prefill_chunk(adi_hip_context *ctx, const adi_hip_decoder_layer *L, uint32_t position,
                   uint32_t count, float *hidden, const adi_hip_layer_state *state);

}  // namespace adi_hip
