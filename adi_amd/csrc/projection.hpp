// projection.hpp -- launch interfaces of the packed projection kernels, shared
// by the Backend entry points and the MoE layer.
#pragma once

#include "context.hpp"

namespace adi_hip {

// Largest vector a Hadamard prologue/epilogue block holds in LDS.
constexpr uint32_t kMaxHadamard = 8192;

// Vectors to transform in one launch: x_hat = H_n(x[src] * su). su is either
// f16 (per matrix, stride su_stride, matrix from matrix_index) or +-1 int8.
struct PrologueSegment {
    const float *x;
    const uint32_t *source_row;    // nullable: identity
    const uint32_t *matrix_index;  // nullable: matrix 0
    const uint16_t *su_f16;        // one of su_f16 / su_sign
    const int8_t *su_sign;
    uint32_t su_stride;
    float *out;
    uint32_t count;
};
struct PrologueJobs {
    PrologueSegment seg[4];
    uint32_t segments;
    uint32_t n;
    float scale;  // set by the launcher
};
bool wave_width(uint32_t n);
void launch_prologues(adi_hip_context *ctx, PrologueJobs &jobs);
template <typename Scale>
void launch_epilogue_any(adi_hip_context *ctx, const float *z, uint32_t splits,
                         size_t split_stride, uint32_t n, const Scale *sv, uint32_t vectors,
                         float *out);

// x_hat[v] = H_n(x[src(v)] * su[mat(v)]) for v < vectors.
// source_row / matrix_index may be null (identity / matrix 0).
void launch_prologue_f16(adi_hip_context *ctx, const float *x, uint32_t n,
                         const uint16_t *su, uint32_t su_stride,
                         const uint32_t *source_row, const uint32_t *matrix_index,
                         uint32_t vectors, float *out);
void launch_prologue_sign(adi_hip_context *ctx, const float *x, uint32_t n,
                          const int8_t *su, uint32_t vectors, float *out);

// y[v] = sv[mat(v)] * H_n(sum_s z[s][v]).
void launch_epilogue_f16(adi_hip_context *ctx, const float *z, uint32_t splits,
                         size_t split_stride, uint32_t n, const uint16_t *sv,
                         uint32_t sv_stride, const uint32_t *matrix_index,
                         uint32_t vectors, float *out);
void launch_epilogue_sign(adi_hip_context *ctx, const float *z, uint32_t splits,
                          size_t split_stride, uint32_t n, const int8_t *sv,
                          uint32_t vectors, float *out);

// Number of partial-sum splits the GEMV kernels write for `columns` inputs.
inline uint32_t gemv_splits(uint32_t columns) {
    const uint32_t tile_columns = columns / kTile;
    return tile_columns > 64 ? tile_columns / 64 : 1;
}

// Expert decode-GEMV over one matrix or over the active experts of a routed
// batch. Writes pre-Hadamard row sums z[split][position][rows].
struct ExpertGemv {
    const uint16_t *trellis;   // matrix 0; matrix e at e * trellis_stride words
    size_t trellis_stride;
    const uint16_t *gamma;     // f16; matrix e at e * gamma_stride
    uint32_t gamma_stride;
    const void *codebook;      // expert codebook (u16[16384][8])
    uint32_t rows;
    uint32_t columns;
    const float *x_hat;        // [positions][columns]
    float *z;                  // [splits][positions][rows]
    size_t z_split_stride;     // positions * rows
    const uint32_t *active;        // null: one matrix, tokens [0, batch)
    const uint32_t *active_count;  // device scalar
    const uint32_t *offsets;       // token range of matrix e: [offsets[e], offsets[e+1])
    uint32_t batch;
    uint32_t max_active;           // grid.y when routed
    uint32_t tokens_per_pass;      // 1 or 4
};
void launch_expert_gemv(adi_hip_context *ctx, const ExpertGemv &args);

struct NeGemv {
    const uint16_t *trellis;
    const void *codebook;   // NE signed table (u16[1024][2])
    float weight_scale;
    uint32_t rows;
    uint32_t columns;
    const float *x_hat;     // [batch][columns]
    float *z;               // [splits][batch][rows]
    size_t z_split_stride;  // batch * rows
    uint32_t batch;
};
void launch_ne_gemv(adi_hip_context *ctx, const NeGemv &args);

// Up to two expert GEMVs (routed over the same active list) and two NE GEMVs
// in one launch. The expert entries must share shape and routing; so must
// the NE entries.
struct MoeGemv {
    ExpertGemv expert[2];
    uint32_t expert_count;
    NeGemv ne[2];
    uint32_t ne_count;
    uint32_t max_active;
    uint32_t expert_blocks;  // set by the launcher
    uint32_t ne_blocks;      // set by the launcher
};
void launch_moe_gemv(adi_hip_context *ctx, MoeGemv &m, bool single_token);

void validate_expert(const adi_hip_expert_matrix *m);
void validate_ne(const adi_hip_ne_matrix *m);

}  // namespace adi_hip
