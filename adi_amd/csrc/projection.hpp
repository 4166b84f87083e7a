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
    XhatOut out;
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
// Checks the segments' alignment and sets jobs.scale (launch_prologues does
// this itself; a fused launcher calls it before its own launch).
void prepare_prologues(PrologueJobs &jobs);

// x_hat = H_n(x[src] * su) of vector v of the jobs (segments in order), by
// one wave; nothing past the last segment's vectors.
template <int VPL>
__device__ __forceinline__ void prologue_vector(const PrologueJobs &j, uint32_t v, uint32_t lane) {
#pragma clang fp contract(off)
    uint32_t s = 0;
    while (s < j.segments && v >= j.seg[s].count) {
        v -= j.seg[s].count;
        ++s;
    }
    if (s >= j.segments) {
        return;
    }
    const PrologueSegment &g = j.seg[s];
    const uint32_t n = 64u * VPL;
    const uint32_t src = g.source_row != nullptr ? g.source_row[v] : v;
    const uint32_t mat = g.matrix_index != nullptr ? g.matrix_index[v] : 0u;
    float val[VPL], su[VPL];
    load_wave<VPL>(g.x + static_cast<size_t>(src) * n, lane, val);
    if (g.su_f16 != nullptr) {
        load_wave_f16<VPL>(g.su_f16 + static_cast<size_t>(mat) * g.su_stride, lane, su);
    } else {
        load_wave_sign<VPL>(g.su_sign, lane, su);
    }
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
        val[i] = val[i] * su[i];
    }
    wave_hadamard<VPL>(val, j.scale, lane);
    store_xhat<VPL>(g.out, v, lane, val);
}
// y = sv * H_n(sum over splits of z). z is scratch: for a few vectors over
// several slices the launch first adds the slices into slice 0, in place.
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

// Groups of 16 tiles in one GEMV wave item (all in one tile row when the
// matrix has at least 16 tile columns).
__host__ __device__ inline uint32_t item_groups(uint32_t tile_columns) {
    return tile_columns >= 64 ? 4u : (tile_columns >= 32 ? 2u : 1u);
}
// Column ranges a tile row is cut into by the wave items.
__host__ __device__ inline uint32_t item_segments(uint32_t tile_columns) {
    const uint32_t span = 16u * item_groups(tile_columns);
    return tile_columns >= span ? tile_columns / span : 1u;
}
// Partial-sum slices of Z the GEMV writes for a matrix with `columns` inputs:
// one per (column range, codebook plane) for the expert codec, one per range
// of 16 tile columns for the NE codec. Slice s of position p, row r is at
// z[s * split_stride + p * rows + r].
inline uint32_t expert_splits(uint32_t columns) { return 2u * item_segments(columns / kTile); }
inline uint32_t ne_splits(uint32_t columns) {
    return columns / kTile > 16u ? columns / kTile / 16u : 1u;  // NE items are 16 tiles
}

// An expert matrix for the GEMV: one matrix (positions [0, batch)), or the
// routed experts of a batch, whose slots come from the MoeGemv slot table
// (matrix e at e * trellis_stride words / e * gamma_stride).
struct ExpertGemv {
    const uint16_t *trellis;
    size_t trellis_stride;
    const uint16_t *gamma;         // f16 wave gammas
    uint32_t gamma_stride;
    uint32_t rows;
    uint32_t columns;
    const float *x_hat;            // [positions][columns]
    float *z;                      // [expert_splits][positions][rows]
    size_t z_split_stride;         // positions * rows
    uint32_t batch;                // positions of a single matrix
    // geometry, set by the launcher
    uint32_t tile_rows;
    uint32_t tc_shift;             // log2(tile columns)
    uint32_t group_shift;          // log2(groups of 16 tiles per item)
};

struct NeGemv {
    const uint16_t *trellis;
    float weight_scale;
    uint32_t rows;
    uint32_t columns;
    const float *x_hat;     // [batch][columns]
    float *z;               // [ne_splits][batch][rows]
    size_t z_split_stride;  // batch * rows
    uint32_t batch;
    // geometry, set by the launcher
    uint32_t tile_rows;
    uint32_t tc_shift;      // log2(tile columns)
};

// One row's SwiGLU, for a down-projection GEMV that builds its own x_hat:
// x_hat = H(su_down * silu(sv_gate * H(sum z_gate)) * (sv_up * H(sum z_up)))
// of the routed slot's grouped row (f16 scales of its expert) and of the
// shared expert (+-1 scales), width 512.
struct GemvSwiglu {
    const float *z_gate;        // [splits][rows][512] by grouped row
    const float *z_up;
    size_t split_stride;
    uint32_t splits;
    const uint16_t *sv_gate;    // [experts][512] f16
    const uint16_t *sv_up;
    const uint16_t *su_down;
    const float *shared_z_gate; // [shared_splits][1][512]
    const float *shared_z_up;
    size_t shared_split_stride;
    uint32_t shared_splits;
    const int8_t *shared_sv_gate;
    const int8_t *shared_sv_up;
    const int8_t *shared_su_down;
    float scale;                // 1 / sqrt(512)
};
constexpr uint32_t kFusedSwigluWidth = 512;

// Up to two expert GEMVs (same shape and routing, one codebook) and two NE
// GEMVs (same shape, one codebook) in one persistent launch.
struct MoeGemv {
    ExpertGemv expert[2];
    uint32_t expert_count;
    NeGemv ne[2];
    uint32_t ne_count;
    const void *expert_book;  // expert codebook planes
    const void *ne_book;      // NE signed table
    const uint4 *slot_info;   // [max_active] {expert, first, end, 0}; null: one matrix
    uint32_t max_active;      // routed slots per expert entry (1 for a single matrix)
    // nonzero: one row, one expert item per wave at most; x_hat of the expert
    // and NE entries comes from `swiglu` (their x_hat pointers are unused)
    uint32_t fused_swiglu;
    GemvSwiglu swiglu;
    // set by the launcher
    uint32_t slot_capacity;
    uint32_t expert_items_per_slot;  // a power of two
    uint32_t item_shift;             // its log2
    uint32_t expert_items;
    uint32_t ne_items_per_matrix;
    uint32_t ne_items;
    uint32_t half_items[2];
};
void launch_trellis_gemv(adi_hip_context *ctx, MoeGemv &m);

// The MoE block of one row in one persistent launch, for decode
// (src/executor.cpp:242-330): router and top-8, the shared expert's
// prologues, the routed and shared gate/up, the SwiGLUs, the down projections
// and the route-order combine, one block per CU. Data passes between blocks
// through device-coherent accesses and counters in `sync` (bounded waits; a
// wait that runs out sets the error word). gu and dn are the plans of the
// separate gate/up and down launches (same buffers, same slices), so the
// arithmetic is the separate launches' exactly.
struct MoeDecodeOne {
    MoeGemv gu;                       // routed gate/up (entries 0, 1), shared gate/up (NE 0, 1)
    MoeGemv dn;                       // routed down (entry 0), shared down (NE 0); dn.swiglu set
    const uint16_t *router;           // [experts][hidden] bf16
    const uint16_t *shared_gate_row;  // [hidden] bf16
    const float *logit_bias;          // [experts] or null
    const float *x;                   // [hidden]
    const uint16_t *su_gate;          // [experts][hidden] f16
    const uint16_t *su_up;
    const int8_t *shared_su_gate;     // [hidden] +-1
    const int8_t *shared_su_up;
    const uint16_t *sv_down;          // [experts][hidden] f16
    const int8_t *shared_sv_down;     // [hidden] +-1
    float scale_hidden;               // 1 / sqrt(hidden)
    float *out;                       // [hidden]
    uint32_t *route_expert_out;       // [8] or null
    float *route_weight_out;          // [8] or null
    uint32_t *sync;                   // kMoeSyncWords words, zero between calls (but the error word)
    uint32_t experts;
    // set by plan_moe_decode_one
    uint32_t expect_slot;             // gate/up wave items per routed slot
    uint32_t expect_down;             // down wave items per routed slot
    uint32_t down_splits;             // Z slices of the routed and shared down projections
    uint32_t shared_down_splits;
};
// Fills the plans; false when the shapes or the device do not fit the launch
// (hidden 2048, expert hidden 512, at most 256 experts, 256 CUs, the ISA
// order of 8 or 16 lanes). The caller then runs the separate launches.
bool plan_moe_decode_one(adi_hip_context *ctx, MoeDecodeOne &a);
void launch_moe_decode_one(adi_hip_context *ctx, const MoeDecodeOne &a);
// The MoE block of 2 to kFewMaxRows rows in one persistent launch
// (src/executor.cpp:242-330 for each row): router and top-8 of every row,
// the expert-sorted slots, the routed and shared gate/up, the SwiGLUs, the
// down projections and the route-order combine, one block per CU, with the
// separate launches' arithmetic (decode-GEMV items, one-wave combine rows),
// so results are bit-identical to theirs. Routed slot s runs on XCD s % 8.
// Data passes between blocks through device-coherent accesses and counters
// from `sync` (bounded waits; a wait that runs out sets the error word).
constexpr uint32_t kFusedHidden = 2048;     // hidden width of the one-launch MoE blocks
constexpr uint32_t kFusedMaxExperts = 256;  // routed experts they handle
// Up to 12 rows: from there the MFMA grouped GEMMs (16 rows: 148.7 against
// 164.8 us a layer) overtake the decode-GEMV items this launch runs.
constexpr uint32_t kFewMaxRows = 12;
constexpr uint32_t kFewMaxRoutes = 8 * kFewMaxRows;
// tile groups of a gate/up and of a down item in that launch (item_groups of
// 2048 and 512 columns)
constexpr uint32_t kFewGuGroups = 4, kFewDnGroups = 2;
struct MoeDecodeFew {
    MoeGemv gu;                       // routed gate/up (entries 0, 1), shared gate/up (NE 0, 1)
    MoeGemv dn;                       // routed down (entry 0), shared down (NE 0); dn.swiglu set
    const uint16_t *router;           // [experts][hidden] bf16
    const uint16_t *shared_gate_row;  // [hidden] bf16
    const float *logit_bias;          // [experts] or null
    const float *x;                   // [batch][hidden]
    const uint16_t *su_gate;          // [experts][hidden] f16
    const uint16_t *su_up;
    const int8_t *shared_su_gate;     // [hidden] +-1
    const int8_t *shared_su_up;
    const uint16_t *sv_down;          // [experts][hidden] f16
    const int8_t *shared_sv_down;     // [hidden] +-1
    float scale_hidden;               // 1 / sqrt(hidden)
    float *out;                       // [batch][hidden]
    uint32_t *route_expert_out;       // [batch * 8] or null
    float *route_weight_out;
    float *logits;                    // [batch][experts + 1]: router logits, then the shared gate's
    float *parts;                     // [batch][9][hidden]: the combine rows
    uint32_t *sync;                   // the counters (zero between calls)
    uint32_t *error;                  // the error word
    uint32_t experts;
    uint32_t batch;
    // set by plan_moe_decode_few
    uint32_t expect_gu;               // gate/up wave items per routed slot (both planes)
    uint32_t expect_dn;               // down wave items per routed slot
    uint32_t down_splits;             // Z slices of the routed and shared down projections
    uint32_t shared_down_splits;
};
// Fills the plans; false when the shapes or the device do not fit the launch
// (hidden 2048, expert hidden 512, at most 256 experts, 2 to kFewMaxRows rows,
// 256 CUs, the ISA order of 8 or 16 lanes).
bool plan_moe_decode_few(adi_hip_context *ctx, MoeDecodeFew &a);
void launch_moe_decode_few(adi_hip_context *ctx, const MoeDecodeFew &a);
// One-launch NE projection of up to kNeFusedRows input rows (k_ne_fused):
// x_hat, the NE items of whole tile rows per block with the slice-order sum
// in LDS, and the row transform by the block that takes the last ticket. One
// launch carries up to kNeFusedJobs matrices of the same column count over the
// same input rows (a layer's query, key and value), each on blocks of its own.
constexpr uint32_t kNeFusedRows = 4;
constexpr uint32_t kNeFusedThreads = 512;
constexpr uint32_t kNeFusedMaxItems = 32;  // NE items of one tile row at 8192 columns
constexpr uint32_t kNeFusedJobs = 3;
constexpr uint32_t kNeFusedMaxRows = 8192;
struct NeFusedJob {
    const uint16_t *trellis;
    const int8_t *su;
    const int8_t *sv;
    const uint32_t *table;  // the 4 KiB signed table
    float *zsum;            // [batch][rows]: the slice-order sums
    float *out;             // [batch][rows]
    float weight_scale, scale_rows;
    uint32_t rows;          // 512, 2048, 4096 or 8192
    uint32_t first_block;   // the job's blocks within a half: first_block .. first_block + blocks - 1
    uint32_t blocks;
    // optional, rows 2048: then tail_row += out and tail_out = rms_norm(tail_row)
    float *tail_row;        // [batch][rows], or null
    const uint16_t *tail_weight;
    float *tail_out;
};
struct NeFused {
    NeFusedJob job[kNeFusedJobs];
    uint32_t jobs;
    const float *x;         // [batch][columns], unless norm_row is set
    // optional, columns 2048: x = rms_norm(norm_row + norm_add), computed by
    // every block for its rows; the first block of each half writes them to
    // x_out, and the last block through writes norm_row + norm_add back
    float *norm_row;        // [batch][columns], or null
    const float *norm_add;  // or null (then norm_row is left as it is)
    const uint16_t *norm_weight;
    float *x_out;
    uint32_t *ticket;       // word 32 * (2 * job + half) per job and half, and word 256 for the
                            // whole grid; zero between launches (the block that takes one last clears it)
    float scale_columns;
    uint32_t batch;
    uint32_t halves;        // 1, or 2 when the grid splits the input rows in two
};
// A decoder layer's RMS norms (weight offset 1, epsilon 1e-6, src/kernels.cpp:
// 1052-1073) folded into its projections. NeNormIn: the projections' input is
// rms_norm(row + add), with row += add written back (add may be null) and
// the normalized rows written to out. NeNormTail: after the projection,
// row += y and out = rms_norm(row).
struct NeNormIn {
    float *row;
    const float *add;
    const uint16_t *weight;
    float *out;
};
struct NeNormTail {
    float *row;
    const uint16_t *weight;
    float *out;
};
// Runs m[0 .. count - 1] on the same `batch` input rows in one launch, output
// j to outputs[j]; false (nothing launched) when a shape is not one the kernel
// is built for (columns 2048 or 4096, the same for all; rows 512, 2048, 4096
// or 8192; at most kNeFusedRows input rows and kNeFusedJobs matrices; 2048
// columns with `in`, 2048 rows of matrix 0 with `tail`). With `in` the
// inputs are its normalized rows (`inputs` unused); `tail` applies to
// matrix 0. `zsum` holds batch x (the sum of the rows) floats.
bool launch_ne_fused(adi_hip_context *ctx, const adi_hip_ne_matrix *const *m, uint32_t count,
                     const float *inputs, uint32_t batch, float *const *outputs, float *zsum,
                     const NeNormIn *in = nullptr, const NeNormTail *tail = nullptr);
// NE projections of the same input rows, outputs[j] = m[j] x inputs (or x
// the normalized rows of `in`), then `tail` on matrix 0's outputs: one
// launch for a few rows where launch_ne_fused takes the shapes, else the
// norm launches and one adi_hip_ne_matmul each. Throws on a rejected call.
void ne_matmul_group(adi_hip_context *ctx, const adi_hip_ne_matrix *const *m, uint32_t count,
                     const float *inputs, uint32_t batch, float *const *outputs,
                     const NeNormIn *in = nullptr, const NeNormTail *tail = nullptr);
// Whether `m` (a down projection of one row) can build its x_hat from
// m.swiglu in the launch: one expert entry of width 512 and at most one
// expert item per wave.
bool trellis_gemv_can_fuse_swiglu(adi_hip_context *ctx, MoeGemv m);

void validate_expert(const adi_hip_expert_matrix *m);
void validate_ne(const adi_hip_ne_matrix *m);

}  // namespace adi_hip
