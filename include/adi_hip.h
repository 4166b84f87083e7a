/*
 * adi_hip.h -- C ABI of the MI355X (gfx950) packed-weight hot path of ADI.
 *
 * This is the drop-in boundary for ADI's backend op table. The reference
 * evaluates every packed projection through `struct adi::Backend`
 * (include/adi/backend.hpp:10-23), a table of C++ function pointers over
 * std::span host views, and its MoE glue lives in the executor
 * (src/executor.cpp:188-330, 1181-1453). Each entry point below replaces one of
 * those, taking plain pointers and sizes:
 *
 *   * matrix descriptors hold DEVICE pointers to the packed data, which stays
 *     packed in HBM and is decoded inside the kernels;
 *   * activations are DEVICE pointers owned by the caller;
 *   * every call is asynchronous on the context's HIP stream;
 *   * no call throws: each returns an ADI_HIP_* status, and
 *     adi_hip_last_error() gives the message. The reference throws
 *     std::invalid_argument for the same shape violations
 *     (src/kernels.cpp:393-408, 504-521, 606-620, 719-735, 855-862,
 *     988-1016); the C++ backend shim maps statuses back to exceptions.
 *
 * Calls on one context are serialised by the caller (one context per host
 * thread, or external locking); contexts are independent.
 */
#ifndef ADI_HIP_H
#define ADI_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes. */
#define ADI_HIP_OK 0
#define ADI_HIP_INVALID_ARGUMENT (-1) /* reference: std::invalid_argument */
#define ADI_HIP_OUT_OF_MEMORY (-2)
#define ADI_HIP_DEVICE_ERROR (-3)     /* a HIP runtime call failed */
#define ADI_HIP_OUT_OF_RANGE (-4)     /* reference: std::out_of_range */

typedef struct adi_hip_context adi_hip_context;
typedef struct adi_hip_codebook adi_hip_codebook;

/* ---- context ------------------------------------------------------------ */

/* Creates a context on `device` (HIP ordinal). Replaces cpu_backend()
 * (src/backend.cpp:11-26): one context is one backend instance. */
int adi_hip_context_create(int device, adi_hip_context **out);
void adi_hip_context_destroy(adi_hip_context *ctx);

/* Message of the last failed call on this context ("" if none). A NULL
 * context gives the message of the last failed adi_hip_context_create. */
const char *adi_hip_last_error(const adi_hip_context *ctx);

/* Stream the context launches on (a hipStream_t; NULL = the null stream). */
int adi_hip_set_stream(adi_hip_context *ctx, void *stream);
int adi_hip_synchronize(adi_hip_context *ctx);

/* CPU reduction order the ISA-ordered bf16 dot reproduces, so that router
 * logits, and therefore routes, are bit-identical with the CPU build:
 * 1 = scalar, 8 = AVX2 lanes, 16 = AVX-512 lanes with fused multiply-add
 * (src/simd.cpp:88-96, src/simd_x86_avx2.cpp:172-193,
 * src/simd_x86_avx512.cpp:109-130; ADI_CPU_ISA selects it there,
 * src/simd.cpp:298-342). Default 16. */
int adi_hip_set_reduction_isa(adi_hip_context *ctx, uint32_t lanes);

/* Whether decode-size calls run as one launch (enabled 1, the default) or
 * as the separate launches (0): adi_hip_moe_forward on 1 to 12 rows (router,
 * routing, both projections of every route, shared expert and combine in
 * one persistent launch) and adi_hip_ne_matmul on up to 4 rows of the shapes
 * it is built for (x_hat, the NE items and the output transform in one
 * launch); in a decoder layer of 1 to 4 tokens, its RMS norms inside the
 * projection launches; and for one token per sequence the Gated DeltaNet
 * core (alpha/beta, convolution, delta rule, gated norm) and the full
 * attention core (query/key norm and rotation, flash-decoding, split merge)
 * as one launch each. All of these give results bit-identical to the
 * separate launches. The one-launch MoE block of 2 to 12 rows runs the decode-GEMV
 * arithmetic; the separate launches take the MFMA GEMMs from 8 rows, except
 * with enabled 2 (separate launches, decode-GEMV up to 16 rows), which gives
 * results bit-identical to the one-launch block at every batch it runs; at
 * 1 to 7 rows, 0 and 2 are the same. No counterpart in the reference (a tuning
 * switch of this backend). A cross-block wait of a one-launch MoE block
 * that runs out (only possible when other work keeps some of its blocks off
 * the GPU) is reported by the next adi_hip_synchronize. */
int adi_hip_set_fused_decode(adi_hip_context *ctx, int enabled);

/* Caps each of the context's grow-on-demand scratch arenas at `bytes`
 * (default SIZE_MAX); arenas already larger stay as they are. A call whose
 * plan needs a larger arena fails with ADI_HIP_OUT_OF_MEMORY where the plan
 * is made, before that arena is freed or regrown. The projection, router,
 * routing, MoE and head entries plan before they launch anything, so their
 * outputs are untouched; a layer entry may already have run some of its
 * steps, as the reference's layer has when one of its steps throws. No
 * counterpart in the reference, whose scratch is host vectors: it bounds
 * device memory in a server and lets a caller force the allocation-failure
 * path from the host. */
int adi_hip_set_workspace_limit(adi_hip_context *ctx, size_t bytes);

/* ---- device memory -------------------------------------------------------- */

/* Device buffers for callers that build descriptors without the HIP runtime
 * (a host-compiled Backend shim). No reference counterpart: the reference's
 * matrices are views into the mmap (include/adi/kernels.hpp:9-77), which
 * this library copies to HBM once. Copies are synchronous on the context's
 * stream. */
int adi_hip_device_alloc(adi_hip_context *ctx, size_t bytes, void **out);
void adi_hip_device_free(adi_hip_context *ctx, void *pointer);
int adi_hip_copy_to_device(adi_hip_context *ctx, void *device, const void *host, size_t bytes);
int adi_hip_copy_to_host(adi_hip_context *ctx, void *host, const void *device, size_t bytes);

/* ---- codebooks ------------------------------------------------------------ */

/* Model-wide decoded-state tables, built once from the host TLUT and kept in
 * HBM as f16 (exact: the reference rounds every lattice value through f16,
 * src/codec_cache.cpp:27-29, 33-115). Replace the ExpertScratch caches and
 * MachModel::cache_descriptors (src/kernels.cpp:33-94, src/model.cpp:549-551).
 *   expert: tlut 32768x8 f32 -> the 16384 reachable rows x 8 f16 (256 KiB,
 *           two planes of components 0-3 and 4-7; state s selects row
 *           (s*(s+1) mod 2^15)/2, always even);
 *   ne:     tlut 512x2 f32 -> the 1024x2 signed table (4 KiB). */
int adi_hip_codebook_create_expert(adi_hip_context *ctx, const float *tlut_host,
                                   adi_hip_codebook **out);
int adi_hip_codebook_create_ne(adi_hip_context *ctx, const float *tlut_host,
                               adi_hip_codebook **out);
void adi_hip_codebook_destroy(adi_hip_codebook *codebook);

/* ---- matrix descriptors (all pointers are device pointers) --------------- */

/* adi::MachExpertMatrix (include/adi/kernels.hpp:9-20). */
typedef struct {
    uint32_t rows;
    uint32_t columns;
    const uint16_t *trellis;        /* (rows/16)*(columns/16)*24 u16 words */
    const uint16_t *su_f16;         /* columns */
    const uint16_t *sv_f16;         /* rows */
    const uint16_t *wave_gamma_f16; /* rows/16 + columns/16 */
    const adi_hip_codebook *codebook; /* expert codebook */
} adi_hip_expert_matrix;

/* adi::MachNeMatrix (include/adi/kernels.hpp:42-52). */
typedef struct {
    uint32_t rows;
    uint32_t columns;
    const uint16_t *trellis; /* (rows/16)*(columns/16)*64 u16 words */
    const int8_t *su;        /* columns, +-1 */
    const int8_t *sv;        /* rows, +-1 */
    float weight_scale;
    const adi_hip_codebook *codebook; /* NE codebook */
} adi_hip_ne_matrix;

/* adi::MachHeadChunk (include/adi/kernels.hpp:64-71). */
typedef struct {
    uint32_t rows;
    uint32_t columns;
    const uint8_t *packed;           /* rows*columns/8*5 bytes */
    const uint16_t *group_scale_f16; /* rows*columns/64 */
    const uint32_t *protected_rows;  /* protected_count, may be NULL if 0 */
    const uint16_t *protected_bf16;  /* protected_count*columns */
    uint32_t protected_count;
} adi_hip_head_chunk;

/* adi::Bf16Matrix (include/adi/kernels.hpp:73-77). */
typedef struct {
    uint32_t rows;
    uint32_t columns;
    const uint16_t *values; /* rows*columns bf16 bits, row-major */
} adi_hip_bf16_matrix;

/* adi::MachEmbedding (include/adi/kernels.hpp:54-62). */
typedef struct {
    uint32_t rows;                     /* vocabulary */
    uint32_t columns;                  /* hidden, a multiple of 64 */
    const uint8_t *packed;             /* rows*columns/2 bytes, high nibble first */
    const uint16_t *minimum_f16;       /* rows*columns/64 */
    const uint16_t *maximum_f16;       /* rows*columns/64 */
    const uint32_t *exception_indexes; /* exception_count, ascending flat indexes */
    const uint16_t *exception_bf16;    /* exception_count */
    uint32_t exception_count;
} adi_hip_embedding;

/* ---- Backend op table entries -------------------------------------------- */
/* Inputs [batch, columns] and outputs [batch, rows], batch-major, device. */

/* Backend::expert_matvec / expert_matmul -> mach_expert_matvec/matmul
 * (src/kernels.cpp:385-593): y = sv * H_R(Z), Z[r] = sum over tile columns of
 * gamma(tile) * (decoded tile row . x_hat), x_hat = H_C(su * x). */
int adi_hip_expert_matmul(adi_hip_context *ctx, const adi_hip_expert_matrix *m,
                          const float *inputs, uint32_t batch, float *outputs);
int adi_hip_expert_matvec(adi_hip_context *ctx, const adi_hip_expert_matrix *m,
                          const float *input, float *output);

/* Backend::ne_matvec / ne_matmul -> mach_ne_matvec/matmul
 * (src/kernels.cpp:595-800). */
int adi_hip_ne_matmul(adi_hip_context *ctx, const adi_hip_ne_matrix *m,
                      const float *inputs, uint32_t batch, float *outputs);
int adi_hip_ne_matvec(adi_hip_context *ctx, const adi_hip_ne_matrix *m,
                      const float *input, float *output);

/* In place, on `count` contiguous device vectors of n floats (n a power of
 * two up to 8192): the normalised fast Walsh-Hadamard transform every packed
 * projection applies to its input and output, hadamard_transform
 * (src/simd.cpp:48-63, 395-397). Butterflies run with strides 1, 2, 4, ...
 * as in the reference, so the result is bit-identical to it. */
int adi_hip_hadamard(adi_hip_context *ctx, float *values, uint32_t n,
                     uint32_t count);

/* The decoded weights of a packed matrix as a dense fp32 [rows, columns]
 * array, through the same loads and decode the GEMV kernels use: expert
 * lattice values V (before the tile gamma and the su/sv/Hadamard rotations),
 * NE values V * Wscale. Bit-identical with the reference's state tables
 * (src/codec_cache.cpp:33-115) walked tile by tile
 * (src/expert_trellis.hpp:44-105, src/ne_trellis.hpp:27-97); no reference
 * function returns them as one array, they exist there only inside the
 * projection loops (src/kernels.cpp:103-264). */
int adi_hip_expert_decode(adi_hip_context *ctx, const adi_hip_expert_matrix *m,
                          float *values);
int adi_hip_ne_decode(adi_hip_context *ctx, const adi_hip_ne_matrix *m,
                      float *values);

/* Backend::head_matvec / head_matmul -> mach_head_matvec/matmul
 * (src/kernels.cpp:847-979): int5_g64 logits, protected rows replaced by the
 * ISA-ordered bf16 dot. Logits agree with the CPU path to fp32 rounding of a
 * different summation order (the argmax is made exact by
 * adi_hip_head_argmax). */
int adi_hip_head_matmul(adi_hip_context *ctx, const adi_hip_head_chunk *h,
                        const float *inputs, uint32_t batch, float *outputs);
int adi_hip_head_matvec(adi_hip_context *ctx, const adi_hip_head_chunk *h,
                        const float *input, float *output);

/* Head logits plus the greedy token of each row: the first maximum, as
 * sample_token at temperature 0 takes it (std::max_element,
 * src/generation.cpp:177-180). Every row whose GPU logit lies within the
 * summation-order error bound of the top GPU logit is re-evaluated in the CPU
 * reduction order of adi_hip_set_reduction_isa, so the index is the one the
 * CPU path returns. logits (nullable, device [batch, rows]) receives the
 * logits of adi_hip_head_matmul; argmax [batch] u32, device. */
int adi_hip_head_argmax(adi_hip_context *ctx, const adi_hip_head_chunk *h,
                        const float *inputs, uint32_t batch, float *logits,
                        uint32_t *argmax);

/* Backend::dense_bf16_matvec / dense_bf16_matmul -> bf16_matvec/matmul
 * (src/kernels.cpp:981-1050), in the CPU reduction order of
 * adi_hip_set_reduction_isa: bit-identical with the CPU build. */
int adi_hip_bf16_matmul(adi_hip_context *ctx, const adi_hip_bf16_matrix *m,
                        const float *inputs, uint32_t batch, float *outputs);
int adi_hip_bf16_matvec(adi_hip_context *ctx, const adi_hip_bf16_matrix *m,
                        const float *input, float *output);

/* Backend::normalize_rms -> rms_norm (src/kernels.cpp:1052-1073), applied to
 * each of `rows` vectors of `count` values. */
int adi_hip_rms_norm(adi_hip_context *ctx, const float *input,
                     const uint16_t *weight_bf16, uint32_t count, uint32_t rows,
                     float weight_offset, float epsilon, float *output);

/* ---- executor-level MoE entries (new backend surface) --------------------- */

/* top_experts for each of `batch` logit rows (src/executor.cpp:193-229):
 * (logit desc, index asc), softmax over the eight. route_expert [batch*8] u32,
 * route_weight [batch*8] f32, device. Indices are exact; weights agree to
 * the last bits of expf. */
int adi_hip_top_experts(adi_hip_context *ctx, const float *logits,
                        uint32_t batch, uint32_t experts,
                        uint32_t *route_expert, float *route_weight);

/* Routing plus the stable counting sort of moe_forward_batch
 * (src/executor.cpp:1221-1258). logit_bias (nullable) [experts] is added to
 * each logit row first. Outputs (device): route_expert/route_weight
 * [batch*8], counts [experts], offsets [experts+1], grouped_batch and
 * route_to_grouped [batch*8]. The permutation is exact. */
int adi_hip_moe_route(adi_hip_context *ctx, const float *logits,
                      const float *logit_bias, uint32_t batch, uint32_t experts,
                      uint32_t *route_expert, float *route_weight,
                      uint32_t *counts, uint32_t *offsets,
                      uint32_t *grouped_batch, uint32_t *route_to_grouped);

/* Per-expert matrices stacked expert-major, as the checkpoint's 32-expert
 * chunks are (src/model.cpp:483-532): expert e's trellis starts at
 * e*(rows/16)*(columns/16)*24 words, su at e*columns, sv at e*rows, gamma at
 * e*(rows/16 + columns/16). */
typedef struct {
    const uint16_t *trellis;
    const uint16_t *su_f16;
    const uint16_t *sv_f16;
    const uint16_t *wave_gamma_f16;
} adi_hip_expert_stack;

/* The fields of one layer's MoE descriptor (include/adi/model.hpp:30-37,
 * read by src/executor.cpp:254-324). */
typedef struct {
    uint32_t hidden;        /* 2048 */
    uint32_t expert_hidden; /* 512 */
    uint32_t experts;       /* 256 */
    adi_hip_bf16_matrix router;             /* experts x hidden */
    adi_hip_bf16_matrix shared_expert_gate; /* 1 x hidden */
    adi_hip_expert_stack gate;  /* experts x (expert_hidden x hidden) */
    adi_hip_expert_stack up;    /* experts x (expert_hidden x hidden) */
    adi_hip_expert_stack down;  /* experts x (hidden x expert_hidden) */
    const adi_hip_codebook *expert_codebook;
    adi_hip_ne_matrix shared_gate; /* expert_hidden x hidden */
    adi_hip_ne_matrix shared_up;   /* expert_hidden x hidden */
    adi_hip_ne_matrix shared_down; /* hidden x expert_hidden */
} adi_hip_moe_layer;

/* One MoE block for `batch` rows: moe_forward (batch 1,
 * src/executor.cpp:242-330) and moe_forward_batch (src/executor.cpp:
 * 1181-1453). Routing uses the bit-exact router and sort; the eight expert
 * outputs are combined in route order, then the sigmoid-gated shared expert
 * is added. logit_bias (nullable, device [experts]) is added to the router
 * logits before top_experts. route_expert/route_weight (nullable, device
 * [batch*8]) receive the routes. Workspace is cached in the context and grows
 * to the largest batch seen. */
int adi_hip_moe_forward(adi_hip_context *ctx, const adi_hip_moe_layer *layer,
                        const float *inputs, uint32_t batch,
                        const float *logit_bias, float *outputs,
                        uint32_t *route_expert, float *route_weight);

/* adi_hip_moe_forward for a decode batch (1..16 rows) without allocating:
 * no hipMalloc, hipFree or allocating library call on any path. No
 * counterpart in the reference; it is for callers that cannot allocate
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * it). The intermediates live in a fixed 12 MiB device array of the library,
 * one per GPU, held until the process ends; a batch or layer geometry whose
 * plan exceeds it is rejected (ADI_HIP_INVALID_ARGUMENT, outputs untouched).
 * Every call on one GPU shares that array: calls that overlap on one GPU (from
 * several contexts or streams) race. Results equal adi_hip_moe_forward's. */
int adi_hip_moe_forward_static(adi_hip_context *ctx, const adi_hip_moe_layer *layer,
                               const float *inputs, uint32_t batch,
                               const float *logit_bias, float *outputs,
                               uint32_t *route_expert, float *route_weight);

/* ---- token side of decoding ----------------------------------------------- */

/* Backend::embedding_row -> mach_embedding_row (src/kernels.cpp:802-845) for
 * `count` tokens at once: per 64-column group value = min + code * step with
 * step = max(max - min, 1e-8) / 15 (f16 min/max, separate multiply and add),
 * then the row's bf16 exceptions overwrite their columns; bit-exact.
 * tokens: DEVICE [count] (a sampled token never leaves HBM); outputs: DEVICE
 * [count, columns]. A token >= rows yields a row of NaN (the reference throws
 * std::invalid_argument; the token is device data here). */
int adi_hip_embedding_rows(adi_hip_context *ctx, const adi_hip_embedding *e,
                           const uint32_t *tokens, uint32_t count, float *outputs);

/* sample_token at temperature 0 (src/generation.cpp:180-183) for `rows` rows
 * of `count` logits: the first index of the largest logit (std::max_element).
 * A row holding a non-finite logit yields 0xFFFFFFFF (the reference rejects
 * such logits with std::invalid_argument). logits: DEVICE [rows, count];
 * tokens: DEVICE [rows]. */
int adi_hip_argmax_rows(adi_hip_context *ctx, const float *logits, uint32_t rows,
                        uint32_t count, uint32_t *tokens);

/* sample_token (src/generation.cpp:161-225) for `rows` rows of `count`
 * logits. temperature 0 is the greedy choice (as adi_hip_argmax_rows); above
 * 0 the tokens are ordered by logit (ties by index), p_i = exp((l_i - max) /
 * temperature) in double, the smallest prefix whose sum of p_i / sum(p)
 * reaches top_p is kept, and the token is where the running sum of p first
 * reaches target = kept_sum * u, u = min(word * 2^-64, 1 - 2^-53) for the row's
 * 64-bit word: the draw of std::uniform_real_distribution<double>(0,
 * kept_sum) from a std::mt19937_64 whose next output is the word (one word
 * per sampled row, as the reference draws). The orderings, prefix and draw
 * follow the reference exactly; sum(p) is added in a fixed tree order rather
 * than in sorted order, so a token can differ only where a threshold lies
 * within the double rounding of a running sum. Rejected like the reference:
 * temperature outside {0} and [1e-4, 2], top_p outside (0, 1], count 0
 * (ADI_HIP_INVALID_ARGUMENT); a row holding a non-finite logit yields
 * 0xFFFFFFFF. logits: DEVICE [rows, count]; words: DEVICE [rows] (unused at
 * temperature 0, may be NULL); tokens: DEVICE [rows]. */
int adi_hip_sample_rows(adi_hip_context *ctx, const float *logits, uint32_t rows,
                        uint32_t count, float temperature, float top_p,
                        const uint64_t *words, uint32_t *tokens);

/* ---- attention of one decode token (the hybrid model's head geometry) --- */

/* adi::FullAttentionDescriptor (include/adi/model.hpp:39-46): 16 query heads
 * and 2 KV heads of 256. query rows hold per head 256 query then 256 gate
 * values (8192 rows); key and value have 512 rows; output has 4096 columns.
 * The norms are 256 bf16 values in device memory. */
typedef struct {
    adi_hip_ne_matrix query;
    adi_hip_ne_matrix key;
    adi_hip_ne_matrix value;
    adi_hip_ne_matrix output;
    const uint16_t *query_norm;
    const uint16_t *key_norm;
} adi_hip_full_attention;

/* full_attention_forward (src/executor.cpp:332-418) for the token at
 * `position` of one sequence: q/k/v projections, per-head RMS norm with
 * (1 + w) and partial RoPE on the first 64 dimensions (theta base 1e7,
 * src/model.cpp:606-615), the new key and value appended to the cache, grouped
 * online-softmax attention over positions 0..position, the sigmoid output
 * gate, and the output projection. keys and values are device caches of
 * `capacity` entries of [2][256] floats; entries below `position` hold the
 * sequence's history and entry `position` receives this token's. Input and
 * output have `hidden` (= the projections' columns) floats. */
int adi_hip_full_attention_forward(adi_hip_context *ctx, const adi_hip_full_attention *layer,
                                   uint32_t position, const float *input, float *output,
                                   float *keys, float *values, uint32_t capacity);
/* The same for `count` consecutive tokens at positions position ..
 * position + count - 1 (inputs and outputs [count][hidden]): the result of
 * calling the one-token form for each in turn, with the projections batched
 * (the attention half of prefill, src/executor.cpp:561-731). position + count
 * must not exceed capacity. */
int adi_hip_full_attention_prefill(adi_hip_context *ctx, const adi_hip_full_attention *layer,
                                   uint32_t position, uint32_t count, const float *inputs,
                                   float *outputs, float *keys, float *values, uint32_t capacity);

/* adi::LinearAttentionDescriptor (include/adi/model.hpp:48-58): Gated
 * DeltaNet with 16 key heads and 32 value heads of 128. qkv has 8192 rows
 * (2048 query, 2048 key, 4096 value channels), gate 4096, output 4096
 * columns; alpha and beta are 32 x hidden bf16; convolution is 8192 x 4 bf16;
 * alpha_bias and a_log 32 bf16; norm 128 bf16. */
typedef struct {
    adi_hip_ne_matrix qkv;
    adi_hip_ne_matrix gate;
    adi_hip_ne_matrix output;
    adi_hip_bf16_matrix alpha;
    adi_hip_bf16_matrix beta;
    const uint16_t *convolution;
    const uint16_t *alpha_bias;
    const uint16_t *a_log;
    const uint16_t *norm;
} adi_hip_linear_attention;

/* linear_attention_forward (src/executor.cpp:420-557) for one token:
 * projections, the width-4 causal convolution with SiLU, L2-normalised query
 * and key heads, the gated delta recurrence (src/executor.cpp:121-184,
 * src/simd.cpp:108-127), per-head RMS norm times SiLU(gate), and the output
 * projection. convolution_state [8192][3] and recurrent_state [32][128][128]
 * are the sequence's device state, updated in place (all zero for a new
 * sequence). alpha and beta use the context's bf16 reduction order. */
int adi_hip_linear_attention_forward(adi_hip_context *ctx, const adi_hip_linear_attention *layer,
                                     const float *input, float *output, float *convolution_state,
                                     float *recurrent_state);
/* The same for `count` consecutive tokens (inputs and outputs
 * [count][hidden]): the recurrence runs over them in order, the projections
 * batched (src/executor.cpp:733-1179). */
int adi_hip_linear_attention_prefill(adi_hip_context *ctx, const adi_hip_linear_attention *layer,
                                     uint32_t count, const float *inputs, float *outputs,
                                     float *convolution_state, float *recurrent_state);

/* ---- one decoder layer of a decode step ---------------------------------- */

/* adi::LayerDescriptor (include/adi/model.hpp:60-66): the two RMS norms,
 * the layer's attention (full or linear) and its MoE block, all in device
 * memory. */
typedef struct {
    const uint16_t *input_norm;          /* hidden bf16 */
    const uint16_t *post_attention_norm; /* hidden bf16 */
    int full_attention;                  /* nonzero: `full` is used, else `linear` */
    adi_hip_full_attention full;
    adi_hip_linear_attention linear;
    adi_hip_moe_layer moe;
} adi_hip_decoder_layer;

/* The layer's share of a sequence's decoder state (adi::DecoderState,
 * include/adi/executor.hpp:86-90): the KV cache of a full-attention layer
 * (capacity entries of [2][256] keys and values) or the convolution
 * [8192][3] and recurrent [32][128][128] state of a linear one. */
typedef struct {
    float *keys;
    float *values;
    uint32_t capacity;
    float *convolution;
    float *recurrent;
} adi_hip_layer_state;

/* decode_layer (src/executor.cpp:1473-1529) for the token at `position`, in
 * place on the device row `hidden` (moe.hidden floats): hidden +=
 * attention(rms_norm(hidden, input_norm)), then hidden +=
 * moe_forward(rms_norm(hidden, post_attention_norm)), both norms with weight
 * offset 1 and epsilon 1e-6. */
int adi_hip_decode_layer(adi_hip_context *ctx, const adi_hip_decoder_layer *layer,
                         uint32_t position, float *hidden, const adi_hip_layer_state *state);
/* The layer for `count` consecutive tokens at positions position ..
 * position + count - 1, rows hidden[count][moe.hidden] in place: the prefill
 * step of a chunk (src/executor.cpp:1827-2101), with batched norms,
 * projections and MoE (adi_hip_moe_forward at batch `count`). */
int adi_hip_prefill_layer(adi_hip_context *ctx, const adi_hip_decoder_layer *layer,
                          uint32_t position, uint32_t count, float *hidden,
                          const adi_hip_layer_state *state);

/* ---- the whole model: decode steps over sequences, prompt prefill -------- */

/* The parts of adi::MachModel (include/adi/model.hpp) that decoding uses, in
 * device memory: the decoder layers (host array of descriptors), the
 * embedding (its rows are the vocabulary, its columns the hidden size), the
 * final RMS norm (hidden bf16) and the head chunks (host array; their rows,
 * in order, cover the vocabulary). `context` is the model's context length
 * (ModelConfig::context, 262,144 for the checkpoint). */
typedef struct {
    uint32_t layers;
    const adi_hip_decoder_layer *layer;
    const adi_hip_embedding *embedding;
    const uint16_t *final_norm;
    uint32_t head_chunks;
    const adi_hip_head_chunk *head;
    uint32_t context;
} adi_hip_model;

/* adi::DecoderState (include/adi/executor.hpp:86-90): the sequence's
 * position (tokens decoded so far) and its state for each layer (host array
 * of `layers` entries). A full-attention layer's cache must hold every
 * position the calls below reach (capacity > position); a new sequence has
 * position 0 and zero linear-attention states. */
typedef struct {
    uint32_t position;
    const adi_hip_layer_state *layers;
} adi_hip_decoder_state;

/* decode_batch (src/executor.cpp:1592-1825): one decode step of `batch`
 * sequences, token tokens[b] (HOST) of sequence states[b] (HOST array):
 * embedding rows, every layer with the norms, projections and MoE batched
 * over the sequences and the attention per sequence at its own position,
 * the final norm, and the head into logits[b][vocabulary] (DEVICE; NULL
 * skips the norm and head, as decode_token with empty logits). Each
 * position advances by one. Rejected before anything runs, states untouched:
 * batch 0 or NULL arrays ("decoder batch shape mismatch"), a token >= the
 * vocabulary ("decoder batch token is out of range") with
 * ADI_HIP_INVALID_ARGUMENT; a position >= context ("decoder context is
 * exhausted") with ADI_HIP_OUT_OF_RANGE; a missing layer state or a full
 * cache with ADI_HIP_INVALID_ARGUMENT. decode_token (src/executor.cpp:
 * 1565-1590) is this call with batch 1. */
int adi_hip_decode_batch(adi_hip_context *ctx, const adi_hip_model *model, const uint32_t *tokens,
                         uint32_t batch, adi_hip_decoder_state *states, float *logits);

/* prefill_prompt (src/generation.cpp:131-159) over prefill (src/executor.cpp:
 * 1827-2101): `count` prompt tokens (HOST) of one sequence in chunks of
 * `ubatch` tokens (0: 128; ExecutionOptions::prefill_ubatch, 1..4096), each
 * chunk through every layer with adi_hip_prefill_layer's arithmetic, then
 * the last token's final norm and head into logits[vocabulary] (DEVICE;
 * NULL skips them). The position advances by count. Rejected before
 * anything runs: count 0 or a prompt past the context ("prefill shape or
 * context is invalid"), a token >= the vocabulary ("prefill token is out of
 * range"), ubatch > 4096, a missing layer state or a cache too small for the
 * prompt, all ADI_HIP_INVALID_ARGUMENT. */
int adi_hip_prefill(adi_hip_context *ctx, const adi_hip_model *model, const uint32_t *tokens,
                    uint32_t count, uint32_t ubatch, adi_hip_decoder_state *state, float *logits);

/* A decode step captured as a HIP graph and replayed, for the serving loop
 * that calls decode_batch once per iteration (src/generation.cpp:560-660)
 * with the same sequences: one hipGraphLaunch in place of the step's
 * several hundred kernel launches. The graph holds adi_hip_decode_batch's
 * launches for `batch` sequences; each replay reads the step's tokens from
 * `tokens` (DEVICE [batch], written by the caller before the launch, e.g. by
 * adi_hip_argmax_rows or adi_hip_sample_rows; a token >= the vocabulary
 * gives NaN rows, it is not checked) and writes logits[b][vocabulary]
 * (DEVICE; NULL skips the norm and head). The positions live in a device
 * array the graph advances itself; every replay gives the bits of
 * adi_hip_decode_batch at the same positions.
 *
 * create copies the model descriptor and each sequence's layer states
 * (same checks as adi_hip_decode_batch; ADI_HIP_INVALID_ARGUMENT with
 * profiling on) and records the step without running it. launch replays
 * it and advances every states[b].position by one; states must be the
 * sequences the graph was created with (same layer state pointers), at any
 * positions (positions the caller changed, e.g. a reset, are taken over).
 * A launch re-records the step by itself when the positions outgrow what
 * the recording covers (steps of 512) or a call since has grown one of the
 * context's scratch arenas. captures returns how many recordings a graph
 * has made. The model, the states, `tokens` and `logits` must outlive the
 * graph. No counterpart in the reference (its CPU loop has no launches). */
typedef struct adi_hip_decode_graph adi_hip_decode_graph;
int adi_hip_decode_graph_create(adi_hip_context *ctx, const adi_hip_model *model, uint32_t batch,
                                const adi_hip_decoder_state *states, const uint32_t *tokens,
                                float *logits, adi_hip_decode_graph **out);
int adi_hip_decode_graph_launch(adi_hip_decode_graph *graph, adi_hip_decoder_state *states);
uint32_t adi_hip_decode_graph_captures(const adi_hip_decode_graph *graph);
void adi_hip_decode_graph_destroy(adi_hip_decode_graph *graph);

/* ---- continuous batching (serving) --------------------------------------- */

/* ContinuousBatcher (src/generation.cpp:343-660) without the tokenizer:
 * requests are prompt token ids, outputs are token ids. One call of
 * adi_hip_batcher_step is one iteration of the reference's worker loop
 * (generation.cpp:540-646): admit the oldest pending request (prefill of its
 * prompt into a free sequence slot, the logits row of its last token), then
 * for every active sequence in order: fail it if cancelled, sample its next
 * token from its logits row (temperature and top_p of the request, the draw
 * from the request's std::mt19937_64 seeded with its seed; the device
 * sampler of adi_hip_sample_rows, or the greedy choice at temperature 0),
 * finish it on a stop token (not kept) or at its output limit, and decode
 * the survivors' tokens in one adi_hip_decode_batch step. The caller drives
 * the loop (a serving thread calls step while work remains); submit, cancel,
 * status and release may come from other threads, while the context belongs
 * to the stepping thread. Sequence state for max_batch slots of `capacity`
 * positions is allocated at creation; a request waits while every slot is
 * busy (the reference admits without a bound). */
typedef struct adi_hip_batcher adi_hip_batcher;

typedef struct {
    uint32_t max_batch;             /* sequence slots (1..256) */
    uint32_t capacity;              /* positions per sequence; the context a request may use */
    uint32_t prefill_ubatch;        /* 0: 128 */
    const uint32_t *stop_tokens;    /* HOST; the tokenizer's eos and <|im_end|> */
    uint32_t stop_count;
    const uint32_t *masked_tokens;  /* HOST; Tokenizer::mask_unused_logits: set to the lowest float */
    uint32_t masked_count;
    uint32_t direct_steps;          /* 0: once the same sequences have stepped twice in a row,
                                       their decode step is recorded (adi_hip_decode_graph) and
                                       replayed while they stay; nonzero: every step launched
                                       directly */
} adi_hip_batcher_options;

/* adi::GenerationOptions (include/adi/generation.hpp:17-22); 0 output
 * tokens means "up to the context". */
typedef struct {
    uint32_t max_output_tokens;
    float temperature;
    float top_p;
    uint64_t seed;
} adi_hip_generation_options;

#define ADI_HIP_REQUEST_PENDING 0
#define ADI_HIP_REQUEST_RUNNING 1
#define ADI_HIP_REQUEST_STOP_TOKEN 2 /* FinishReason::stop_token */
#define ADI_HIP_REQUEST_LENGTH 3     /* FinishReason::length */
#define ADI_HIP_REQUEST_FAILED 4     /* the request's exception; message in adi_hip_batcher_request_error */

/* adi::GenerationResult (include/adi/generation.hpp:29-38) of a request so
 * far: its state, prompt and output token counts, and the prefill and decode
 * wall times in seconds. */
typedef struct {
    uint32_t state;
    uint32_t input_tokens;
    uint32_t output_tokens;
    double prefill_seconds;
    double decode_seconds;
} adi_hip_request_status;

/* Copies the model descriptor (its arrays too) and the options; the model's
 * device memory must outlive the batcher. Rejects max_batch outside 1..256,
 * capacity 0 or above the model's context, a stop or masked token outside
 * the vocabulary. */
int adi_hip_batcher_create(adi_hip_context *ctx, const adi_hip_model *model,
                           const adi_hip_batcher_options *options, adi_hip_batcher **out);
void adi_hip_batcher_destroy(adi_hip_batcher *batcher);
/* Queues a request (validate_generation_options, generation.cpp:93-110:
 * "max_output_tokens must be positive" is not possible here, 0 meaning
 * unbounded; above the context "max_output_tokens exceeds model context";
 * "invalid generation options"). `request` receives its id (from 1). */
int adi_hip_batcher_submit(adi_hip_batcher *batcher, const uint32_t *prompt, uint32_t count,
                           const adi_hip_generation_options *options, uint64_t *request);
/* Marks a request cancelled: the next step fails it ("generation
 * cancelled") whether pending or active. */
int adi_hip_batcher_cancel(adi_hip_batcher *batcher, uint64_t request);
/* One iteration of the loop; `remaining` (may be NULL) receives the number
 * of requests pending or active afterwards. A failure of the decode step
 * fails every active request and is returned. */
int adi_hip_batcher_step(adi_hip_batcher *batcher, uint32_t *remaining);
/* The request's status and up to `capacity` of its output tokens (HOST,
 * may be NULL). */
int adi_hip_batcher_status(adi_hip_batcher *batcher, uint64_t request,
                           adi_hip_request_status *status, uint32_t *tokens, uint32_t capacity);
/* The failure message of a failed request ("" otherwise); valid until the
 * request is released. */
const char *adi_hip_batcher_request_error(adi_hip_batcher *batcher, uint64_t request);
/* Forgets a finished or failed request. */
int adi_hip_batcher_release(adi_hip_batcher *batcher, uint64_t request);
/* Failure injection for tests of the loop's failure handling; no counterpart
 * in the reference, whose tests throw from a stub model instead. `where` =
 * ADI_HIP_BATCHER_FAIL_ADMISSION makes the next admission fail after its
 * prefill, as a device error there would (that request alone fails and its
 * slot stays free); ADI_HIP_BATCHER_FAIL_STEP makes the next step's sampling
 * fail after its synchronize, as a one-launch MoE wait that ran out would
 * (every active request fails, the step returns the error). Nothing faults:
 * the device work runs normally and the host reports the failure. */
#define ADI_HIP_BATCHER_FAIL_ADMISSION 1
#define ADI_HIP_BATCHER_FAIL_STEP 2
int adi_hip_batcher_force_failure(adi_hip_batcher *batcher, int where);

/* ---- kernel profiling ----------------------------------------------------- */

/* Per-kernel timing with HIP events on the context stream, the counterpart
 * of the reference's KernelTimer / kernel_profiles()
 * (include/adi/profiling.hpp:9-40). Enabling resets the counters. */
typedef struct {
    char name[48];
    uint64_t launches;
    double total_ms;
} adi_hip_kernel_profile;

int adi_hip_profiling_enable(adi_hip_context *ctx, int enabled);
/* Writes up to `capacity` entries; *count receives the number of kinds. The
 * event timings are resolved here (this call synchronizes the stream). */
int adi_hip_profiling_read(adi_hip_context *ctx, adi_hip_kernel_profile *out,
                           uint32_t capacity, uint32_t *count);

#ifdef __cplusplus
}
#endif

#endif
