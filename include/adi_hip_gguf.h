/*
 * adi_hip_gguf.h -- the checkpoint side of the packed path: a GGUF v3 reader
 * and the upload of a layer's packed MoE tensors, of whole decoder layers, of
 * the output head and of the embedding table into the device descriptors of
 * adi_hip.h.
 *
 * The reference maps the checkpoint with adi::GgufFile (include/adi/gguf.hpp,
 * src/gguf.cpp) and reads the packed tensors as non-owning host views in
 * adi::MachModel (src/model.cpp:267-314 non_expert, 431-533 bf16_matrix and
 * expert, 808-880 validate_manifest). Here the same tensors, under the same
 * names and with the same shape rules, are copied once into HBM, where they
 * stay packed; the kernels decode them in place.
 *
 * Tensor names (docs/gguf.md of the reference):
 *   mach.expert.{layer}.e{chunk}.{gate|up|down}.{trellis|su|sv|wave_gamma}
 *       32-expert chunks, chunk = 0, 32, 64, ...; GGUF dims {24, tiles, 32},
 *       {columns, 32}, {rows, 32}, {rows/16 + columns/16, 32}; i16, f16 x 3
 *   mach.ne.{layer}.{source}|{trellis|SU|SV|Wscale}
 *       source = model.language_model.layers.{layer}.mlp.shared_expert.
 *       {gate|up|down}_proj.weight; dims {64, tiles}, {columns}, {rows}, {1};
 *       i16, i8, i8, f32
 *   hf.model.language_model.layers.{layer}.mlp.gate.weight          bf16 {hidden, experts}
 *   hf.model.language_model.layers.{layer}.mlp.shared_expert_gate.weight  bf16 {hidden, 1}
 *   mach.tlut.expert.tlut  f32 {8, 32768};  mach.tlut.ne.tlut  f32 {2, 512}
 *   mach.embedding.{q_packed|mn|mx|exc_idx|exc_bits}
 *   hf.model.language_model.layers.{layer}.{input_layernorm|post_attention_layernorm}.weight,
 *   .self_attn.{q|k|v|o}_proj.weight (NE), .self_attn.{q|k}_norm.weight,
 *   .linear_attn.{in_proj_qkv|in_proj_z|out_proj}.weight (NE),
 *   .linear_attn.{in_proj_a|in_proj_b|conv1d|norm}.weight, .linear_attn.{dt_bias|A_log}
 *   mach.output.{chunk}.LMHEADCHUNK:{begin}:{end}|{qp|gscale|prot_rows|prot_dense},
 *   hf.model.language_model.norm.weight
 *
 * File-level calls take no context: their failures leave a message for
 * adi_hip_gguf_error() (per calling thread). Upload calls take a context and
 * report through adi_hip_last_error().
 */
#ifndef ADI_HIP_GGUF_H
#define ADI_HIP_GGUF_H

#include "adi_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

#define ADI_HIP_NOT_FOUND (-5) /* tensor or metadata key absent (or of another type) */

/* GGML storage types the reader accepts (adi::GgmlType,
 * include/adi/gguf.hpp:30-39). */
#define ADI_HIP_GGML_F32 0
#define ADI_HIP_GGML_F16 1
#define ADI_HIP_GGML_I8 24
#define ADI_HIP_GGML_I16 25
#define ADI_HIP_GGML_I32 26
#define ADI_HIP_GGML_I64 27
#define ADI_HIP_GGML_F64 28
#define ADI_HIP_GGML_BF16 30

typedef struct adi_hip_gguf adi_hip_gguf;

/* adi::GgufTensor (include/adi/gguf.hpp:47-54) with its data. */
typedef struct {
    uint32_t type;            /* ADI_HIP_GGML_* */
    uint32_t dimension_count; /* 1..4 */
    uint64_t dimensions[4];   /* GGUF order: dimensions[0] is contiguous */
    uint64_t elements;
    uint64_t bytes;
    const void *data;         /* host pointer into the file mapping */
} adi_hip_gguf_tensor;

/* GgufFile::GgufFile (src/gguf.cpp:232-330): maps the file read-only and
 * validates it: magic "GGUF", version 3, known metadata value types (arrays
 * nested at most 8 deep), no duplicate metadata key or tensor name, 1 to 4
 * nonzero dimensions, a supported tensor type, general.alignment a nonzero
 * power of two (default 32), and every tensor's bytes inside the file.
 * On failure *out is NULL. */
int adi_hip_gguf_open(const char *path, adi_hip_gguf **out);
void adi_hip_gguf_close(adi_hip_gguf *file);
/* Message of the calling thread's last failed file-level call. */
const char *adi_hip_gguf_error(void);

uint32_t adi_hip_gguf_version(const adi_hip_gguf *file);
uint64_t adi_hip_gguf_alignment(const adi_hip_gguf *file);
uint64_t adi_hip_gguf_metadata_count(const adi_hip_gguf *file);
uint64_t adi_hip_gguf_tensor_count(const adi_hip_gguf *file);

/* GgufFile::find_tensor + tensor_data (src/gguf.cpp:417-425, 570-572). */
int adi_hip_gguf_find_tensor(const adi_hip_gguf *file, const char *name,
                             adi_hip_gguf_tensor *out);

/* GgufFile::integer / number / boolean / string (src/gguf.cpp:427-503):
 * integer accepts unsigned types and non-negative signed ones; number also
 * f32/f64; boolean only bool; string only string. */
int adi_hip_gguf_integer(const adi_hip_gguf *file, const char *key, uint64_t *out);
int adi_hip_gguf_number(const adi_hip_gguf *file, const char *key, double *out);
int adi_hip_gguf_boolean(const adi_hip_gguf *file, const char *key, int *out);
int adi_hip_gguf_string(const adi_hip_gguf *file, const char *key, const char **data,
                        uint64_t *length);
/* GgufFile::string_array / integer_array (src/gguf.cpp:505-568): *count
 * receives the element count of an array of strings (string_array) or of
 * unsigned integers (integer_array); item `index` when index < count. */
int adi_hip_gguf_string_array(const adi_hip_gguf *file, const char *key, uint64_t index,
                              uint64_t *count, const char **data, uint64_t *length);
int adi_hip_gguf_integer_array(const adi_hip_gguf *file, const char *key, uint64_t index,
                               uint64_t *count, uint64_t *value);

/* The MoE geometry of the checkpoint (adi::MachConfig, src/model.cpp:216-223,
 * qwen35moe.* keys). */
typedef struct {
    uint32_t layers;         /* qwen35moe.block_count */
    uint32_t hidden;         /* qwen35moe.embedding_length */
    uint32_t experts;        /* qwen35moe.expert_count */
    uint32_t active_experts; /* qwen35moe.expert_used_count */
    uint32_t expert_hidden;  /* qwen35moe.expert_feed_forward_length */
    uint32_t shared_hidden;  /* qwen35moe.expert_shared_feed_forward_length */
} adi_hip_moe_geometry;

/* Reads the geometry and checks the codec metadata the packed path depends
 * on (src/model.cpp:180-213): general.architecture qwen35moe, adi.additive,
 * adi.format_version 1, the expert and NE codec names, adi.expert.k_num 3,
 * k_den 2, l 16, v 8, tlut_bits 15, tile_x and tile_y 16; the geometry the
 * kernels need (top-8 routing, a shared expert as wide as the routed ones,
 * whole 32-expert chunks, power-of-two widths of at least 64); and the two
 * TLUT tensors (shape, type, finite values, src/model.cpp:808-833). */
int adi_hip_gguf_moe_geometry(const adi_hip_gguf *file, adi_hip_moe_geometry *out);

/* Validates layer `layer`'s MoE tensors on the host as
 * MachModel::validate_manifest does (src/model.cpp:834-880 with the checks of
 * expert, non_expert and bf16_matrix): presence, type and shape of every
 * tensor, finite f16 su/sv/wave_gamma and bf16 router rows, +-1 SU/SV and a
 * positive finite Wscale. */
int adi_hip_gguf_check_moe_layer(const adi_hip_gguf *file, uint32_t layer);

/* The model's codebooks from mach.tlut.expert.tlut and mach.tlut.ne.tlut (the
 * tables MachModel::cache_descriptors derives, src/model.cpp:546-551). */
int adi_hip_gguf_upload_codebooks(adi_hip_context *ctx, const adi_hip_gguf *file,
                                  adi_hip_codebook **expert_codebook,
                                  adi_hip_codebook **ne_codebook);

/* Device copies of checkpoint tensors, in one allocation. */
typedef struct adi_hip_weights adi_hip_weights;

/* Validates layer `layer` (as adi_hip_gguf_check_moe_layer), copies its
 * packed tensors into HBM once, still packed, and fills *descriptor with
 * device pointers into that copy: the 32-expert chunks are laid end to end,
 * so expert e's trellis, su, sv and gamma sit where adi_hip_expert_stack
 * expects them. The weights stay valid until adi_hip_weights_destroy;
 * the file may be closed after the call. */
int adi_hip_gguf_upload_moe_layer(adi_hip_context *ctx, const adi_hip_gguf *file, uint32_t layer,
                                  const adi_hip_codebook *expert_codebook,
                                  const adi_hip_codebook *ne_codebook,
                                  adi_hip_weights **weights,
                                  adi_hip_moe_layer *descriptor);
void adi_hip_weights_destroy(adi_hip_weights *weights);

/* The embedding table (MachModel::embedding, src/model.cpp:316-363, and its
 * checks in validate_manifest, src/model.cpp:836-849): mach.embedding.q_packed
 * i8 {hidden/2, vocabulary}, .mn and .mx f16 {hidden/64, vocabulary},
 * .exc_idx i32 {n} strictly ascending below vocabulary*hidden, .exc_bits i16
 * {n} (bf16 bits); finite f16 and bf16 values and min <= max per group. The
 * hidden width is qwen35moe.embedding_length. Copies the tensors into HBM
 * once and fills *descriptor with device pointers. */
int adi_hip_gguf_upload_embedding(adi_hip_context *ctx, const adi_hip_gguf *file,
                                  adi_hip_weights **weights, adi_hip_embedding *descriptor);
/* The same checks on the host, without uploading. */
int adi_hip_gguf_check_embedding(const adi_hip_gguf *file);

/* The decoder layer around the MoE block (MachModel::cache_descriptors,
 * src/model.cpp:619-683, with the shapes and values validate_manifest checks,
 * src/model.cpp:808-880): hf.{prefix}input_layernorm.weight and
 * post_attention_layernorm.weight bf16 {hidden}; every fourth layer ((layer +
 * 1) % 4 == 0) self_attn.{q,k,v,o}_proj.weight as NE matrices of 8192, 512,
 * 512 rows x hidden and hidden x 4096, with q_norm and k_norm bf16 {256};
 * the others linear_attn.in_proj_qkv (8192 x hidden), in_proj_z (4096 x
 * hidden), out_proj (hidden x 4096) as NE matrices, in_proj_a and in_proj_b
 * bf16 {hidden, 32}, conv1d bf16 {4, 1, 8192}, dt_bias and A_log bf16 {32},
 * norm bf16 {128}. NE matrices as mach.ne.{layer}.{prefix}{name}|{trellis|SU|
 * SV|Wscale} (src/model.cpp:267-314). The check runs on the host; the upload
 * also checks the MoE block (as adi_hip_gguf_upload_moe_layer), copies the
 * whole layer into one allocation and fills every part of *descriptor. */
int adi_hip_gguf_check_decoder_layer(const adi_hip_gguf *file, uint32_t layer);
int adi_hip_gguf_upload_decoder_layer(adi_hip_context *ctx, const adi_hip_gguf *file, uint32_t layer,
                                      const adi_hip_codebook *expert_codebook,
                                      const adi_hip_codebook *ne_codebook, adi_hip_weights **weights,
                                      adi_hip_decoder_layer *descriptor);

/* The int5 output head and the final norm (MachModel::head_chunk,
 * src/model.cpp:367-420, final_norm_, src/model.cpp:604): eight chunks of
 * vocabulary / 8 rows, mach.output.{c}.LMHEADCHUNK:{begin}:{end}|qp i8
 * {hidden/8*5, rows} and |gscale f16 {hidden/64, rows} (finite), optionally
 * |prot_rows i32 {n} with |prot_dense bf16 {hidden, n} (both or neither; rows
 * inside their chunk; finite); hf.model.language_model.norm.weight bf16
 * {hidden}. The vocabulary and hidden width are the embedding's
 * (mach.embedding.q_packed; this library takes any vocabulary divisible by 8,
 * where the reference accepts 248,320 only). The upload lays the chunks end
 * to end as one head of vocabulary rows, protected rows renumbered to it
 * (the logits are the chunks' in order), and returns the final norm's device
 * copy in *final_norm. */
int adi_hip_gguf_check_head(const adi_hip_gguf *file);
int adi_hip_gguf_upload_head(adi_hip_context *ctx, const adi_hip_gguf *file, adi_hip_weights **weights,
                             adi_hip_head_chunk *head, const uint16_t **final_norm);

#ifdef __cplusplus
}
#endif

#endif
