/*
 * adi_oracle.h -- CPU restatement of ADI's packed-weight hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker that the HIP path is
 * compared against; it is never part of the product path. Only tests,
 * the smoke check and the benchmark's CPU-baseline leg may load it.
 *
 * Every function restates the arithmetic of the reference CPU path in its
 * scalar order (the order every SIMD variant of the reference reproduces bit
 * for bit), citing the reference file:line it follows. The two reductions whose
 * order depends on the CPU ISA in the reference (int5 head dot, bf16 dot) take
 * an explicit lane count: 1 = scalar, 8 = AVX2, 16 = AVX-512.
 *
 * Built with -ffp-contract=off: a fused multiply-add rounds differently from
 * the reference's separate multiply and add.
 */
#ifndef ADI_ORACLE_H
#define ADI_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    AO_OK = 0,
    AO_INVALID_ARGUMENT = -1,
    AO_OUT_OF_MEMORY = -2,
};

/* Mirrors adi::MachExpertMatrix (include/adi/kernels.hpp:9-20). */
typedef struct {
    uint32_t rows;
    uint32_t columns;
    const uint16_t *trellis;        /* (rows/16)*(columns/16)*24 words */
    const uint16_t *su_f16;         /* columns */
    const uint16_t *sv_f16;         /* rows */
    const uint16_t *wave_gamma_f16; /* rows/16 + columns/16 */
    const float *tlut;              /* 32768*8 */
    const float *state_values;      /* optional 65536*8 cache, NULL = build */
} ao_expert_matrix;

/* Mirrors adi::MachNeMatrix (include/adi/kernels.hpp:42-52). */
typedef struct {
    uint32_t rows;
    uint32_t columns;
    const uint16_t *trellis;   /* (rows/16)*(columns/16)*64 words */
    const int8_t *su;          /* columns, +-1 */
    const int8_t *sv;          /* rows, +-1 */
    float weight_scale;
    const float *tlut;         /* 512*2 */
    const float *state_values; /* optional 65536*2 cache, NULL = build */
} ao_ne_matrix;

/* Mirrors adi::MachHeadChunk (include/adi/kernels.hpp:64-71). */
typedef struct {
    uint32_t rows;
    uint32_t columns;
    const uint8_t *packed;           /* rows*columns/8*5 bytes */
    const uint16_t *group_scale_f16; /* rows*columns/64 */
    const uint32_t *protected_rows;  /* protected_count */
    const uint16_t *protected_bf16;  /* protected_count*columns */
    uint32_t protected_count;
} ao_head_chunk;

/* Mirrors adi::Bf16Matrix (include/adi/kernels.hpp:73-77). */
typedef struct {
    uint32_t rows;
    uint32_t columns;
    const uint16_t *values;
} ao_bf16_matrix;

/* Mirrors adi::MachEmbedding (include/adi/kernels.hpp:54-62). */
typedef struct {
    uint32_t rows;
    uint32_t columns;
    const uint8_t *packed;             /* rows*columns/2, high nibble first */
    const uint16_t *minimum_f16;       /* rows*columns/64 */
    const uint16_t *maximum_f16;       /* rows*columns/64 */
    const uint32_t *exception_indexes; /* ascending flat indexes */
    const uint16_t *exception_bf16;
    uint32_t exception_count;
} ao_embedding;

/* One MoE block: the fields moe_forward reads from the model's layer
 * descriptor (src/executor.cpp:254, 270-288, 300-324). */
typedef struct {
    uint32_t hidden;
    uint32_t expert_hidden;
    uint32_t experts;
    ao_bf16_matrix router;             /* experts x hidden */
    ao_bf16_matrix shared_expert_gate; /* 1 x hidden */
    const ao_expert_matrix *expert_matrices; /* experts*3: gate, up, down */
    ao_ne_matrix shared_gate;          /* expert_hidden x hidden */
    ao_ne_matrix shared_up;            /* expert_hidden x hidden */
    ao_ne_matrix shared_down;          /* hidden x expert_hidden */
} ao_moe_layer;

/* Conversions (src/kernels.cpp:309-383). */
float ao_f16_to_f32(uint16_t bits);
uint16_t ao_f32_to_f16(float value);
float ao_bf16_to_f32(uint16_t bits);

/* Trellis walks (src/expert_trellis.hpp:44-59, src/ne_trellis.hpp:27-41). */
void ao_expert_tile_states(const uint16_t *words, uint16_t *states /*32*/);
void ao_ne_tile_states(const uint16_t *words, uint16_t *states /*128*/);

/* Codec caches (src/codec_cache.cpp:33-147). */
void ao_build_expert_state_values(const float *tlut, float *out /*65536*8*/);
void ao_build_ne_state_values(const float *tlut, float *out /*65536*2*/);
void ao_build_ne_signed_tlut(const float *tlut, float *out /*1024*2*/);
int ao_build_wave_indexes(uint32_t tile_rows, uint32_t tile_columns,
                          uint16_t *out /*tile_rows*tile_columns*/);

/* Normalised fast Walsh-Hadamard transform (src/simd.cpp:48-63). */
int ao_hadamard(float *values, uint32_t count);

/* Dense decoded weights of one projection, W[row][column], before su/sv and
 * the Hadamard rotations (expert: includes the tile gamma as a separate
 * output; NE: V*Wscale). Used to cross-check the tile walk by brute force. */
int ao_expert_decode_tiles(const ao_expert_matrix *matrix, float *values /*rows*columns*/);
int ao_ne_decode_tiles(const ao_ne_matrix *matrix, float *values /*rows*columns*/);

/* Projections (src/kernels.cpp:385-800). Inputs [batch, columns] and outputs
 * [batch, rows], batch-major. Scalar reference order. */
int ao_expert_matmul(const ao_expert_matrix *matrix, const float *inputs,
                     uint32_t batch, float *outputs);
int ao_ne_matmul(const ao_ne_matrix *matrix, const float *inputs,
                 uint32_t batch, float *outputs);

/* Pre-Hadamard row sums Z (the tile accumulation alone, src/kernels.cpp:103-264,
 * 433-482): inputs are already transformed (x_hat). */
int ao_expert_accumulate(const ao_expert_matrix *matrix, const float *x_hat,
                         uint32_t batch, float *row_sums);
int ao_ne_accumulate(const ao_ne_matrix *matrix, const float *x_hat,
                     uint32_t batch, float *row_sums);

/* int5_g64 output head (src/kernels.cpp:847-979, src/simd.cpp:65-86,
 * src/simd_x86_avx2.cpp:101-120, src/simd_x86_avx512.cpp:87-107). */
int ao_head_matmul(const ao_head_chunk *head, const float *inputs,
                   uint32_t batch, float *outputs, uint32_t lanes);

/* bf16 dense (src/kernels.cpp:981-1050, src/simd.cpp:88-96,
 * src/simd_x86_avx2.cpp:172-193, src/simd_x86_avx512.cpp:109-130). */
float ao_bf16_dot(const uint16_t *weights, const float *input, uint32_t count,
                  uint32_t lanes);
int ao_bf16_matmul(const ao_bf16_matrix *matrix, const float *inputs,
                   uint32_t batch, float *outputs, uint32_t lanes);

/* RMS norm (src/kernels.cpp:1052-1073). */
int ao_rms_norm(const float *input, const uint16_t *weight_bf16, uint32_t count,
                float weight_offset, float epsilon, float *output);

float ao_silu(float value);    /* src/kernels.cpp:1089-1091 */
float ao_sigmoid(float value); /* src/kernels.cpp:1093-1095 */

/* top_experts (src/executor.cpp:193-229). */
int ao_top_experts(const float *logits, uint32_t count, uint32_t *experts,
                   float *weights);

/* Routing + stable counting sort of a batch (src/executor.cpp:1221-1258).
 * logits [batch, experts]; route_expert/route_weight [batch*8];
 * counts [experts]; offsets [experts+1]; grouped_batch and
 * route_to_grouped [batch*8]. */
int ao_moe_route(const float *logits, uint32_t batch, uint32_t experts,
                 uint32_t *route_expert, float *route_weight, uint32_t *counts,
                 uint32_t *offsets, uint32_t *grouped_batch,
                 uint32_t *route_to_grouped);

/* MoE block for a batch (src/executor.cpp:1181-1453; batch 1 equals
 * moe_forward, src/executor.cpp:242-330). logit_bias (nullable, [experts]) is
 * added to the router logits before top_experts. route_expert/route_weight
 * (nullable) receive the routes. threads: 0 = OpenMP default. */
int ao_moe_forward(const ao_moe_layer *layer, const float *inputs,
                   uint32_t batch, const float *logit_bias, uint32_t lanes,
                   float *outputs, uint32_t *route_expert, float *route_weight,
                   int threads);

/* Embedding row decode (mach_embedding_row, src/kernels.cpp:802-845). */
int ao_embedding_row(const ao_embedding *embedding, uint32_t token, float *output);

/* FNV-1a (64-bit) over raw bytes, continuing from `hash` (the benchmark's
 * hash_bytes, src/main.cpp:90-103; start from 0xCBF29CE484222325 as
 * decoder_state_checksum does, src/main.cpp:105-117). */
uint64_t ao_fnv1a64(uint64_t hash, const void *data, size_t bytes);

/* Greedy choice of sample_token at temperature 0: the first index of the
 * largest logit (std::max_element, src/generation.cpp:180-183). */
uint32_t ao_argmax(const float *logits, uint32_t count);

/* sample_token (src/generation.cpp:161-225) with the engine's draw given as
 * its 64-bit word: tokens sorted by logit descending (ties by index, -0 ==
 * +0), p = exp((l - max) / temperature) in double, the prefix whose running
 * p / sum(p) reaches top_p, target = kept_sum * (word * 2^-64, capped below
 * 1), and the first token where the running p reaches target. The sums run
 * in sorted order as the reference's. AO_INVALID_ARGUMENT for the
 * reference's rejected parameters or a non-finite logit. */
int ao_sample_token(const float *logits, uint32_t count, float temperature, float top_p,
                    uint64_t word, uint32_t *token);

/* The first `count` outputs of std::mt19937_64 seeded with `seed` (the
 * engine ContinuousBatcher and generate give each request,
 * src/generation.cpp:270, 495): the 64-bit Mersenne Twister with the
 * parameters of C++11 [rand.predef] (n 312, m 156, r 31, a
 * 0xB5026F5AA96619E9, tempering u 29 d 0x5555555555555555, s 17 b
 * 0x71D67FFFEDA60000, t 37 c 0xFFF7EEE000000000, l 43, initialisation
 * multiplier 6364136223846793005). */
void ao_mt19937_64(uint64_t seed, uint32_t count, uint64_t *out);

/* ---- attention of one decode token (src/executor.cpp:25-186, 332-557,
 * src/attention.cpp) -------------------------------------------------------- */

/* normalize_head (src/executor.cpp:25-41): values[i] *= scale * (1 + w[i]),
 * scale = 1 / sqrt(sum(v^2) / count + epsilon). */
int ao_normalize_head(float *values, const uint16_t *weights, uint32_t count, float epsilon);

/* prepare_rope (src/executor.cpp:43-58) with MachModel's divisors
 * (src/model.cpp:606-615): divisor_i = powf(1e7, 2i / 64), theta = position /
 * divisor_i, for i < 32. */
void ao_rope_table(uint32_t position, float *cosine /*32*/, float *sine /*32*/);
/* apply_rope (src/executor.cpp:60-72): pairs (i, i + 32), i < 32. */
void ao_apply_rope(float *values, const float *cosine, const float *sine);

/* grouped_query_online_attention (src/attention.cpp:38-229) with a
 * sequential dot: queries [query_heads][query_stride] (the first head_size
 * values of each row), keys/values [tokens][kv_heads][head_size], output
 * [query_heads][head_size]. */
int ao_grouped_attention(const float *queries, const float *keys, const float *values,
                         uint32_t tokens, uint32_t query_heads, uint32_t kv_heads,
                         uint32_t head_size, uint32_t query_stride, float *output);

/* l2_normalize (src/kernels.cpp:1075-1087). */
int ao_l2_normalize(float *values, uint32_t count, float epsilon);

/* The scalar gated_delta_update (src/simd.cpp:108-127): one state row. */
float ao_gated_delta_update(float *state, const float *query, const float *key, float value,
                            float beta, float decay, uint32_t count);

/* Full attention layer weights (adi::FullAttentionDescriptor,
 * include/adi/model.hpp:39-46): 16 query heads and 2 KV heads of 256. */
typedef struct {
    ao_ne_matrix query;         /* 8192 x hidden: per head 256 query, 256 gate */
    ao_ne_matrix key;           /* 512 x hidden */
    ao_ne_matrix value;         /* 512 x hidden */
    ao_ne_matrix output;        /* hidden x 4096 */
    const uint16_t *query_norm; /* 256 bf16 */
    const uint16_t *key_norm;   /* 256 bf16 */
} ao_full_attention;

/* full_attention_forward (src/executor.cpp:332-418) for the token at
 * `position`: keys and values hold `position` earlier entries of [2][256]
 * and receive this token's at index `position`. */
int ao_full_attention_forward(const ao_full_attention *layer, uint32_t position,
                              const float *input, float *output, float *keys, float *values);

/* Linear attention layer weights (adi::LinearAttentionDescriptor,
 * include/adi/model.hpp:48-58): Gated DeltaNet, 16 key heads and 32 value
 * heads of 128, a width-4 causal convolution over the 8192 qkv channels. */
typedef struct {
    ao_ne_matrix qkv;            /* 8192 x hidden */
    ao_ne_matrix gate;           /* 4096 x hidden */
    ao_ne_matrix output;         /* hidden x 4096 */
    ao_bf16_matrix alpha;        /* 32 x hidden */
    ao_bf16_matrix beta;         /* 32 x hidden */
    const uint16_t *convolution; /* 8192 x 4 bf16 */
    const uint16_t *alpha_bias;  /* 32 bf16 */
    const uint16_t *a_log;       /* 32 bf16 */
    const uint16_t *norm;        /* 128 bf16 */
} ao_linear_attention;

/* linear_attention_forward (src/executor.cpp:420-557): convolution [8192][3]
 * and recurrent [32][128][128] are the layer's state, updated in place (zero
 * for a new sequence). `lanes` is the bf16 dot order of alpha and beta. */
uint32_t ao_gated_delta_key_head(uint32_t value_head, uint32_t value_heads, uint32_t key_heads);
int ao_linear_attention_forward(const ao_linear_attention *layer, const float *input,
                                float *output, float *convolution, float *recurrent,
                                uint32_t lanes);

/* One decoder layer (adi::LayerDescriptor, include/adi/model.hpp:60-66). */
typedef struct {
    const uint16_t *input_norm;          /* hidden bf16 */
    const uint16_t *post_attention_norm; /* hidden bf16 */
    int full_attention;                  /* nonzero: full, else linear */
    ao_full_attention full;
    ao_linear_attention linear;
    ao_moe_layer moe;
} ao_decoder_layer;

/* decode_layer (src/executor.cpp:1473-1529) for the token at `position`:
 * hidden += attention(rms_norm(hidden, input_norm, 1, 1e-6)), then hidden +=
 * moe_forward(rms_norm(hidden, post_attention_norm, 1, 1e-6)). keys/values
 * (full) or convolution/recurrent (linear) are the layer's state. */
int ao_decode_layer(const ao_decoder_layer *layer, uint32_t position, float *hidden,
                    float *keys, float *values, float *convolution, float *recurrent,
                    uint32_t lanes);

#ifdef __cplusplus
}
#endif

#endif
