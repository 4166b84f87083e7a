/*
 * adi_oracle.c -- CPU restatement of ADI's packed-weight hot path.
 *
 * TEST INFRASTRUCTURE ONLY: the reference the HIP kernels are compared
 * against (tests, smoke check, benchmark CPU-baseline leg). Nothing in the
 * product links it.
 *
 * Reduction orders. The reference evaluates every expert and non-expert
 * projection in one order on every ISA (its SIMD batch kernels are compiled
 * with -ffp-contract=off and asserted bit-identical to the scalar loop,
 * tests/expert_batch_test.cpp:95-133, tests/ne_batch_test.cpp:79-117), so those
 * are restated in scalar order only. The int5 head dot and the bf16 dot depend
 * on the CPU ISA the reference selects at run time (src/simd.cpp:298-355):
 *   isa 1  scalar: sum += w*x sequentially (src/simd.cpp:65-96);
 *   isa 8  AVX2: eight lane sums, lane j takes columns j, j+8, ..., separate
 *          multiply and add, then the lanes summed 0..7 from 0.0f
 *          (src/simd_x86_avx2.cpp:22-30, 101-120, 172-193);
 *   isa 16 AVX-512: sixteen lane sums the same way, but the reference's
 *          AVX-512 translation unit is built without -ffp-contract=off
 *          (CMakeLists.txt:108-111) and GCC's C++ default contracts each lane
 *          multiply-add into one fused multiply-add (src/simd_x86_avx512.cpp:
 *          87-130, src/simd_x86_vbmi.cpp:77-116); the lanes are then summed
 *          0..15 from 0.0f. A trailing partial vector is added afterwards,
 *          fused as well.
 * This file itself is compiled with -ffp-contract=off; fused steps call fmaf.
 */
#include "adi_oracle.h"

#include <math.h>
#include <omp.h>
#include <stdlib.h>
#include <string.h>

#define TILE 16u
#define EXPERT_WORDS 24u
#define EXPERT_STATES 32u
#define NE_WORDS 64u
#define NE_STATES 128u
#define STATE_COUNT 65536u

static int is_power_of_two(uint32_t value) {
    return value != 0 && (value & (value - 1)) == 0;
}

static uint32_t float_bits(float value) {
    uint32_t bits;
    memcpy(&bits, &value, sizeof bits);
    return bits;
}

static float bits_float(uint32_t bits) {
    float value;
    memcpy(&value, &bits, sizeof value);
    return value;
}

/* ---- conversions (src/kernels.cpp:309-383) ---------------------------- */

float ao_f16_to_f32(uint16_t bits) {
    const uint32_t sign = (uint32_t)(bits & 0x8000u) << 16;
    const uint32_t exponent = (bits >> 10) & 0x1Fu;
    uint32_t mantissa = bits & 0x3FFu;
    if (exponent == 0x1Fu) {
        return bits_float(sign | 0x7F800000u | (mantissa << 13));
    }
    if (exponent != 0) {
        return bits_float(sign | ((exponent + 112u) << 23) | (mantissa << 13));
    }
    if (mantissa == 0) {
        return bits_float(sign);
    }
    /* Subnormal: value = mantissa * 2^-24, renormalised. */
    uint32_t e = 113u;
    while ((mantissa & 0x400u) == 0) {
        mantissa <<= 1;
        --e;
    }
    return bits_float(sign | (e << 23) | ((mantissa & 0x3FFu) << 13));
}

uint16_t ao_f32_to_f16(float value) {
    const uint32_t bits = float_bits(value);
    const uint16_t sign = (uint16_t)((bits >> 16) & 0x8000u);
    const uint32_t biased = (bits >> 23) & 0xFFu;
    const uint32_t mantissa = bits & 0x7FFFFFu;
    if (biased == 0xFFu) {
        /* Inf stays inf; NaN keeps its top payload bits and is forced quiet
         * by setting the lowest f16 mantissa bit. */
        return (uint16_t)(sign | 0x7C00u | (mantissa ? ((mantissa >> 13) | 1u) : 0u));
    }
    const int32_t exponent = (int32_t)biased - 112; /* f16 biased exponent */
    if (exponent >= 31) {
        return (uint16_t)(sign | 0x7C00u);
    }
    if (exponent <= 0) {
        if (exponent < -10) {
            return sign;
        }
        const uint32_t full = mantissa | 0x800000u;
        const uint32_t shift = (uint32_t)(14 - exponent);
        uint32_t q = full >> shift;
        const uint32_t rest = full & ((1u << shift) - 1u);
        const uint32_t half = 1u << (shift - 1u);
        if (rest > half || (rest == half && (q & 1u))) {
            ++q; /* may carry into the smallest normal: still correct */
        }
        return (uint16_t)(sign | q);
    }
    uint32_t result = ((uint32_t)exponent << 10) | (mantissa >> 13);
    const uint32_t rest = mantissa & 0x1FFFu;
    if (rest > 0x1000u || (rest == 0x1000u && (result & 1u))) {
        ++result; /* a mantissa carry bumps the exponent, up to inf */
    }
    return (uint16_t)(sign | result);
}

float ao_bf16_to_f32(uint16_t bits) {
    return bits_float((uint32_t)bits << 16);
}

/* ---- trellis walks ---------------------------------------------------- */

/* The expert tile stream is 24 big-endian-within-word u16 words = 384 bits.
 * State 0 is words[0]; each later state shifts in 12 fresh bits read at bit
 * 16 + 12*(i-1), wrapping at the end of the stream
 * (src/expert_trellis.hpp:20-31, 44-59). */
static uint32_t stream_bits(const uint16_t *words, uint32_t word_count,
                            uint32_t position, uint32_t width) {
    position %= word_count * 16u;
    const uint32_t word = position / 16u;
    const uint32_t offset = position % 16u;
    const uint32_t window = ((uint32_t)words[word] << 16) |
                            words[(word + 1u) % word_count];
    return (window >> (32u - offset - width)) & ((1u << width) - 1u);
}

void ao_expert_tile_states(const uint16_t *words, uint16_t *states) {
    uint32_t state = words[0];
    states[0] = (uint16_t)state;
    for (uint32_t index = 1; index < EXPERT_STATES; ++index) {
        const uint32_t position = 16u + (index - 1u) * 12u;
        state = ((state << 12) & 0xFFFFu) |
                stream_bits(words, EXPERT_WORDS, position, 12u);
        states[index] = (uint16_t)state;
    }
}

/* The NE stream is 64 words = 1024 bits with 8 fresh bits per transition
 * (src/ne_trellis.hpp:27-41). */
void ao_ne_tile_states(const uint16_t *words, uint16_t *states) {
    uint32_t state = words[0];
    states[0] = (uint16_t)state;
    for (uint32_t index = 1; index < NE_STATES; ++index) {
        const uint32_t position = 16u + (index - 1u) * 8u;
        state = ((state << 8) & 0xFFFFu) |
                stream_bits(words, NE_WORDS, position, 8u);
        states[index] = (uint16_t)state;
    }
}

/* ---- codec caches (src/codec_cache.cpp:17-147) ------------------------ */

static uint64_t state_product(uint32_t state) {
    return (uint64_t)state * (uint64_t)(state + 1u);
}

static float rounded_lattice(float value) {
    return ao_f16_to_f32(ao_f32_to_f16(value));
}

void ao_build_expert_state_values(const float *tlut, float *out) {
    for (uint32_t state = 0; state < STATE_COUNT; ++state) {
        const uint64_t p = state_product(state);
        const uint32_t row = (uint32_t)(p & 0x7FFFu);
        const int negative = (int)((p >> 15) & 1u);
        for (uint32_t c = 0; c < 8; ++c) {
            float value = tlut[(size_t)row * 8u + c];
            if (c == 0 && negative) {
                value = -value;
            }
            out[(size_t)state * 8u + c] = rounded_lattice(value);
        }
    }
}

void ao_build_ne_state_values(const float *tlut, float *out) {
    for (uint32_t state = 0; state < STATE_COUNT; ++state) {
        const uint64_t p = state_product(state);
        const uint32_t row = (uint32_t)((p >> 6) & 0x1FFu);
        const int negative = (int)((p >> 15) & 1u);
        for (uint32_t c = 0; c < 2; ++c) {
            float value = tlut[(size_t)row * 2u + c];
            if (c == 0 && negative) {
                value = -value;
            }
            out[(size_t)state * 2u + c] = rounded_lattice(value);
        }
    }
}

void ao_build_ne_signed_tlut(const float *tlut, float *out) {
    for (uint32_t index = 0; index < 1024u; ++index) {
        const uint32_t row = index & 0x1FFu;
        const int negative = (int)(index >> 9);
        for (uint32_t c = 0; c < 2; ++c) {
            float value = rounded_lattice(tlut[(size_t)row * 2u + c]);
            if (c == 0 && negative) {
                value = -value;
            }
            out[(size_t)index * 2u + c] = value;
        }
    }
}

/* Anti-diagonal wave numbering of the tile grid (src/codec_cache.cpp:
 * 117-147): waves are numbered first along the last tile column from the
 * bottom-right corner upwards, then along the first tile row leftwards. */
int ao_build_wave_indexes(uint32_t tile_rows, uint32_t tile_columns,
                          uint16_t *out) {
    if (tile_rows == 0 || tile_columns == 0 ||
        tile_rows + tile_columns > 65536u) {
        return AO_INVALID_ARGUMENT;
    }
    uint32_t wave = 0;
    for (uint32_t start = 0; start < tile_rows; ++start, ++wave) {
        int32_t row = (int32_t)(tile_rows - start - 1u);
        int32_t column = (int32_t)tile_columns - 1;
        for (; row < (int32_t)tile_rows && column >= 0; ++row, --column) {
            out[(size_t)row * tile_columns + (uint32_t)column] = (uint16_t)wave;
        }
    }
    for (uint32_t start = 0; start < tile_columns; ++start, ++wave) {
        int32_t row = 0;
        int32_t column = (int32_t)(tile_columns - start - 1u);
        for (; row < (int32_t)tile_rows && column >= 0; ++row, --column) {
            out[(size_t)row * tile_columns + (uint32_t)column] = (uint16_t)wave;
        }
    }
    return AO_OK;
}

/* ---- Hadamard (src/simd.cpp:48-63) ------------------------------------ */

int ao_hadamard(float *values, uint32_t count) {
    if (!is_power_of_two(count)) {
        return AO_INVALID_ARGUMENT;
    }
    for (uint32_t stride = 1; stride < count; stride *= 2u) {
        for (uint32_t block = 0; block < count; block += 2u * stride) {
            for (uint32_t index = 0; index < stride; ++index) {
                const float left = values[block + index];
                const float right = values[block + stride + index];
                values[block + index] = left + right;
                values[block + stride + index] = left - right;
            }
        }
    }
    const float scale = 1.0f / sqrtf((float)count);
    for (uint32_t index = 0; index < count; ++index) {
        values[index] *= scale;
    }
    return AO_OK;
}

/* ---- expert projection (src/kernels.cpp:192-264, 385-593) -------------- */

static int expert_shape_ok(const ao_expert_matrix *m) {
    if (!m || !is_power_of_two(m->rows) || !is_power_of_two(m->columns) ||
        m->rows % TILE || m->columns % TILE) {
        return 0;
    }
    return m->trellis && m->su_f16 && m->sv_f16 && m->wave_gamma_f16 &&
           (m->tlut || m->state_values);
}

static const float *expert_table(const ao_expert_matrix *m, float **owned) {
    *owned = NULL;
    if (m->state_values) {
        return m->state_values;
    }
    float *table = (float *)malloc((size_t)STATE_COUNT * 8u * sizeof(float));
    if (!table) {
        return NULL;
    }
    ao_build_expert_state_values(m->tlut, table);
    *owned = table;
    return table;
}

static int expert_accumulate_with(const ao_expert_matrix *m,
                                  const float *values, const float *x_hat,
                                  uint32_t batch, float *row_sums) {
    const uint32_t tile_rows = m->rows / TILE;
    const uint32_t tile_columns = m->columns / TILE;
    uint16_t *waves = (uint16_t *)malloc((size_t)tile_rows * tile_columns * 2u);
    if (!waves) {
        return AO_OUT_OF_MEMORY;
    }
    ao_build_wave_indexes(tile_rows, tile_columns, waves);
    uint16_t states[EXPERT_STATES];
    for (uint32_t tr = 0; tr < tile_rows; ++tr) {
        for (uint32_t b = 0; b < batch; ++b) {
            for (uint32_t r = 0; r < TILE; ++r) {
                row_sums[(size_t)b * m->rows + tr * TILE + r] = 0.0f;
            }
        }
        for (uint32_t tc = 0; tc < tile_columns; ++tc) {
            const size_t tile = (size_t)tr * tile_columns + tc;
            ao_expert_tile_states(m->trellis + tile * EXPERT_WORDS, states);
            const float gamma = ao_f16_to_f32(m->wave_gamma_f16[waves[tile]]);
            for (uint32_t b = 0; b < batch; ++b) {
                const float *x = x_hat + (size_t)b * m->columns + tc * TILE;
                float *sums = row_sums + (size_t)b * m->rows + tr * TILE;
                for (uint32_t r = 0; r < TILE; ++r) {
                    /* sixteen products into a fresh partial, the states of
                     * the row in walk order, components in order, then one
                     * gamma-scaled add into the row (src/kernels.cpp:443-476) */
                    float partial = 0.0f;
                    for (uint32_t step = 0; step < 2; ++step) {
                        const float *v =
                            values + (size_t)states[2u * r + step] * 8u;
                        for (uint32_t c = 0; c < 8; ++c) {
                            partial += v[c] * x[step * 8u + c];
                        }
                    }
                    sums[r] += partial * gamma;
                }
            }
        }
    }
    free(waves);
    return AO_OK;
}

int ao_expert_accumulate(const ao_expert_matrix *m, const float *x_hat,
                         uint32_t batch, float *row_sums) {
    if (!expert_shape_ok(m) || batch == 0 || !x_hat || !row_sums) {
        return AO_INVALID_ARGUMENT;
    }
    float *owned;
    const float *values = expert_table(m, &owned);
    if (!values) {
        return AO_OUT_OF_MEMORY;
    }
    const int status = expert_accumulate_with(m, values, x_hat, batch, row_sums);
    free(owned);
    return status;
}

int ao_expert_matmul(const ao_expert_matrix *m, const float *inputs,
                     uint32_t batch, float *outputs) {
    if (!expert_shape_ok(m) || batch == 0 || !inputs || !outputs) {
        return AO_INVALID_ARGUMENT;
    }
    float *owned;
    const float *values = expert_table(m, &owned);
    if (!values) {
        return AO_OUT_OF_MEMORY;
    }
    float *x_hat = (float *)malloc((size_t)batch * m->columns * sizeof(float));
    float *sums = (float *)malloc((size_t)batch * m->rows * sizeof(float));
    int status = (x_hat && sums) ? AO_OK : AO_OUT_OF_MEMORY;
    if (status == AO_OK) {
        for (uint32_t b = 0; b < batch; ++b) {
            float *xh = x_hat + (size_t)b * m->columns;
            const float *x = inputs + (size_t)b * m->columns;
            for (uint32_t c = 0; c < m->columns; ++c) {
                xh[c] = x[c] * ao_f16_to_f32(m->su_f16[c]);
            }
            ao_hadamard(xh, m->columns);
        }
        status = expert_accumulate_with(m, values, x_hat, batch, sums);
    }
    if (status == AO_OK) {
        for (uint32_t b = 0; b < batch; ++b) {
            float *z = sums + (size_t)b * m->rows;
            ao_hadamard(z, m->rows);
            float *y = outputs + (size_t)b * m->rows;
            for (uint32_t r = 0; r < m->rows; ++r) {
                y[r] = z[r] * ao_f16_to_f32(m->sv_f16[r]);
            }
        }
    }
    free(x_hat);
    free(sums);
    free(owned);
    return status;
}

int ao_expert_decode_tiles(const ao_expert_matrix *m, float *out) {
    if (!expert_shape_ok(m) || !out) {
        return AO_INVALID_ARGUMENT;
    }
    float *owned;
    const float *values = expert_table(m, &owned);
    if (!values) {
        return AO_OUT_OF_MEMORY;
    }
    const uint32_t tile_columns = m->columns / TILE;
    uint16_t states[EXPERT_STATES];
    for (uint32_t tr = 0; tr < m->rows / TILE; ++tr) {
        for (uint32_t tc = 0; tc < tile_columns; ++tc) {
            const size_t tile = (size_t)tr * tile_columns + tc;
            ao_expert_tile_states(m->trellis + tile * EXPERT_WORDS, states);
            for (uint32_t i = 0; i < EXPERT_STATES; ++i) {
                for (uint32_t c = 0; c < 8; ++c) {
                    const uint32_t row = tr * TILE + (i >> 1);
                    const uint32_t col = tc * TILE + (i & 1u) * 8u + c;
                    out[(size_t)row * m->columns + col] =
                        values[(size_t)states[i] * 8u + c];
                }
            }
        }
    }
    free(owned);
    return AO_OK;
}

/* ---- non-expert projection (src/kernels.cpp:103-183, 595-800) ---------- */

static int ne_shape_ok(const ao_ne_matrix *m) {
    if (!m || !is_power_of_two(m->rows) || !is_power_of_two(m->columns) ||
        m->rows % TILE || m->columns % TILE) {
        return 0;
    }
    return m->trellis && m->su && m->sv && (m->tlut || m->state_values);
}

static const float *ne_table(const ao_ne_matrix *m, float **owned) {
    *owned = NULL;
    if (m->state_values) {
        return m->state_values;
    }
    float *table = (float *)malloc((size_t)STATE_COUNT * 2u * sizeof(float));
    if (!table) {
        return NULL;
    }
    ao_build_ne_state_values(m->tlut, table);
    *owned = table;
    return table;
}

static void ne_accumulate_with(const ao_ne_matrix *m, const float *values,
                               const float *x_hat, uint32_t batch,
                               float *row_sums) {
    const uint32_t tile_rows = m->rows / TILE;
    const uint32_t tile_columns = m->columns / TILE;
    uint16_t states[NE_STATES];
    for (uint32_t tr = 0; tr < tile_rows; ++tr) {
        for (uint32_t b = 0; b < batch; ++b) {
            for (uint32_t r = 0; r < TILE; ++r) {
                row_sums[(size_t)b * m->rows + tr * TILE + r] = 0.0f;
            }
        }
        for (uint32_t tc = 0; tc < tile_columns; ++tc) {
            const size_t tile = (size_t)tr * tile_columns + tc;
            ao_ne_tile_states(m->trellis + tile * NE_WORDS, states);
            for (uint32_t i = 0; i < NE_STATES; ++i) {
                /* both weights rounded to fp32 first, then two separate
                 * adds into the row sum, which carries across tile columns
                 * (src/kernels.cpp:671-685) */
                const float w0 = values[(size_t)states[i] * 2u] * m->weight_scale;
                const float w1 = values[(size_t)states[i] * 2u + 1u] * m->weight_scale;
                const uint32_t r = i >> 3;
                const uint32_t col = tc * TILE + ((i & 7u) << 1);
                for (uint32_t b = 0; b < batch; ++b) {
                    const float *x = x_hat + (size_t)b * m->columns;
                    float *sum = row_sums + (size_t)b * m->rows + tr * TILE + r;
                    *sum += w0 * x[col];
                    *sum += w1 * x[col + 1u];
                }
            }
        }
    }
}

int ao_ne_accumulate(const ao_ne_matrix *m, const float *x_hat,
                     uint32_t batch, float *row_sums) {
    if (!ne_shape_ok(m) || batch == 0 || !x_hat || !row_sums) {
        return AO_INVALID_ARGUMENT;
    }
    float *owned;
    const float *values = ne_table(m, &owned);
    if (!values) {
        return AO_OUT_OF_MEMORY;
    }
    ne_accumulate_with(m, values, x_hat, batch, row_sums);
    free(owned);
    return AO_OK;
}

int ao_ne_matmul(const ao_ne_matrix *m, const float *inputs, uint32_t batch,
                 float *outputs) {
    if (!ne_shape_ok(m) || batch == 0 || !inputs || !outputs) {
        return AO_INVALID_ARGUMENT;
    }
    float *owned;
    const float *values = ne_table(m, &owned);
    if (!values) {
        return AO_OUT_OF_MEMORY;
    }
    float *x_hat = (float *)malloc((size_t)batch * m->columns * sizeof(float));
    float *sums = (float *)malloc((size_t)batch * m->rows * sizeof(float));
    if (!x_hat || !sums) {
        free(x_hat);
        free(sums);
        free(owned);
        return AO_OUT_OF_MEMORY;
    }
    for (uint32_t b = 0; b < batch; ++b) {
        float *xh = x_hat + (size_t)b * m->columns;
        const float *x = inputs + (size_t)b * m->columns;
        for (uint32_t c = 0; c < m->columns; ++c) {
            xh[c] = x[c] * (float)m->su[c];
        }
        ao_hadamard(xh, m->columns);
    }
    ne_accumulate_with(m, values, x_hat, batch, sums);
    for (uint32_t b = 0; b < batch; ++b) {
        float *z = sums + (size_t)b * m->rows;
        ao_hadamard(z, m->rows);
        float *y = outputs + (size_t)b * m->rows;
        for (uint32_t r = 0; r < m->rows; ++r) {
            y[r] = z[r] * (float)m->sv[r];
        }
    }
    free(x_hat);
    free(sums);
    free(owned);
    return AO_OK;
}

int ao_ne_decode_tiles(const ao_ne_matrix *m, float *out) {
    if (!ne_shape_ok(m) || !out) {
        return AO_INVALID_ARGUMENT;
    }
    float *owned;
    const float *values = ne_table(m, &owned);
    if (!values) {
        return AO_OUT_OF_MEMORY;
    }
    const uint32_t tile_columns = m->columns / TILE;
    uint16_t states[NE_STATES];
    for (uint32_t tr = 0; tr < m->rows / TILE; ++tr) {
        for (uint32_t tc = 0; tc < tile_columns; ++tc) {
            const size_t tile = (size_t)tr * tile_columns + tc;
            ao_ne_tile_states(m->trellis + tile * NE_WORDS, states);
            for (uint32_t i = 0; i < NE_STATES; ++i) {
                const uint32_t row = tr * TILE + (i >> 3);
                const uint32_t col = tc * TILE + ((i & 7u) << 1);
                out[(size_t)row * m->columns + col] =
                    values[(size_t)states[i] * 2u] * m->weight_scale;
                out[(size_t)row * m->columns + col + 1u] =
                    values[(size_t)states[i] * 2u + 1u] * m->weight_scale;
            }
        }
    }
    free(owned);
    return AO_OK;
}

/* ---- ISA-ordered reductions ------------------------------------------- */

static int isa_ok(uint32_t isa) {
    return isa == 1u || isa == 8u || isa == 16u;
}

/* One lane-ordered dot over `count` products w[k]*x[k], the weights supplied
 * by a callback-free array. */
static float ordered_dot(const float *w, const float *x, uint32_t count,
                         uint32_t isa) {
    if (isa == 1u) {
        float sum = 0.0f;
        for (uint32_t k = 0; k < count; ++k) {
            sum += w[k] * x[k];
        }
        return sum;
    }
    float lanes[16] = {0};
    uint32_t k = 0;
    for (; k + isa <= count; k += isa) {
        for (uint32_t j = 0; j < isa; ++j) {
            if (isa == 16u) {
                lanes[j] = fmaf(w[k + j], x[k + j], lanes[j]);
            } else {
                lanes[j] = lanes[j] + w[k + j] * x[k + j];
            }
        }
    }
    float sum = 0.0f;
    for (uint32_t j = 0; j < isa; ++j) {
        sum += lanes[j];
    }
    for (; k < count; ++k) {
        if (isa == 16u) {
            sum = fmaf(w[k], x[k], sum);
        } else {
            sum += w[k] * x[k];
        }
    }
    return sum;
}

float ao_bf16_dot(const uint16_t *weights, const float *input, uint32_t count,
                  uint32_t isa) {
    if (!isa_ok(isa)) {
        return NAN;
    }
    float *w = (float *)malloc((size_t)(count ? count : 1u) * sizeof(float));
    if (!w) {
        return NAN;
    }
    for (uint32_t k = 0; k < count; ++k) {
        w[k] = ao_bf16_to_f32(weights[k]);
    }
    const float result = ordered_dot(w, input, count, isa);
    free(w);
    return result;
}

int ao_bf16_matmul(const ao_bf16_matrix *m, const float *inputs,
                   uint32_t batch, float *outputs, uint32_t isa) {
    if (!m || !m->values || !inputs || !outputs || batch == 0 || !isa_ok(isa)) {
        return AO_INVALID_ARGUMENT;
    }
    float *w = (float *)malloc((size_t)(m->columns ? m->columns : 1u) * sizeof(float));
    if (!w) {
        return AO_OUT_OF_MEMORY;
    }
    for (uint32_t r = 0; r < m->rows; ++r) {
        for (uint32_t k = 0; k < m->columns; ++k) {
            w[k] = ao_bf16_to_f32(m->values[(size_t)r * m->columns + k]);
        }
        for (uint32_t b = 0; b < batch; ++b) {
            outputs[(size_t)b * m->rows + r] =
                ordered_dot(w, inputs + (size_t)b * m->columns, m->columns, isa);
        }
    }
    free(w);
    return AO_OK;
}

/* int5_g64: each row is columns/8 five-byte little-endian blocks of eight
 * 5-bit codes; weight = float(code - 16) * f16 scale of its 64-column group
 * (src/simd.cpp:65-86). */
int ao_head_matmul(const ao_head_chunk *h, const float *inputs, uint32_t batch,
                   float *outputs, uint32_t isa) {
    if (!h || !h->packed || !h->group_scale_f16 || !inputs || !outputs ||
        batch == 0 || h->columns % 64u || !isa_ok(isa) ||
        (h->protected_count && (!h->protected_rows || !h->protected_bf16))) {
        return AO_INVALID_ARGUMENT;
    }
    for (uint32_t p = 0; p < h->protected_count; ++p) {
        if (h->protected_rows[p] >= h->rows) {
            return AO_INVALID_ARGUMENT;
        }
    }
    const uint32_t bytes_per_row = h->columns / 8u * 5u;
    const uint32_t groups = h->columns / 64u;
    float *w = (float *)malloc((size_t)h->columns * sizeof(float));
    if (!w) {
        return AO_OUT_OF_MEMORY;
    }
    for (uint32_t r = 0; r < h->rows; ++r) {
        const uint8_t *row = h->packed + (size_t)r * bytes_per_row;
        for (uint32_t block = 0; block < h->columns / 8u; ++block) {
            uint64_t word = 0;
            for (uint32_t byte = 0; byte < 5; ++byte) {
                word |= (uint64_t)row[block * 5u + byte] << (byte * 8u);
            }
            for (uint32_t i = 0; i < 8; ++i) {
                const uint32_t col = block * 8u + i;
                const int32_t code = (int32_t)((word >> (i * 5u)) & 0x1Fu) - 16;
                const float scale = ao_f16_to_f32(
                    h->group_scale_f16[(size_t)r * groups + col / 64u]);
                w[col] = (float)code * scale;
            }
        }
        for (uint32_t b = 0; b < batch; ++b) {
            outputs[(size_t)b * h->rows + r] =
                ordered_dot(w, inputs + (size_t)b * h->columns, h->columns, isa);
        }
    }
    free(w);
    /* protected rows are overwritten by the bf16 dot (src/kernels.cpp:878-896) */
    for (uint32_t p = 0; p < h->protected_count; ++p) {
        const uint32_t r = h->protected_rows[p];
        for (uint32_t b = 0; b < batch; ++b) {
            outputs[(size_t)b * h->rows + r] = ao_bf16_dot(
                h->protected_bf16 + (size_t)p * h->columns,
                inputs + (size_t)b * h->columns, h->columns, isa);
        }
    }
    return AO_OK;
}

/* ---- elementwise (src/kernels.cpp:1052-1095) --------------------------- */

int ao_rms_norm(const float *input, const uint16_t *weight_bf16, uint32_t count,
                float weight_offset, float epsilon, float *output) {
    if (!input || !weight_bf16 || !output || count == 0) {
        return AO_INVALID_ARGUMENT;
    }
    float squares = 0.0f;
    for (uint32_t i = 0; i < count; ++i) {
        squares += input[i] * input[i];
    }
    const float scale = 1.0f / sqrtf(squares / (float)count + epsilon);
    for (uint32_t i = 0; i < count; ++i) {
        output[i] = input[i] * scale *
                    (weight_offset + ao_bf16_to_f32(weight_bf16[i]));
    }
    return AO_OK;
}

/* ---- embedding rows and the greedy choice ---------------------------------- */

/* src/kernels.cpp:802-845: per 64-column group, step = max(max - min, 1e-8)
 * / 15 and value = min + code * step (separate multiply and add), codes high
 * nibble first; then the row's bf16 exceptions, found by lower_bound over the
 * ascending flat indexes, overwrite their columns. */
int ao_embedding_row(const ao_embedding *e, uint32_t token, float *output) {
    if (!e || !output || token >= e->rows || e->columns % 64 != 0 || !e->packed ||
        !e->minimum_f16 || !e->maximum_f16 ||
        (e->exception_count && (!e->exception_indexes || !e->exception_bf16))) {
        return AO_INVALID_ARGUMENT;
    }
    const uint32_t groups = e->columns / 64;
    const uint8_t *row = e->packed + (size_t)token * e->columns / 2;
    const size_t scale_offset = (size_t)token * groups;
    for (uint32_t c = 0; c < e->columns; ++c) {
        const uint8_t byte = row[c / 2];
        const uint32_t code = c % 2 == 0 ? (uint32_t)(byte >> 4) : (uint32_t)(byte & 0x0F);
        const float minimum = ao_f16_to_f32(e->minimum_f16[scale_offset + c / 64]);
        const float maximum = ao_f16_to_f32(e->maximum_f16[scale_offset + c / 64]);
        const float span = maximum - minimum;
        const float step = (span < 1.0e-8f ? 1.0e-8f : span) / 15.0f;
        output[c] = minimum + (float)code * step;
    }
    const uint64_t first = (uint64_t)token * e->columns;
    const uint64_t last = first + e->columns;
    uint32_t lo = 0, hi = e->exception_count;
    while (lo < hi) { /* lower_bound */
        const uint32_t mid = lo + (hi - lo) / 2;
        if (e->exception_indexes[mid] < first) {
            lo = mid + 1;
        } else {
            hi = mid;
        }
    }
    for (uint32_t i = lo; i < e->exception_count && e->exception_indexes[i] < last; ++i) {
        output[e->exception_indexes[i] - first] = ao_bf16_to_f32(e->exception_bf16[i]);
    }
    return AO_OK;
}

uint64_t ao_fnv1a64(uint64_t hash, const void *data, size_t bytes) {
    const unsigned char *p = (const unsigned char *)data;
    for (size_t i = 0; i < bytes; ++i) {
        hash ^= p[i];
        hash *= 0x00000100000001B3ULL;
    }
    return hash;
}

uint32_t ao_argmax(const float *logits, uint32_t count) {
    uint32_t best = 0;
    for (uint32_t i = 1; i < count; ++i) {
        if (logits[best] < logits[i]) {
            best = i;
        }
    }
    return best;
}

/* src/generation.cpp:36-47: ascending order of this key is descending logit
 * order, with -0 folded into +0. */
static uint32_t descending_key(float value) {
    uint32_t bits = 0;
    if (value != 0.0f) {
        memcpy(&bits, &value, sizeof(bits));
    }
    const uint32_t ascending = (bits & 0x80000000u) ? ~bits : bits ^ 0x80000000u;
    return ~ascending;
}

static int by_key_then_index(const void *a, const void *b) {
    const uint64_t x = *(const uint64_t *)a, y = *(const uint64_t *)b;
    return x < y ? -1 : (x > y ? 1 : 0);
}

void ao_mt19937_64(uint64_t seed, uint32_t count, uint64_t *out) {
    enum { N = 312, M = 156 };
    const uint64_t upper = 0xFFFFFFFF80000000ull, lower = 0x7FFFFFFFull;
    uint64_t mt[N];
    mt[0] = seed;
    for (uint32_t i = 1; i < N; ++i) {
        mt[i] = 6364136223846793005ull * (mt[i - 1] ^ (mt[i - 1] >> 62)) + i;
    }
    uint32_t index = N;
    for (uint32_t k = 0; k < count; ++k) {
        if (index == N) {
            for (uint32_t i = 0; i < N; ++i) {
                const uint64_t x = (mt[i] & upper) | (mt[(i + 1) % N] & lower);
                const uint64_t shifted = (x >> 1) ^ ((x & 1u) ? 0xB5026F5AA96619E9ull : 0u);
                mt[i] = mt[(i + M) % N] ^ shifted;
            }
            index = 0;
        }
        uint64_t y = mt[index++];
        y ^= (y >> 29) & 0x5555555555555555ull;
        y ^= (y << 17) & 0x71D67FFFEDA60000ull;
        y ^= (y << 37) & 0xFFF7EEE000000000ull;
        y ^= y >> 43;
        out[k] = y;
    }
}

int ao_sample_token(const float *logits, uint32_t count, float temperature, float top_p,
                    uint64_t word, uint32_t *token) {
    if (!logits || !token || count == 0 || !isfinite(temperature) || !isfinite(top_p) ||
        temperature < 0.0f || (temperature > 0.0f && temperature < 1.0e-4f) ||
        temperature > 2.0f || top_p <= 0.0f || top_p > 1.0f) {
        return AO_INVALID_ARGUMENT;
    }
    for (uint32_t i = 0; i < count; ++i) {
        if (!isfinite(logits[i])) {
            return AO_INVALID_ARGUMENT;
        }
    }
    if (temperature == 0.0f) {
        *token = ao_argmax(logits, count);
        return AO_OK;
    }
    /* the reference's stable LSD radix sort over the key from ascending
     * indexes is the order of (key, index) */
    uint64_t *order = malloc(sizeof(uint64_t) * count);
    double *p = malloc(sizeof(double) * count);
    if (!order || !p) {
        free(order);
        free(p);
        return AO_OUT_OF_MEMORY;
    }
    for (uint32_t i = 0; i < count; ++i) {
        order[i] = ((uint64_t)descending_key(logits[i]) << 32) | i;
    }
    qsort(order, count, sizeof(uint64_t), by_key_then_index);
    const double maximum = (double)logits[(uint32_t)order[0]];
    double denominator = 0.0;
    for (uint32_t k = 0; k < count; ++k) {
        p[k] = exp(((double)logits[(uint32_t)order[k]] - maximum) / (double)temperature);
        denominator += p[k];
    }
    double cumulative = 0.0;
    uint32_t retained = 0;
    for (; retained < count; ++retained) {
        cumulative += p[retained] / denominator;
        if (cumulative >= top_p) {
            ++retained;
            break;
        }
    }
    if (retained == 0) {
        retained = 1;
    }
    double retained_sum = 0.0;
    for (uint32_t k = 0; k < retained; ++k) {
        retained_sum += p[k];
    }
    /* uniform_real_distribution<double>(0, retained_sum) over
     * generate_canonical<double, 53> of a 64-bit engine: one word */
    double u = (double)word * 0x1p-64;
    if (u >= 1.0) {
        u = nextafter(1.0, 0.0);
    }
    const double target = u * retained_sum + 0.0;
    double running = 0.0;
    *token = (uint32_t)order[retained - 1];
    for (uint32_t k = 0; k < retained; ++k) {
        running += p[k];
        if (target <= running) {
            *token = (uint32_t)order[k];
            break;
        }
    }
    free(order);
    free(p);
    return AO_OK;
}

float ao_silu(float value) {
    return value / (1.0f + expf(-value));
}

float ao_sigmoid(float value) {
    return 1.0f / (1.0f + expf(-value));
}

/* ---- routing (src/executor.cpp:193-229, 1221-1258) --------------------- */

/* Strict total order of top_experts: larger logit first, lower index on
 * ties. */
static int routes_before(const float *logits, uint32_t a, uint32_t b) {
    if (logits[a] == logits[b]) {
        return a < b;
    }
    return logits[a] > logits[b];
}

int ao_top_experts(const float *logits, uint32_t count, uint32_t *experts,
                   float *weights) {
    if (!logits || count < 8 || !experts || !weights) {
        return AO_INVALID_ARGUMENT;
    }
    /* Selection of the first eight of the total order: the same result as
     * the reference's partial_sort under the same comparator. */
    uint32_t chosen[8];
    uint32_t filled = 0;
    for (uint32_t e = 0; e < count; ++e) {
        uint32_t at = filled;
        while (at > 0 && routes_before(logits, e, chosen[at - 1])) {
            --at;
        }
        if (at >= 8) {
            continue;
        }
        const uint32_t last = filled < 8 ? filled : 7;
        for (uint32_t k = last; k > at; --k) {
            chosen[k] = chosen[k - 1];
        }
        chosen[at] = e;
        if (filled < 8) {
            ++filled;
        }
    }
    const float maximum = logits[chosen[0]];
    float selected[8];
    float sum = 0.0f;
    for (uint32_t i = 0; i < 8; ++i) {
        selected[i] = expf(logits[chosen[i]] - maximum);
        sum += selected[i];
    }
    if (sum < 6.103515625e-5f) {
        sum = 6.103515625e-5f;
    }
    for (uint32_t i = 0; i < 8; ++i) {
        experts[i] = chosen[i];
        weights[i] = selected[i] / sum;
    }
    return AO_OK;
}

int ao_moe_route(const float *logits, uint32_t batch, uint32_t experts,
                 uint32_t *route_expert, float *route_weight, uint32_t *counts,
                 uint32_t *offsets, uint32_t *grouped_batch,
                 uint32_t *route_to_grouped) {
    if (!logits || batch == 0 || experts < 8 || !route_expert || !route_weight ||
        !counts || !offsets || !grouped_batch || !route_to_grouped) {
        return AO_INVALID_ARGUMENT;
    }
    memset(counts, 0, (size_t)experts * sizeof(uint32_t));
    for (uint32_t b = 0; b < batch; ++b) {
        ao_top_experts(logits + (size_t)b * experts, experts,
                       route_expert + (size_t)b * 8u,
                       route_weight + (size_t)b * 8u);
        for (uint32_t r = 0; r < 8; ++r) {
            ++counts[route_expert[(size_t)b * 8u + r]];
        }
    }
    uint32_t *cursors = (uint32_t *)malloc((size_t)experts * sizeof(uint32_t));
    if (!cursors) {
        return AO_OUT_OF_MEMORY;
    }
    uint32_t total = 0;
    for (uint32_t e = 0; e < experts; ++e) {
        offsets[e] = total;
        cursors[e] = total;
        total += counts[e];
    }
    offsets[experts] = total;
    /* stable scatter in (token, route) order */
    for (uint32_t b = 0; b < batch; ++b) {
        for (uint32_t r = 0; r < 8; ++r) {
            const uint32_t e = route_expert[(size_t)b * 8u + r];
            const uint32_t position = cursors[e]++;
            grouped_batch[position] = b;
            route_to_grouped[(size_t)b * 8u + r] = position;
        }
    }
    free(cursors);
    return AO_OK;
}

/* ---- MoE block (src/executor.cpp:1181-1453) --------------------------- */

static void swiglu(float *gate, const float *up, size_t count) {
    for (size_t i = 0; i < count; ++i) {
        gate[i] = ao_silu(gate[i]) * up[i];
    }
}

int ao_moe_forward(const ao_moe_layer *L, const float *inputs, uint32_t batch,
                   const float *logit_bias, uint32_t isa, float *outputs,
                   uint32_t *route_expert_out, float *route_weight_out,
                   int threads) {
    if (!L || !inputs || !outputs || batch == 0 || !isa_ok(isa) ||
        !L->expert_matrices || L->experts < 8 ||
        L->router.rows != L->experts || L->router.columns != L->hidden ||
        L->shared_expert_gate.rows != 1 ||
        L->shared_expert_gate.columns != L->hidden) {
        return AO_INVALID_ARGUMENT;
    }
    const uint32_t H = L->hidden, I = L->expert_hidden, E = L->experts;
    const size_t positions = (size_t)batch * 8u;
    int status = AO_OK;

    float *logits = (float *)malloc((size_t)batch * E * sizeof(float));
    uint32_t *rexp = (uint32_t *)malloc(positions * sizeof(uint32_t));
    float *rw = (float *)malloc(positions * sizeof(float));
    uint32_t *counts = (uint32_t *)malloc((size_t)E * sizeof(uint32_t));
    uint32_t *offsets = (uint32_t *)malloc(((size_t)E + 1u) * sizeof(uint32_t));
    uint32_t *grouped = (uint32_t *)malloc(positions * sizeof(uint32_t));
    uint32_t *r2g = (uint32_t *)malloc(positions * sizeof(uint32_t));
    float *gathered = (float *)malloc(positions * H * sizeof(float));
    float *gate = (float *)malloc(positions * I * sizeof(float));
    float *up = (float *)malloc(positions * I * sizeof(float));
    float *projected = (float *)malloc(positions * H * sizeof(float));
    float *table = (float *)malloc((size_t)STATE_COUNT * 8u * sizeof(float));
    if (!logits || !rexp || !rw || !counts || !offsets || !grouped || !r2g ||
        !gathered || !gate || !up || !projected || !table) {
        status = AO_OUT_OF_MEMORY;
        goto done;
    }

    status = ao_bf16_matmul(&L->router, inputs, batch, logits, isa);
    if (status != AO_OK) {
        goto done;
    }
    if (logit_bias) {
        for (uint32_t b = 0; b < batch; ++b) {
            for (uint32_t e = 0; e < E; ++e) {
                logits[(size_t)b * E + e] += logit_bias[e];
            }
        }
    }
    status = ao_moe_route(logits, batch, E, rexp, rw, counts, offsets, grouped, r2g);
    if (status != AO_OK) {
        goto done;
    }
    for (size_t p = 0; p < positions; ++p) {
        memcpy(gathered + p * H, inputs + (size_t)grouped[p] * H, H * sizeof(float));
    }
    /* The reference splits an expert's rows into tasks of at most 32; rows are
     * independent and a batched call equals per-row calls bit for bit
     * (tests/expert_batch_test.cpp:95-133), so one call per expert computes
     * the same values. The expert state table is model-wide
     * (src/model.cpp:549-551): build it once from the first expert's TLUT. */
    ao_build_expert_state_values(L->expert_matrices[0].tlut, table);
    {
        int failed = 0;
        int64_t e;
        const int workers = threads > 0 ? threads : omp_get_max_threads();
#pragma omp parallel for schedule(dynamic) num_threads(workers) reduction(| : failed)
        for (e = 0; e < (int64_t)E; ++e) {
            const uint32_t rows = counts[e];
            if (rows == 0) {
                continue;
            }
            const size_t begin = offsets[e];
            ao_expert_matrix g = L->expert_matrices[(size_t)e * 3u + 0u];
            ao_expert_matrix u = L->expert_matrices[(size_t)e * 3u + 1u];
            ao_expert_matrix d = L->expert_matrices[(size_t)e * 3u + 2u];
            g.state_values = u.state_values = d.state_values = table;
            failed |= ao_expert_matmul(&g, gathered + begin * H, rows, gate + begin * I) != AO_OK;
            failed |= ao_expert_matmul(&u, gathered + begin * H, rows, up + begin * I) != AO_OK;
            swiglu(gate + begin * I, up + begin * I, (size_t)rows * I);
            failed |= ao_expert_matmul(&d, gate + begin * I, rows, projected + begin * H) != AO_OK;
        }
        if (failed) {
            status = AO_INVALID_ARGUMENT;
            goto done;
        }
    }
    /* route-order combine (src/executor.cpp:1373-1399) */
    memset(outputs, 0, (size_t)batch * H * sizeof(float));
    for (uint32_t b = 0; b < batch; ++b) {
        float *out = outputs + (size_t)b * H;
        for (uint32_t r = 0; r < 8; ++r) {
            const float *src = projected + (size_t)r2g[(size_t)b * 8u + r] * H;
            const float w = rw[(size_t)b * 8u + r];
            for (uint32_t i = 0; i < H; ++i) {
                out[i] += w * src[i];
            }
        }
    }
    /* shared expert and its sigmoid gate (src/executor.cpp:1401-1452) */
    {
        float *sg = (float *)malloc((size_t)batch * I * sizeof(float));
        float *su = (float *)malloc((size_t)batch * I * sizeof(float));
        float *sd = (float *)malloc((size_t)batch * H * sizeof(float));
        float *sgate = (float *)malloc((size_t)batch * sizeof(float));
        if (!sg || !su || !sd || !sgate) {
            status = AO_OUT_OF_MEMORY;
        } else if ((status = ao_ne_matmul(&L->shared_gate, inputs, batch, sg)) == AO_OK &&
                   (status = ao_ne_matmul(&L->shared_up, inputs, batch, su)) == AO_OK) {
            swiglu(sg, su, (size_t)batch * I);
            if ((status = ao_ne_matmul(&L->shared_down, sg, batch, sd)) == AO_OK &&
                (status = ao_bf16_matmul(&L->shared_expert_gate, inputs, batch, sgate, isa)) == AO_OK) {
                for (uint32_t b = 0; b < batch; ++b) {
                    const float w = ao_sigmoid(sgate[b]);
                    for (uint32_t i = 0; i < H; ++i) {
                        outputs[(size_t)b * H + i] += w * sd[(size_t)b * H + i];
                    }
                }
            }
        }
        free(sg);
        free(su);
        free(sd);
        free(sgate);
    }
    if (status == AO_OK) {
        if (route_expert_out) {
            memcpy(route_expert_out, rexp, positions * sizeof(uint32_t));
        }
        if (route_weight_out) {
            memcpy(route_weight_out, rw, positions * sizeof(float));
        }
    }
done:
    free(logits);
    free(rexp);
    free(rw);
    free(counts);
    free(offsets);
    free(grouped);
    free(r2g);
    free(gathered);
    free(gate);
    free(up);
    free(projected);
    free(table);
    return status;
}

/* ---- attention of one decode token ----------------------------------------- */

/* src/executor.cpp:25-41 */
int ao_normalize_head(float *values, const uint16_t *weights, uint32_t count, float epsilon) {
    if (!values || !weights || count == 0) {
        return AO_INVALID_ARGUMENT;
    }
    float squares = 0.0f;
    for (uint32_t i = 0; i < count; ++i) {
        squares += values[i] * values[i];
    }
    const float scale = 1.0f / sqrtf(squares / (float)count + epsilon);
    for (uint32_t i = 0; i < count; ++i) {
        values[i] *= scale * (1.0f + ao_bf16_to_f32(weights[i]));
    }
    return AO_OK;
}

/* src/executor.cpp:43-58, src/model.cpp:606-615 */
void ao_rope_table(uint32_t position, float *cosine, float *sine) {
    for (uint32_t i = 0; i < 32; ++i) {
        const float divisor = powf(10000000.0f, 2.0f * (float)i / 64.0f);
        const float theta = (float)position / divisor;
        cosine[i] = cosf(theta);
        sine[i] = sinf(theta);
    }
}

/* src/executor.cpp:60-72 */
void ao_apply_rope(float *values, const float *cosine, const float *sine) {
    for (uint32_t i = 0; i < 32; ++i) {
        const float first = values[i];
        const float second = values[i + 32];
        values[i] = first * cosine[i] - second * sine[i];
        values[i + 32] = second * cosine[i] + first * sine[i];
    }
}

/* update_online_softmax (src/attention.cpp:15-35) */
static void online_softmax_step(float score, const float *value, uint32_t count,
                                float *maximum, float *denominator, float *attended) {
    if (score <= *maximum) {
        const float weight = expf(score - *maximum);
        *denominator += weight;
        for (uint32_t i = 0; i < count; ++i) {
            attended[i] += value[i] * weight;
        }
        return;
    }
    const float previous_scale = expf(*maximum - score);
    *denominator = *denominator * previous_scale + 1.0f;
    for (uint32_t i = 0; i < count; ++i) {
        attended[i] = attended[i] * previous_scale + value[i];
    }
    *maximum = score;
}

/* src/attention.cpp:38-229: per query head, tokens in order, then * 1/den */
int ao_grouped_attention(const float *queries, const float *keys, const float *values,
                         uint32_t tokens, uint32_t query_heads, uint32_t kv_heads,
                         uint32_t head_size, uint32_t query_stride, float *output) {
    if (!queries || !keys || !values || !output || tokens == 0 || kv_heads == 0 ||
        head_size == 0 || query_heads % kv_heads != 0 || query_stride < head_size) {
        return AO_INVALID_ARGUMENT;
    }
    const uint32_t group = query_heads / kv_heads;
    const float score_scale = 1.0f / sqrtf((float)head_size);
    for (uint32_t h = 0; h < query_heads; ++h) {
        const uint32_t kv = h / group;
        const float *q = queries + (size_t)h * query_stride;
        float *attended = output + (size_t)h * head_size;
        memset(attended, 0, head_size * sizeof(float));
        float maximum = -INFINITY, denominator = 0.0f;
        for (uint32_t t = 0; t < tokens; ++t) {
            const size_t at = ((size_t)t * kv_heads + kv) * head_size;
            float dot = 0.0f;
            for (uint32_t i = 0; i < head_size; ++i) {
                dot += q[i] * keys[at + i];
            }
            online_softmax_step(dot * score_scale, values + at, head_size, &maximum, &denominator,
                                attended);
        }
        const float inverse = 1.0f / denominator;
        for (uint32_t i = 0; i < head_size; ++i) {
            attended[i] *= inverse;
        }
    }
    return AO_OK;
}

/* src/kernels.cpp:1075-1087 */
int ao_l2_normalize(float *values, uint32_t count, float epsilon) {
    if (!values || count == 0 || epsilon < 0.0f) {
        return AO_INVALID_ARGUMENT;
    }
    float squares = 0.0f;
    for (uint32_t i = 0; i < count; ++i) {
        squares += values[i] * values[i];
    }
    const float scale = 1.0f / sqrtf(squares + epsilon);
    for (uint32_t i = 0; i < count; ++i) {
        values[i] *= scale;
    }
    return AO_OK;
}

/* src/simd.cpp:108-127 */
float ao_gated_delta_update(float *state, const float *query, const float *key, float value,
                            float beta, float decay, uint32_t count) {
    float prediction = 0.0f;
    for (uint32_t i = 0; i < count; ++i) {
        state[i] *= decay;
        prediction += state[i] * key[i];
    }
    const float delta = (value - prediction) * beta;
    float attended = 0.0f;
    for (uint32_t i = 0; i < count; ++i) {
        state[i] += key[i] * delta;
        attended += state[i] * query[i];
    }
    return attended;
}

/* src/executor.cpp:332-418 */
int ao_full_attention_forward(const ao_full_attention *L, uint32_t position,
                              const float *input, float *output, float *keys, float *values) {
    enum { query_heads = 16, kv_heads = 2, head_size = 256, stride = 512 };
    const float epsilon = 1.0e-6f;
    if (!L || !input || !output || !keys || !values || L->query.rows != query_heads * stride ||
        L->key.rows != kv_heads * head_size || L->value.rows != kv_heads * head_size ||
        L->output.columns != query_heads * head_size || !L->query_norm || !L->key_norm) {
        return AO_INVALID_ARGUMENT;
    }
    float *query_gate = malloc(sizeof(float) * query_heads * stride);
    float *attended = malloc(sizeof(float) * query_heads * head_size);
    float *key = keys + (size_t)position * kv_heads * head_size;
    float *value = values + (size_t)position * kv_heads * head_size;
    int rc = query_gate && attended ? AO_OK : AO_INVALID_ARGUMENT;
    if (rc == AO_OK) {
        rc = ao_ne_matmul(&L->query, input, 1, query_gate);
    }
    if (rc == AO_OK) {
        rc = ao_ne_matmul(&L->key, input, 1, key);
    }
    if (rc == AO_OK) {
        rc = ao_ne_matmul(&L->value, input, 1, value);
    }
    if (rc == AO_OK) {
        float cosine[32], sine[32];
        ao_rope_table(position, cosine, sine);
        for (uint32_t h = 0; h < query_heads; ++h) {
            ao_normalize_head(query_gate + (size_t)h * stride, L->query_norm, head_size, epsilon);
            ao_apply_rope(query_gate + (size_t)h * stride, cosine, sine);
        }
        for (uint32_t h = 0; h < kv_heads; ++h) {
            ao_normalize_head(key + (size_t)h * head_size, L->key_norm, head_size, epsilon);
            ao_apply_rope(key + (size_t)h * head_size, cosine, sine);
        }
        rc = ao_grouped_attention(query_gate, keys, values, position + 1, query_heads, kv_heads,
                                  head_size, stride, attended);
    }
    if (rc == AO_OK) {
        for (uint32_t h = 0; h < query_heads; ++h) {
            for (uint32_t i = 0; i < head_size; ++i) {
                attended[h * head_size + i] *=
                    ao_sigmoid(query_gate[(size_t)h * stride + head_size + i]);
            }
        }
        rc = ao_ne_matmul(&L->output, attended, 1, output);
    }
    free(query_gate);
    free(attended);
    return rc;
}

/* gated_delta_key_head (src/executor.cpp:231-240): the key head a value head
 * reads; UINT32_MAX for an invalid geometry. */
uint32_t ao_gated_delta_key_head(uint32_t value_head, uint32_t value_heads, uint32_t key_heads) {
    if (key_heads == 0 || value_heads == 0 || value_heads % key_heads != 0 || value_head >= value_heads) {
        return UINT32_MAX;
    }
    return value_head / (value_heads / key_heads);
}

/* src/executor.cpp:420-557, with gated_delta_recurrent (157-184) and
 * gated_delta_head (121-155) */
int ao_linear_attention_forward(const ao_linear_attention *L, const float *input,
                                float *output, float *convolution, float *recurrent,
                                uint32_t lanes) {
    enum { key_heads = 16, value_heads = 32, head_size = 128, qk_size = key_heads * head_size,
           value_size = value_heads * head_size, channels = 2 * qk_size + value_size };
    const float epsilon = 1.0e-6f;
    if (!L || !input || !output || !convolution || !recurrent || L->qkv.rows != channels ||
        L->gate.rows != value_size || L->output.columns != value_size ||
        L->alpha.rows != value_heads || L->beta.rows != value_heads || !L->convolution ||
        !L->alpha_bias || !L->a_log || !L->norm) {
        return AO_INVALID_ARGUMENT;
    }
    float *qkv = malloc(sizeof(float) * channels);
    float *gate = malloc(sizeof(float) * value_size);
    float *convolved = malloc(sizeof(float) * channels);
    float *recurrent_output = malloc(sizeof(float) * value_size);
    float *normalized = malloc(sizeof(float) * value_size);
    float alpha[value_heads], beta[value_heads];
    int rc = qkv && gate && convolved && recurrent_output && normalized ? AO_OK
                                                                       : AO_INVALID_ARGUMENT;
    if (rc == AO_OK) {
        rc = ao_ne_matmul(&L->qkv, input, 1, qkv);
    }
    if (rc == AO_OK) {
        rc = ao_ne_matmul(&L->gate, input, 1, gate);
    }
    if (rc == AO_OK) {
        rc = ao_bf16_matmul(&L->alpha, input, 1, alpha, lanes);
    }
    if (rc == AO_OK) {
        rc = ao_bf16_matmul(&L->beta, input, 1, beta, lanes);
    }
    if (rc == AO_OK) {
        for (uint32_t c = 0; c < channels; ++c) {
            float *history = convolution + (size_t)c * 3;
            const uint16_t *w = L->convolution + (size_t)c * 4;
            float v = 0.0f;
            for (uint32_t i = 0; i < 3; ++i) {
                v += history[i] * ao_bf16_to_f32(w[i]);
            }
            v += qkv[c] * ao_bf16_to_f32(w[3]);
            convolved[c] = ao_silu(v);
            history[0] = history[1];
            history[1] = history[2];
            history[2] = qkv[c];
        }
        for (uint32_t h = 0; h < key_heads; ++h) {
            ao_l2_normalize(convolved + (size_t)h * head_size, head_size, epsilon);
            ao_l2_normalize(convolved + qk_size + (size_t)h * head_size, head_size, epsilon);
        }
        const float output_scale = 1.0f / sqrtf((float)head_size);
        const float *query = convolved, *key = convolved + qk_size, *value = convolved + 2 * qk_size;
        for (uint32_t h = 0; h < value_heads; ++h) {
            const uint32_t kh = ao_gated_delta_key_head(h, value_heads, key_heads);
            const float *q = query + (size_t)kh * head_size;
            const float *k = key + (size_t)kh * head_size;
            const float *v = value + (size_t)h * head_size;
            const float beta_value = ao_sigmoid(beta[h]);
            const float biased = alpha[h] + ao_bf16_to_f32(L->alpha_bias[h]);
            const float softplus = biased > 20.0f ? biased : log1pf(expf(biased));
            const float decay = expf(-expf(ao_bf16_to_f32(L->a_log[h])) * softplus);
            for (uint32_t r = 0; r < head_size; ++r) {
                float *row = recurrent + ((size_t)h * head_size + r) * head_size;
                recurrent_output[(size_t)h * head_size + r] =
                    ao_gated_delta_update(row, q, k, v[r], beta_value, decay, head_size) *
                    output_scale;
            }
        }
        for (uint32_t h = 0; h < value_heads && rc == AO_OK; ++h) {
            float *dst = normalized + (size_t)h * head_size;
            rc = ao_rms_norm(recurrent_output + (size_t)h * head_size, L->norm, head_size, 0.0f,
                             epsilon, dst);
            for (uint32_t i = 0; i < head_size; ++i) {
                dst[i] *= ao_silu(gate[(size_t)h * head_size + i]);
            }
        }
    }
    if (rc == AO_OK) {
        rc = ao_ne_matmul(&L->output, normalized, 1, output);
    }
    free(qkv);
    free(gate);
    free(convolved);
    free(recurrent_output);
    free(normalized);
    return rc;
}

/* src/executor.cpp:1473-1529 */
int ao_decode_layer(const ao_decoder_layer *L, uint32_t position, float *hidden,
                    float *keys, float *values, float *convolution, float *recurrent,
                    uint32_t lanes) {
    if (!L || !hidden || !L->input_norm || !L->post_attention_norm) {
        return AO_INVALID_ARGUMENT;
    }
    const uint32_t n = L->moe.hidden;
    float *normalized = malloc(sizeof(float) * n);
    float *branch = malloc(sizeof(float) * n);
    int rc = normalized && branch ? AO_OK : AO_INVALID_ARGUMENT;
    if (rc == AO_OK) {
        rc = ao_rms_norm(hidden, L->input_norm, n, 1.0f, 1.0e-6f, normalized);
    }
    if (rc == AO_OK) {
        rc = L->full_attention
                 ? ao_full_attention_forward(&L->full, position, normalized, branch, keys, values)
                 : ao_linear_attention_forward(&L->linear, normalized, branch, convolution,
                                               recurrent, lanes);
    }
    if (rc == AO_OK) {
        for (uint32_t i = 0; i < n; ++i) {
            hidden[i] += branch[i];
        }
        rc = ao_rms_norm(hidden, L->post_attention_norm, n, 1.0f, 1.0e-6f, normalized);
    }
    if (rc == AO_OK) {
        rc = ao_moe_forward(&L->moe, normalized, 1, NULL, lanes, branch, NULL, NULL, 1);
    }
    if (rc == AO_OK) {
        for (uint32_t i = 0; i < n; ++i) {
            hidden[i] += branch[i];
        }
    }
    free(normalized);
    free(branch);
    return rc;
}
