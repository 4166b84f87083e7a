// backend_driver.cpp -- TEST INFRASTRUCTURE ONLY.
//
// C entry points that run one adi::Backend entry, from either the reference's
// cpu_backend() (src/backend.cpp:11-26) or the HIP library's hip_backend(), on host
// arrays, so the parity tests can drive the reference's own dispatch table.
// Linked with the reference's compiled runtime into _ref/libadi_backend.so.
// Every function returns 0, 1 for std::invalid_argument or 2 for any other
// exception, whose message goes to `error`.
#include "adi/backend.hpp"
#include "hip_backend.hpp"

#include <cstdio>
#include <cstring>
#include <span>
#include <stdexcept>

namespace {

const adi::Backend &table(int hip) { return hip ? adi::hip_backend() : adi::cpu_backend(); }

template <typename F>
int run(char *error, std::size_t error_size, F &&call) {
    try {
        call();
        return 0;
    } catch (const std::invalid_argument &e) {
        std::snprintf(error, error_size, "%s", e.what());
        return 1;
    } catch (const std::exception &e) {
        std::snprintf(error, error_size, "%s", e.what());
        return 2;
    }
}

}  // namespace

extern "C" {

int bd_backend_name(int hip, char *out, std::size_t out_size) {
    return run(out, out_size, [&] {
        const std::string_view name = table(hip).name;
        std::snprintf(out, out_size, "%.*s", static_cast<int>(name.size()), name.data());
    });
}

// Sizes are passed explicitly so that tests can hand over mismatched spans.
int bd_expert_matmul(int hip, std::uint32_t rows, std::uint32_t columns, const std::uint16_t *trellis,
                     std::size_t trellis_size, const std::uint16_t *su, std::size_t su_size,
                     const std::uint16_t *sv, std::size_t sv_size, const std::uint16_t *gamma,
                     std::size_t gamma_size, const float *tlut, const float *inputs,
                     std::size_t inputs_size, std::uint32_t batch, float *outputs,
                     std::size_t outputs_size, char *error, std::size_t error_size) {
    return run(error, error_size, [&] {
        adi::MachExpertMatrix m{rows, columns, {trellis, trellis_size}, {su, su_size}, {sv, sv_size},
                                {gamma, gamma_size}, {tlut, std::size_t(32768) * 8}};
        adi::ExpertScratch scratch;
        if (batch == 1) {
            table(hip).expert_matvec(m, {inputs, inputs_size}, {outputs, outputs_size}, scratch);
        } else {
            table(hip).expert_matmul(m, {inputs, inputs_size}, batch, {outputs, outputs_size}, scratch);
        }
    });
}

int bd_ne_matmul(int hip, std::uint32_t rows, std::uint32_t columns, const std::uint16_t *trellis,
                 std::size_t trellis_size, const std::int8_t *su, const std::int8_t *sv,
                 float weight_scale, const float *tlut, const float *inputs, std::size_t inputs_size,
                 std::uint32_t batch, float *outputs, std::size_t outputs_size, char *error,
                 std::size_t error_size) {
    return run(error, error_size, [&] {
        adi::MachNeMatrix m{rows, columns, {trellis, trellis_size}, {su, columns}, {sv, rows},
                            weight_scale, {tlut, std::size_t(512) * 2}};
        adi::ExpertScratch scratch;
        if (batch == 1) {
            table(hip).ne_matvec(m, {inputs, inputs_size}, {outputs, outputs_size}, scratch);
        } else {
            table(hip).ne_matmul(m, {inputs, inputs_size}, batch, {outputs, outputs_size}, scratch);
        }
    });
}

int bd_head_matmul(int hip, std::uint32_t rows, std::uint32_t columns, const std::uint8_t *packed,
                   const std::uint16_t *scales, const std::uint32_t *protected_rows,
                   const std::uint16_t *protected_bf16, std::size_t protected_count,
                   const float *inputs, std::size_t inputs_size, std::uint32_t batch, float *outputs,
                   std::size_t outputs_size, char *error, std::size_t error_size) {
    return run(error, error_size, [&] {
        adi::MachHeadChunk h{rows, columns, {packed, std::size_t(rows) * columns / 8 * 5},
                             {scales, std::size_t(rows) * columns / 64},
                             {protected_rows, protected_count},
                             {protected_bf16, protected_count * columns}};
        if (batch == 1) {
            table(hip).head_matvec(h, {inputs, inputs_size}, {outputs, outputs_size});
        } else {
            table(hip).head_matmul(h, {inputs, inputs_size}, batch, {outputs, outputs_size});
        }
    });
}

int bd_bf16_matmul(int hip, std::uint32_t rows, std::uint32_t columns, const std::uint16_t *values,
                   const float *inputs, std::size_t inputs_size, std::uint32_t batch, float *outputs,
                   std::size_t outputs_size, char *error, std::size_t error_size) {
    return run(error, error_size, [&] {
        adi::Bf16Matrix m{rows, columns, {values, std::size_t(rows) * columns}};
        if (batch == 1) {
            table(hip).dense_bf16_matvec(m, {inputs, inputs_size}, {outputs, outputs_size});
        } else {
            table(hip).dense_bf16_matmul(m, {inputs, inputs_size}, batch, {outputs, outputs_size});
        }
    });
}

int bd_embedding_row(int hip, std::uint32_t rows, std::uint32_t columns, const std::uint8_t *packed,
                     const std::uint16_t *minimum, const std::uint16_t *maximum,
                     const std::uint32_t *indexes, const std::uint16_t *bits,
                     std::size_t exceptions, std::uint32_t token, float *output,
                     std::size_t output_size, char *error, std::size_t error_size) {
    return run(error, error_size, [&] {
        const std::size_t groups = columns / 64;
        const adi::MachEmbedding e{rows,
                                   columns,
                                   {packed, std::size_t(rows) * columns / 2},
                                   {minimum, std::size_t(rows) * groups},
                                   {maximum, std::size_t(rows) * groups},
                                   {indexes, exceptions},
                                   {bits, exceptions}};
        table(hip).embedding_row(e, token, {output, output_size});
    });
}

int bd_rms_norm(int hip, const float *input, const std::uint16_t *weight, std::size_t count,
                float offset, float epsilon, float *output, char *error, std::size_t error_size) {
    return run(error, error_size, [&] {
        table(hip).normalize_rms({input, count}, {weight, count}, offset, epsilon, {output, count});
    });
}

int bd_release_weights(char *error, std::size_t error_size) {
    return run(error, error_size, [&] { adi::hip_backend_release_weights(); });
}

}  // extern "C"
