// moe.hip -- one MoE block on the device: moe_forward / moe_forward_batch
// (src/executor.cpp:242-330, 1181-1453).
//
// Launch sequence for a batch of B rows (P = 8B route positions):
//   1  router logits, ISA-ordered bf16 (bit-exact)       [B, E]
//      shared-expert gate logit, same kernel              [B]
//   2  top_experts (+ optional fp32 logit bias)           routes [P]
//   3  stable counting sort                               offsets, grouped_batch,
//                                                         route_to_grouped, active list
//   4  prologues x_hat = H(su_e * x[grouped_batch[p]]) for gate and up, and
//      H(SU * x) for the shared expert
//   5  decode-GEMV gate/up over the active experts, NE GEMV shared gate/up
//   6  SwiGLU: g = sv*H(Zg), u = sv*H(Zu), a = silu(g)*u, x_hat = H(su_d * a)
//   7  decode-GEMV down over the active experts, NE GEMV shared down
//   8  combine per row: sum_r w_r * sv_d*H(Zd[p_r]) in route order, then
//      + sigmoid(gate) * SV*H(Zshared)
// Expert work is sized for the worst case (min(P, E) active experts); blocks
// past the device-side active count return at once, so the host never waits
// for the routing.
#include "dense.hpp"
#include "projection.hpp"

namespace adi_hip {
namespace {

__device__ __forceinline__ float silu(float v) { return v / (1.0f + expf(-v)); }
__device__ __forceinline__ float sigmoid(float v) { return 1.0f / (1.0f + expf(-v)); }

template <typename Scale>
__device__ __forceinline__ float to_float(Scale s);
template <>
__device__ __forceinline__ float to_float<uint16_t>(uint16_t s) { return half_bits_to_float(s); }
template <>
__device__ __forceinline__ float to_float<int8_t>(int8_t s) { return static_cast<float>(s); }

// One block per vector v of the intermediate width I.
template <typename Scale>
__global__ __launch_bounds__(256) void k_swiglu(
    const float *__restrict__ z_gate, const float *__restrict__ z_up, uint32_t splits,
    size_t split_stride, uint32_t n, const Scale *__restrict__ sv_gate,
    const Scale *__restrict__ sv_up, const Scale *__restrict__ su_down, uint32_t stride,
    const uint32_t *__restrict__ matrix_index, float scale, float *__restrict__ x_hat) {
    extern __shared__ float lds[];
    float *g = lds;
    float *u = lds + n;
    const uint32_t vec = blockIdx.x;
    const size_t mat = matrix_index != nullptr ? matrix_index[vec] : 0u;
    const float *zg = z_gate + static_cast<size_t>(vec) * n;
    const float *zu = z_up + static_cast<size_t>(vec) * n;
    for (uint32_t k = threadIdx.x; k < n; k += blockDim.x) {
        float sg = zg[k], su = zu[k];
        for (uint32_t s = 1; s < splits; ++s) {
            sg += zg[s * split_stride + k];
            su += zu[s * split_stride + k];
        }
        g[k] = sg;
        u[k] = su;
    }
    block_hadamard(g, n, scale);
    block_hadamard(u, n, scale);
    for (uint32_t k = threadIdx.x; k < n; k += blockDim.x) {
        const float gv = g[k] * to_float(sv_gate[mat * stride + k]);
        const float uv = u[k] * to_float(sv_up[mat * stride + k]);
        g[k] = silu(gv) * uv * to_float(su_down[mat * stride + k]);
    }
    block_hadamard(g, n, scale);
    float *dst = x_hat + static_cast<size_t>(vec) * n;
    for (uint32_t k = threadIdx.x; k < n; k += blockDim.x) {
        dst[k] = g[k];
    }
}

// One block per row b: the eight routed outputs in route order, then the
// gated shared expert (src/executor.cpp:1373-1399, 1437-1452).
__global__ __launch_bounds__(256) void k_combine(
    const float *__restrict__ z_down, uint32_t splits, size_t split_stride, uint32_t n,
    const uint16_t *__restrict__ sv_down, const uint32_t *__restrict__ route_expert,
    const float *__restrict__ route_weight, const uint32_t *__restrict__ route_to_grouped,
    const float *__restrict__ z_shared, uint32_t shared_splits, size_t shared_split_stride,
    const int8_t *__restrict__ sv_shared, const float *__restrict__ shared_logit, float scale,
    float *__restrict__ out) {
    extern __shared__ float v[];
    constexpr uint32_t kPerThread = kMaxHadamard / 256;
    float acc[kPerThread];
#pragma unroll
    for (uint32_t i = 0; i < kPerThread; ++i) {
        acc[i] = 0.0f;
    }
    const uint32_t b = blockIdx.x;
    for (uint32_t r = 0; r < 8; ++r) {
        const uint32_t position = route_to_grouped[b * 8u + r];
        const uint32_t expert = route_expert[b * 8u + r];
        const float w = route_weight[b * 8u + r];
        const float *src = z_down + static_cast<size_t>(position) * n;
        for (uint32_t k = threadIdx.x; k < n; k += blockDim.x) {
            float s = src[k];
            for (uint32_t sp = 1; sp < splits; ++sp) {
                s += src[sp * split_stride + k];
            }
            v[k] = s;
        }
        block_hadamard(v, n, scale);
        const uint16_t *sv = sv_down + static_cast<size_t>(expert) * n;
#pragma unroll
        for (uint32_t i = 0; i < kPerThread; ++i) {
            const uint32_t k = threadIdx.x + i * 256u;
            if (k < n) {
                acc[i] += w * (v[k] * half_bits_to_float(sv[k]));
            }
        }
    }
    const float *src = z_shared + static_cast<size_t>(b) * n;
    __syncthreads();
    for (uint32_t k = threadIdx.x; k < n; k += blockDim.x) {
        float s = src[k];
        for (uint32_t sp = 1; sp < shared_splits; ++sp) {
            s += src[sp * shared_split_stride + k];
        }
        v[k] = s;
    }
    block_hadamard(v, n, scale);
    const float gate = sigmoid(shared_logit[b]);
    float *dst = out + static_cast<size_t>(b) * n;
#pragma unroll
    for (uint32_t i = 0; i < kPerThread; ++i) {
        const uint32_t k = threadIdx.x + i * 256u;
        if (k < n) {
            dst[k] = acc[i] + gate * (v[k] * static_cast<float>(sv_shared[k]));
        }
    }
}

void validate_layer(const adi_hip_moe_layer *L) {
    require(L != nullptr, "MoE layer is null");
    require(L->experts >= 8 && L->experts <= kMaxExperts, "MoE expert count must be in 8..1024");
    require(is_power_of_two(L->hidden) && is_power_of_two(L->expert_hidden) &&
                L->hidden >= kTile && L->expert_hidden >= kTile &&
                L->hidden <= kMaxHadamard && L->expert_hidden <= kMaxHadamard,
            "MoE widths must be tiled powers of two up to 8192");
    require(L->router.values != nullptr && L->router.rows == L->experts &&
                L->router.columns == L->hidden,
            "MoE router shape mismatch");
    require(L->shared_expert_gate.values != nullptr && L->shared_expert_gate.rows == 1 &&
                L->shared_expert_gate.columns == L->hidden,
            "MoE shared expert gate shape mismatch");
    const adi_hip_expert_stack *stacks[3] = {&L->gate, &L->up, &L->down};
    for (const auto *s : stacks) {
        require(s->trellis != nullptr && s->su_f16 != nullptr && s->sv_f16 != nullptr &&
                    s->wave_gamma_f16 != nullptr,
                "MoE expert stack tensor is null");
    }
    require(L->expert_codebook != nullptr && L->expert_codebook->kind == adi_hip_codebook::expert,
            "MoE layer needs an expert codebook");
    validate_ne(&L->shared_gate);
    validate_ne(&L->shared_up);
    validate_ne(&L->shared_down);
    require(L->shared_gate.rows == L->expert_hidden && L->shared_gate.columns == L->hidden &&
                L->shared_up.rows == L->expert_hidden && L->shared_up.columns == L->hidden &&
                L->shared_down.rows == L->hidden && L->shared_down.columns == L->expert_hidden,
            "MoE shared expert shape mismatch");
}

}  // namespace
}  // namespace adi_hip

using namespace adi_hip;

extern "C" {

int adi_hip_moe_forward(adi_hip_context *ctx, const adi_hip_moe_layer *L, const float *inputs,
                        uint32_t batch, const float *logit_bias, float *outputs,
                        uint32_t *route_expert_out, float *route_weight_out) {
    return guarded(ctx, [&] {
        validate_layer(L);
        require(batch > 0, "MoE batch shape mismatch");
        require(inputs != nullptr && outputs != nullptr, "MoE vector is null");
        const uint32_t H = L->hidden, I = L->expert_hidden, E = L->experts;
        const size_t B = batch, P = B * 8;
        const uint32_t sg = gemv_splits(H);  // gate/up: H inputs
        const uint32_t sd = gemv_splits(I);  // down: I inputs
        const uint32_t max_active = static_cast<uint32_t>(P < E ? P : E);

        auto &ws = ctx->workspace;
        ws.used = 0;
        const size_t bytes =
            Workspace::round(B * E * 4) + Workspace::round(B * 4) +
            Workspace::round(P * 4) * 5 + Workspace::round(E * 4) * 3 +
            Workspace::round((E + 1) * 4) + Workspace::round(4) +
            Workspace::round(P * H * 4) * 2 + Workspace::round(sg * P * I * 4) * 2 +
            Workspace::round(P * I * 4) + Workspace::round(sd * P * H * 4) +
            Workspace::round(B * H * 4) * 2 + Workspace::round(sg * B * I * 4) * 2 +
            Workspace::round(B * I * 4) + Workspace::round(sd * B * H * 4);
        ws.ensure(bytes);
        float *logits = ws.take<float>(B * E);
        float *shared_logit = ws.take<float>(B);
        uint32_t *route_expert = ws.take<uint32_t>(P);
        float *route_weight = ws.take<float>(P);
        uint32_t *position_expert = ws.take<uint32_t>(P);
        uint32_t *grouped_batch = ws.take<uint32_t>(P);
        uint32_t *route_to_grouped = ws.take<uint32_t>(P);
        uint32_t *counts = ws.take<uint32_t>(E);
        uint32_t *active = ws.take<uint32_t>(E);
        (void)ws.take<uint32_t>(E);
        uint32_t *offsets = ws.take<uint32_t>(E + 1);
        uint32_t *active_count = ws.take<uint32_t>(1);
        float *xh_gate = ws.take<float>(P * H);
        float *xh_up = ws.take<float>(P * H);
        float *z_gate = ws.take<float>(sg * P * I);
        float *z_up = ws.take<float>(sg * P * I);
        float *xh_down = ws.take<float>(P * I);
        float *z_down = ws.take<float>(sd * P * H);
        float *sxh_gate = ws.take<float>(B * H);
        float *sxh_up = ws.take<float>(B * H);
        float *sz_gate = ws.take<float>(sg * B * I);
        float *sz_up = ws.take<float>(sg * B * I);
        float *sxh_down = ws.take<float>(B * I);
        float *sz_down = ws.take<float>(sd * B * H);

        // 1-3: routing
        launch_bf16_ordered(ctx, L->router.values, E, H, inputs, batch, logits, ctx->isa_lanes);
        launch_bf16_ordered(ctx, L->shared_expert_gate.values, 1, H, inputs, batch, shared_logit,
                            ctx->isa_lanes);
        launch_top_experts(ctx, logits, logit_bias, batch, E, route_expert, route_weight);
        RouteSort sort{};
        sort.route_expert = route_expert;
        sort.positions = static_cast<uint32_t>(P);
        sort.experts = E;
        sort.counts = counts;
        sort.offsets = offsets;
        sort.active = active;
        sort.active_count = active_count;
        sort.position_expert = position_expert;
        sort.grouped_batch = grouped_batch;
        sort.route_to_grouped = route_to_grouped;
        launch_route_sort(ctx, sort);

        // 4: prologues
        launch_prologue_f16(ctx, inputs, H, L->gate.su_f16, H, grouped_batch, position_expert,
                            static_cast<uint32_t>(P), xh_gate);
        launch_prologue_f16(ctx, inputs, H, L->up.su_f16, H, grouped_batch, position_expert,
                            static_cast<uint32_t>(P), xh_up);
        launch_prologue_sign(ctx, inputs, H, L->shared_gate.su, batch, sxh_gate);
        launch_prologue_sign(ctx, inputs, H, L->shared_up.su, batch, sxh_up);

        // 5: gate / up
        const size_t gu_words = size_t(I / kTile) * (H / kTile) * kExpertWords;
        const size_t d_words = size_t(H / kTile) * (I / kTile) * kExpertWords;
        const uint32_t gamma_stride = H / kTile + I / kTile;
        ExpertGemv g{};
        g.codebook = L->expert_codebook->data;
        g.active = active;
        g.active_count = active_count;
        g.offsets = offsets;
        g.max_active = max_active;
        g.tokens_per_pass = batch == 1 ? 1 : 4;
        g.gamma_stride = gamma_stride;
        g.rows = I;
        g.columns = H;
        g.trellis_stride = gu_words;
        g.z_split_stride = P * I;
        g.trellis = L->gate.trellis;
        g.gamma = L->gate.wave_gamma_f16;
        g.x_hat = xh_gate;
        g.z = z_gate;
        launch_expert_gemv(ctx, g);
        g.trellis = L->up.trellis;
        g.gamma = L->up.wave_gamma_f16;
        g.x_hat = xh_up;
        g.z = z_up;
        launch_expert_gemv(ctx, g);
        NeGemv n{};
        n.batch = batch;
        n.rows = I;
        n.columns = H;
        n.z_split_stride = B * I;
        n.trellis = L->shared_gate.trellis;
        n.codebook = L->shared_gate.codebook->data;
        n.weight_scale = L->shared_gate.weight_scale;
        n.x_hat = sxh_gate;
        n.z = sz_gate;
        launch_ne_gemv(ctx, n);
        n.trellis = L->shared_up.trellis;
        n.codebook = L->shared_up.codebook->data;
        n.weight_scale = L->shared_up.weight_scale;
        n.x_hat = sxh_up;
        n.z = sz_up;
        launch_ne_gemv(ctx, n);

        // 6: SwiGLU and the down prologue
        const float scale_i = hadamard_scale(I);
        launch(ctx, "swiglu", k_swiglu<uint16_t>, dim3(static_cast<uint32_t>(P)), dim3(256),
               2 * I * sizeof(float), static_cast<const float *>(z_gate),
               static_cast<const float *>(z_up), sg, P * I, I, L->gate.sv_f16, L->up.sv_f16,
               L->down.su_f16, I, static_cast<const uint32_t *>(position_expert), scale_i,
               xh_down);
        launch(ctx, "swiglu", k_swiglu<int8_t>, dim3(batch), dim3(256), 2 * I * sizeof(float),
               static_cast<const float *>(sz_gate), static_cast<const float *>(sz_up), sg, B * I, I,
               L->shared_gate.sv, L->shared_up.sv, L->shared_down.su, 0u,
               static_cast<const uint32_t *>(nullptr), scale_i, sxh_down);

        // 7: down
        g.rows = H;
        g.columns = I;
        g.trellis_stride = d_words;
        g.z_split_stride = P * H;
        g.trellis = L->down.trellis;
        g.gamma = L->down.wave_gamma_f16;
        g.x_hat = xh_down;
        g.z = z_down;
        launch_expert_gemv(ctx, g);
        n.rows = H;
        n.columns = I;
        n.z_split_stride = B * H;
        n.trellis = L->shared_down.trellis;
        n.codebook = L->shared_down.codebook->data;
        n.weight_scale = L->shared_down.weight_scale;
        n.x_hat = sxh_down;
        n.z = sz_down;
        launch_ne_gemv(ctx, n);

        // 8: combine
        launch(ctx, "combine", k_combine, dim3(batch), dim3(256), H * sizeof(float),
               static_cast<const float *>(z_down), sd, P * H, H, L->down.sv_f16,
               static_cast<const uint32_t *>(route_expert),
               static_cast<const float *>(route_weight),
               static_cast<const uint32_t *>(route_to_grouped),
               static_cast<const float *>(sz_down), sd, B * H, L->shared_down.sv,
               static_cast<const float *>(shared_logit), hadamard_scale(H), outputs);

        if (route_expert_out != nullptr) {
            check_hip(hipMemcpyAsync(route_expert_out, route_expert, P * 4,
                                     hipMemcpyDeviceToDevice, ctx->stream),
                      "route copy");
        }
        if (route_weight_out != nullptr) {
            check_hip(hipMemcpyAsync(route_weight_out, route_weight, P * 4,
                                     hipMemcpyDeviceToDevice, ctx->stream),
                      "route copy");
        }
    });
}

}  // extern "C"
