// moe.hip -- one MoE block on the device: moe_forward / moe_forward_batch
// (src/executor.cpp:242-330, 1181-1453).
//
// Launch sequence for a batch of B rows (P = 8B route positions):
//   1 router   router logits and the shared-expert gate logit, ISA-ordered
//              bf16 (bit-exact)
//   2 route    top_experts for every row (+ optional fp32 logit bias) and the
//              stable counting sort: offsets, grouped_batch, route_to_grouped,
//              the ascending list of active experts
//   3 prologue x_hat = H(su_e * x[grouped_batch[p]]) for gate and up of every
//              route position, H(SU * x) for the shared expert (one wave per
//              vector)
//   4 gemv     decode-GEMV gate and up over the active experts and the NE
//              GEMV of the shared gate and up, one launch
//   5 swiglu   g = sv*H(Zg), u = sv*H(Zu), a = silu(g)*u, x_hat = H(su_d * a)
//   6 gemv     down over the active experts and the shared down, one launch
//   7 combine  per row: sum_r w_r * sv_d*H(Zd[p_r]) in route order, then
//              + sigmoid(gate) * SV*H(Zshared)
// Expert work is sized for the worst case (min(P, E) active experts); blocks
// past the device-side active count return at once, so the host never waits
// for the routing.
#include "dense.hpp"
#include "grouped.hpp"
#include "projection.hpp"
#include "route.hpp"

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

struct SwigluSegment {
    const float *z_gate;
    const float *z_up;
    size_t split_stride;
    const uint16_t *sv_gate_f16;  // f16 per matrix (routed) ...
    const uint16_t *sv_up_f16;
    const uint16_t *su_down_f16;
    const int8_t *sv_gate_sign;   // ... or +-1 (shared expert)
    const int8_t *sv_up_sign;
    const int8_t *su_down_sign;
    const uint32_t *matrix_index;
    XhatOut x_hat;
    uint32_t count;
    uint32_t splits;              // slices of z_gate / z_up
};

struct SwigluJobs {
    SwigluSegment seg[2];
    uint32_t segments;
    float scale;
};

// One wave per vector of the intermediate width n = 64*VPL.
template <int VPL>
__global__ __launch_bounds__(256) void k_swiglu_wave(SwigluJobs j) {
    const uint32_t lane = threadIdx.x & 63u;
    uint32_t v = blockIdx.x * 4u + (threadIdx.x >> 6);
    uint32_t s = 0;
    while (s < j.segments && v >= j.seg[s].count) {
        v -= j.seg[s].count;
        ++s;
    }
    if (s >= j.segments) {
        return;
    }
    const SwigluSegment &g = j.seg[s];
    const uint32_t n = 64u * VPL;
    const size_t base = static_cast<size_t>(v) * n;
    // the matrix index, then the slices (up to four at once), then the scales
    // that depend on the index: the slices are in flight during its wait
    const size_t mat = g.matrix_index != nullptr ? g.matrix_index[v] : 0u;
    float gv[VPL], uv[VPL];
    const bool at_once = VPL <= 8 && g.splits >= 1 && g.splits <= 4;
    SliceLoads<VPL <= 8 ? VPL : 1> lg, lu;
    if constexpr (VPL <= 8) {
        if (at_once) {
            load_slices<VPL>(g.z_gate + base, g.split_stride, g.splits, lane, lg);
            load_slices<VPL>(g.z_up + base, g.split_stride, g.splits, lane, lu);
        }
    }
    float sa[VPL], sb[VPL], sc[VPL];
    if (g.sv_gate_f16 != nullptr) {
        load_wave_f16<VPL>(g.sv_gate_f16 + mat * n, lane, sa);
        load_wave_f16<VPL>(g.sv_up_f16 + mat * n, lane, sb);
        load_wave_f16<VPL>(g.su_down_f16 + mat * n, lane, sc);
    } else {
        load_wave_sign<VPL>(g.sv_gate_sign, lane, sa);
        load_wave_sign<VPL>(g.sv_up_sign, lane, sb);
        load_wave_sign<VPL>(g.su_down_sign, lane, sc);
    }
    if constexpr (VPL <= 8) {
        if (at_once) {
            add_slices<VPL>(lg, g.splits, gv);
            add_slices<VPL>(lu, g.splits, uv);
        }
    }
    if (!at_once) {
        sum_slices<VPL>(g.z_gate + base, g.split_stride, g.splits, lane, gv);
        sum_slices<VPL>(g.z_up + base, g.split_stride, g.splits, lane, uv);
    }
    wave_hadamard<VPL>(gv, j.scale, lane);
    wave_hadamard<VPL>(uv, j.scale, lane);
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
        gv[i] = silu(gv[i] * sa[i]) * (uv[i] * sb[i]) * sc[i];
    }
    wave_hadamard<VPL>(gv, j.scale, lane);
    store_xhat<VPL>(g.x_hat, v, lane, gv);
}

struct CombineArgs {
    const float *z_down;
    uint32_t splits;
    size_t split_stride;
    const uint16_t *sv_down;  // f16 per expert, stride n
    const uint32_t *route_expert;
    const float *route_weight;
    const uint32_t *route_to_grouped;
    const float *z_shared;
    uint32_t shared_splits;
    size_t shared_split_stride;
    const int8_t *sv_shared;
    const float *shared_logit;
    float scale;
    float *out;
};

// One block of nine waves per row: wave r < 8 transforms route r's output,
// wave 8 the shared expert's, each into its own LDS row; after one barrier
// every thread adds four columns over the nine rows, in route order and then
// the shared expert (src/executor.cpp:1373-1399, 1437-1452).
template <int VPL>
__global__ __launch_bounds__(576) void k_combine_wave(CombineArgs a) {
    extern __shared__ float parts[];  // [9][64 * VPL]
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t n = 64u * VPL;
    const uint32_t b = blockIdx.x;
    float val[VPL], scale[VPL];
    const float *src;
    uint32_t splits;
    size_t stride;
    float weight;
    // the route's indexes first, then its slices and scales together
    if (wave < 8) {
        const uint32_t grouped = a.route_to_grouped[b * 8u + wave];
        const uint32_t expert = a.route_expert[b * 8u + wave];
        weight = a.route_weight[b * 8u + wave];
        src = a.z_down + static_cast<size_t>(grouped) * n;
        splits = a.splits;
        stride = a.split_stride;
        load_wave_f16<VPL>(a.sv_down + static_cast<size_t>(expert) * n, lane, scale);
    } else {
        weight = sigmoid(a.shared_logit[b]);
        src = a.z_shared + static_cast<size_t>(b) * n;
        splits = a.shared_splits;
        stride = a.shared_split_stride;
        load_wave_sign<VPL>(a.sv_shared, lane, scale);
    }
    sum_slices<VPL>(src, stride, splits, lane, val);
    wave_hadamard<VPL>(val, a.scale, lane);
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
        val[i] = weight * (val[i] * scale[i]);
    }
    store_wave<VPL>(parts + wave * n, lane, val);
    __syncthreads();
    // acc = v0, acc += v1, ..., acc += v7, then + the shared expert's
    const float4 *rows = reinterpret_cast<const float4 *>(parts);
    float4 *row_out = reinterpret_cast<float4 *>(a.out + static_cast<size_t>(b) * n);
    for (uint32_t c = threadIdx.x; c < n / 4u; c += blockDim.x) {
        float4 acc = rows[c];
#pragma unroll
        for (uint32_t r = 1; r < 9; ++r) {
            const float4 v = rows[r * (n / 4u) + c];
            acc.x = acc.x + v.x;
            acc.y = acc.y + v.y;
            acc.z = acc.z + v.z;
            acc.w = acc.w + v.w;
        }
        row_out[c] = acc;
    }
}

template <int VPL>
void launch_combine(adi_hip_context *ctx, const CombineArgs &c, uint32_t batch) {
    const size_t lds = size_t(9) * 64u * VPL * sizeof(float);
    static const bool ready =
        lds <= 65536 || set_lds_limit(reinterpret_cast<const void *>(&k_combine_wave<VPL>), lds);
    (void)ready;
    launch(ctx, "combine", k_combine_wave<VPL>, dim3(batch), dim3(576), lds, c);
}

// Batch 1: routing and the Hadamard prologues in one launch. Block 0 routes
// the row as the routing launch does (top_experts, the counting sort and all
// of its outputs). Every other wave holds one prologue vector. A routed
// vector's expert is the one at its grouped position, and for one row the
// grouped order is the ascending order of the eight chosen experts, so the
// wave recomputes the row's top-8 in registers (the computation of block 0,
// deterministic) and takes the v-th smallest. The input row is loaded before
// the top-8, which hides its load.
template <int SLOTS, int VPL>
__global__ __launch_bounds__(256) void k_route_prologue(const float *__restrict__ logits,
                                                        const float *__restrict__ bias,
                                                        uint32_t *__restrict__ route_expert,
                                                        float *__restrict__ route_weight,
                                                        RouteSort a, PrologueJobs j) {
#pragma clang fp contract(off)
    __shared__ uint32_t counts[kMaxExperts];
    __shared__ uint32_t cursor[kMaxExperts];
    __shared__ uint32_t local_expert[8];
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    if (blockIdx.x == 0) {
        if (wave == 0) {
            top8_wave<SLOTS>(logits, bias, a.experts, lane, route_expert, route_weight, local_expert);
        }
        __syncthreads();
        route_sort_block(a, local_expert, counts, cursor);
        return;
    }
    uint32_t v = (blockIdx.x - 1u) * 4u + wave;
    uint32_t s = 0;
    while (s < j.segments && v >= j.seg[s].count) {
        v -= j.seg[s].count;
        ++s;
    }
    if (s >= j.segments) {
        return;
    }
    const PrologueSegment &g = j.seg[s];
    float val[VPL], su[VPL];
    load_wave<VPL>(g.x, lane, val);  // one row: every vector's source row is 0
    if (g.matrix_index != nullptr) {
        uint32_t chosen[8];
        top8_wave<SLOTS>(logits, bias, a.experts, lane, nullptr, nullptr, nullptr, chosen);
        uint32_t expert = 0;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            uint32_t rank = 0;
#pragma unroll
            for (int m = 0; m < 8; ++m) {
                rank += chosen[m] < chosen[k] ? 1u : 0u;
            }
            expert = rank == v ? chosen[k] : expert;
        }
        load_wave_f16<VPL>(g.su_f16 + static_cast<size_t>(expert) * g.su_stride, lane, su);
    } else if (g.su_f16 != nullptr) {
        load_wave_f16<VPL>(g.su_f16, lane, su);
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

// The fused batch-1 launch for widths of 256..2048 and up to 256 experts;
// false when the shape is outside that range.
template <int SLOTS>
bool launch_route_prologue_slots(adi_hip_context *ctx, const float *logits, const float *bias,
                                 uint32_t *route_expert, float *route_weight, const RouteSort &a,
                                 PrologueJobs &j, dim3 grid) {
    switch (j.n) {
    case 256: launch(ctx, "route_prologue", k_route_prologue<SLOTS, 4>, grid, dim3(256), 0, logits, bias, route_expert, route_weight, a, j); return true;
    case 512: launch(ctx, "route_prologue", k_route_prologue<SLOTS, 8>, grid, dim3(256), 0, logits, bias, route_expert, route_weight, a, j); return true;
    case 1024: launch(ctx, "route_prologue", k_route_prologue<SLOTS, 16>, grid, dim3(256), 0, logits, bias, route_expert, route_weight, a, j); return true;
    case 2048: launch(ctx, "route_prologue", k_route_prologue<SLOTS, 32>, grid, dim3(256), 0, logits, bias, route_expert, route_weight, a, j); return true;
    default: return false;
    }
}

bool launch_route_prologue(adi_hip_context *ctx, const float *logits, const float *bias,
                           uint32_t *route_expert, float *route_weight, const RouteSort &a,
                           PrologueJobs &j) {
    if (j.n < 256 || j.n > 2048 || a.experts > 256 || a.positions != 8) {
        return false;
    }
    uint32_t vectors = 0;
    for (uint32_t s = 0; s < j.segments; ++s) {
        vectors += j.seg[s].count;
    }
    prepare_prologues(j);
    const dim3 grid(1u + ceil_div(vectors, 4u));
    if (a.experts <= 64) {
        return launch_route_prologue_slots<1>(ctx, logits, bias, route_expert, route_weight, a, j, grid);
    }
    if (a.experts <= 128) {
        return launch_route_prologue_slots<2>(ctx, logits, bias, route_expert, route_weight, a, j, grid);
    }
    return launch_route_prologue_slots<4>(ctx, logits, bias, route_expert, route_weight, a, j, grid);
}

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
        require(aligned_to(s->su_f16, 8) && aligned_to(s->sv_f16, 8),
                "MoE expert scale rows must be 8-byte aligned");
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

// The fixed scratch of adi_hip_moe_forward_static: every intermediate of a
// decode batch (batch <= kStaticBatch) of the model's layer geometry fits in
// it (about 6.5 MiB at batch 16, hidden 2048, 256 experts). Each device
// holds its own copy until the process ends; host code uses the address
// static_scratch_address() returns for its device, never this name. Nothing
// in it needs to start at zero: every kernel writes what it later reads.
constexpr size_t kStaticScratchBytes = size_t(12) << 20;
constexpr uint32_t kStaticBatch = 16;
__device__ __align__(256) unsigned char scratch[kStaticScratchBytes];

// One MoE block; `arena` (non-null) is a fixed scratch the call must fit in,
// otherwise the context workspace grows to the call's plan.
void moe_forward_body(adi_hip_context *ctx, const adi_hip_moe_layer *L, const float *inputs,
                      uint32_t batch, const float *logit_bias, float *outputs,
                      uint32_t *route_expert_out, float *route_weight_out, Workspace *arena) {
    {
        validate_layer(L);
        require(batch > 0, "MoE batch shape mismatch");
        require(inputs != nullptr && outputs != nullptr, "MoE vector is null");
        require(aligned_to(inputs, 16) && aligned_to(outputs, 16), "MoE vectors must be 16-byte aligned");
        const uint32_t H = L->hidden, I = L->expert_hidden, E = L->experts;
        const size_t B = batch, P = B * 8;
        const uint32_t max_active = static_cast<uint32_t>(P < E ? P : E);
        const bool wave_path = wave_width(H) && wave_width(I);
        // 2-12 rows of the one-launch block's geometry: the whole block in one
        // persistent launch on the decode-GEMV arithmetic
        const bool few = ctx->fused_moe && wave_path && batch >= 2 && batch <= kFewMaxRows &&
                         H == kFusedHidden && I == kFusedSwigluWidth && E <= kFusedMaxExperts &&
                         L->shared_up.codebook->data == L->shared_gate.codebook->data;
        // prefill microbatches: MFMA grouped GEMMs over the expert-sorted
        // positions; decode batches: the persistent decode-GEMV
        const bool gemv_batch = few || (ctx->gemv_up_to_16 && batch <= 16u);
        const bool mfma = !gemv_batch && wave_path && batch >= kMfmaBatch && expert_mfma_supports(I, H) &&
                          expert_mfma_supports(H, I);
        const uint32_t sg = mfma ? 2u : expert_splits(H);
        const uint32_t sd = mfma ? 2u : expert_splits(I);
        const uint32_t ssg = mfma ? ne_mfma_slices(I, H, batch) : ne_splits(H);
        const uint32_t ssd = mfma ? ne_mfma_slices(H, I, batch) : ne_splits(I);

        auto &ws = arena != nullptr ? *arena : ctx->workspace;
        ws.used = 0;
        const size_t bytes =
            Workspace::round(B * E * 4) + Workspace::round(B * 4) +
            Workspace::round(P * 4) * 5 + Workspace::round(E * 4) * 3 +
            Workspace::round((E + 1) * 4) + Workspace::round(4) + Workspace::round(E * 16) +
            Workspace::round(P * 4) + Workspace::round((route_sort_scratch(P, E) - P) * 4) +
            Workspace::round(P * H * 4) * 2 + Workspace::round(sg * P * I * 4) * 2 +
            Workspace::round(P * I * 4) + Workspace::round(sd * P * H * 4) +
            Workspace::round(B * H * 4) * 2 + Workspace::round(ssg * B * I * 4) * 2 +
            Workspace::round(B * I * 4) + Workspace::round(ssd * B * H * 4) +
            (few ? Workspace::round(B * (E + 1) * 4) + Workspace::round(B * 9 * H * 4) : 0);
        if (arena != nullptr) {
            require(bytes <= arena->capacity,
                    "MoE batch needs more scratch than the fixed no-allocation buffer holds");
        } else {
            ws.ensure(bytes);
        }
        float *logits = ws.take<float>(B * E);
        float *shared_logit = ws.take<float>(B);
        // routes go straight to the caller's buffers when it asks for them
        uint32_t *route_expert_ws = ws.take<uint32_t>(P);
        float *route_weight_ws = ws.take<float>(P);
        uint32_t *route_expert = route_expert_out != nullptr ? route_expert_out : route_expert_ws;
        float *route_weight = route_weight_out != nullptr ? route_weight_out : route_weight_ws;
        uint32_t *position_expert = ws.take<uint32_t>(P);
        uint32_t *grouped_batch = ws.take<uint32_t>(P);
        uint32_t *route_to_grouped = ws.take<uint32_t>(P);
        uint32_t *counts = ws.take<uint32_t>(E);
        uint32_t *active = ws.take<uint32_t>(E);
        (void)ws.take<uint32_t>(E);
        uint32_t *offsets = ws.take<uint32_t>(E + 1);
        uint32_t *active_count = ws.take<uint32_t>(1);
        uint4 *slot_info = ws.take<uint4>(E);
        uint32_t *position_rank = ws.take<uint32_t>(P);
        uint32_t *chunk_hist = ws.take<uint32_t>(route_sort_scratch(P, E) - P);
        // x_hat buffers: fp32 for the GEMV, or f16 hi then lo (same bytes) for MFMA
        float *xh_gate = ws.take<float>(P * H);
        float *xh_up = ws.take<float>(P * H);
        float *z_gate = ws.take<float>(sg * P * I);
        float *z_up = ws.take<float>(sg * P * I);
        float *xh_down = ws.take<float>(P * I);
        float *z_down = ws.take<float>(sd * P * H);
        float *sxh_gate = ws.take<float>(B * H);
        float *sxh_up = ws.take<float>(B * H);
        float *sz_gate = ws.take<float>(ssg * B * I);
        float *sz_up = ws.take<float>(ssg * B * I);
        float *sxh_down = ws.take<float>(B * I);
        float *sz_down = ws.take<float>(ssd * B * H);
        float *few_logits = few ? ws.take<float>(B * (E + 1)) : nullptr;
        float *few_parts = few ? ws.take<float>(B * 9 * H) : nullptr;

        // where x_hat goes: fp32, or f16 pairs (planes 2: expert, 1: NE)
        auto xhat = [&](float *buffer, size_t vectors, size_t n, uint32_t planes) {
            if (!mfma) {
                return XhatOut{buffer, nullptr, nullptr, 0u, static_cast<uint32_t>(vectors)};
            }
            uint16_t *hi = reinterpret_cast<uint16_t *>(buffer);
            return XhatOut{nullptr, hi, hi + vectors * n, planes, static_cast<uint32_t>(vectors)};
        };
        auto hi_of = [&](float *buffer) { return reinterpret_cast<const uint16_t *>(buffer); };
        auto lo_of = [&](float *buffer, size_t count) {
            return reinterpret_cast<const uint16_t *>(buffer) + count;
        };

        const size_t gu_words = size_t(I / kTile) * (H / kTile) * kExpertWords;
        const size_t d_words = size_t(H / kTile) * (I / kTile) * kExpertWords;
        const uint32_t gamma_stride = H / kTile + I / kTile;
        // the decode-GEMV plans of the gate/up and down launches
        auto expert_job = [&](const adi_hip_expert_stack &st, uint32_t rows, uint32_t columns,
                              size_t words, const float *x_hat, float *z) {
            ExpertGemv g{};
            g.gamma_stride = gamma_stride;
            g.rows = rows;
            g.columns = columns;
            g.trellis_stride = words;
            g.z_split_stride = P * rows;
            g.trellis = st.trellis;
            g.gamma = st.wave_gamma_f16;
            g.x_hat = x_hat;
            g.z = z;
            return g;
        };
        auto ne_job = [&](const adi_hip_ne_matrix &m, const float *x_hat, float *z) {
            NeGemv n{};
            n.batch = batch;
            n.rows = m.rows;
            n.columns = m.columns;
            n.z_split_stride = B * m.rows;
            n.trellis = m.trellis;
            n.weight_scale = m.weight_scale;
            n.x_hat = x_hat;
            n.z = z;
            return n;
        };
        auto gate_up_plan = [&]() {
            MoeGemv gu{};
            gu.expert[0] = expert_job(L->gate, I, H, gu_words, xh_gate, z_gate);
            gu.expert[1] = expert_job(L->up, I, H, gu_words, xh_up, z_up);
            gu.expert_count = 2;
            gu.ne[0] = ne_job(L->shared_gate, sxh_gate, sz_gate);
            gu.ne_count = 1;
            gu.expert_book = L->expert_codebook->data;
            gu.slot_info = slot_info;
            gu.ne_book = L->shared_gate.codebook->data;
            gu.max_active = max_active;
            return gu;
        };
        auto down_plan = [&]() {
            MoeGemv dn{};
            dn.expert[0] = expert_job(L->down, H, I, d_words, xh_down, z_down);
            dn.expert_count = 1;
            dn.ne[0] = ne_job(L->shared_down, sxh_down, sz_down);
            dn.ne_count = 1;
            dn.expert_book = L->expert_codebook->data;
            dn.slot_info = slot_info;
            dn.ne_book = L->shared_down.codebook->data;
            dn.max_active = max_active;
            return dn;
        };
        auto swiglu_plan = [&]() {
            return GemvSwiglu{z_gate, z_up, P * I, sg, L->gate.sv_f16, L->up.sv_f16,
                              L->down.su_f16, sz_gate, sz_up, B * I, ssg,
                              L->shared_gate.sv, L->shared_up.sv, L->shared_down.su,
                              hadamard_scale(I)};
        };

        // one row: the whole block in one persistent launch when it fits
        if (batch == 1 && !mfma && wave_path &&
            L->shared_up.codebook->data == L->shared_gate.codebook->data) {
            MoeDecodeOne f{};
            f.gu = gate_up_plan();
            f.gu.ne[1] = ne_job(L->shared_up, sxh_up, sz_up);
            f.gu.ne_count = 2;
            f.dn = down_plan();
            f.dn.swiglu = swiglu_plan();
            f.router = L->router.values;
            f.shared_gate_row = L->shared_expert_gate.values;
            f.logit_bias = logit_bias;
            f.x = inputs;
            f.su_gate = L->gate.su_f16;
            f.su_up = L->up.su_f16;
            f.shared_su_gate = L->shared_gate.su;
            f.shared_su_up = L->shared_up.su;
            f.sv_down = L->down.sv_f16;
            f.shared_sv_down = L->shared_down.sv;
            f.scale_hidden = hadamard_scale(H);
            f.out = outputs;
            f.route_expert_out = route_expert_out;
            f.route_weight_out = route_weight_out;
            f.sync = ctx->moe_sync;
            f.experts = E;
            if (ctx->fused_moe && plan_moe_decode_one(ctx, f)) {
                launch_moe_decode_one(ctx, f);
                ctx->moe_sync_pending = true;
                return;
            }
        }

        // 2-12 rows: the whole block in one persistent launch when it fits
        if (few) {
            MoeDecodeFew f{};
            f.gu = gate_up_plan();
            f.gu.ne[1] = ne_job(L->shared_up, sxh_up, sz_up);
            f.gu.ne_count = 2;
            f.dn = down_plan();
            f.dn.swiglu = swiglu_plan();
            f.router = L->router.values;
            f.shared_gate_row = L->shared_expert_gate.values;
            f.logit_bias = logit_bias;
            f.x = inputs;
            f.su_gate = L->gate.su_f16;
            f.su_up = L->up.su_f16;
            f.shared_su_gate = L->shared_gate.su;
            f.shared_su_up = L->shared_up.su;
            f.sv_down = L->down.sv_f16;
            f.shared_sv_down = L->shared_down.sv;
            f.scale_hidden = hadamard_scale(H);
            f.out = outputs;
            f.route_expert_out = route_expert_out;
            f.route_weight_out = route_weight_out;
            f.logits = few_logits;
            f.parts = few_parts;
            f.sync = ctx->moe_sync + kMoeSyncFew;
            f.error = ctx->moe_sync + kMoeSyncError;
            f.experts = E;
            f.batch = batch;
            if (plan_moe_decode_few(ctx, f)) {
                launch_moe_decode_few(ctx, f);
                ctx->moe_sync_pending = true;
                return;
            }
        }

        // 1-2: router logits (+ the shared gate row) and routing
        launch_bf16_ordered_extra(ctx, L->router.values, E, L->shared_expert_gate.values, H, inputs,
                                  batch, logits, shared_logit, ctx->isa_lanes);
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
        sort.slot_info = slot_info;
        sort.position_rank = position_rank;
        sort.chunk_hist = chunk_hist;

        // 3: prologues, routed gate/up and shared gate/up
        PrologueJobs pro{};
        pro.segments = 4;
        pro.n = H;
        pro.seg[0] = PrologueSegment{inputs, grouped_batch, position_expert, L->gate.su_f16, nullptr,
                                     H, xhat(xh_gate, P, H, 2), static_cast<uint32_t>(P)};
        pro.seg[1] = PrologueSegment{inputs, grouped_batch, position_expert, L->up.su_f16, nullptr,
                                     H, xhat(xh_up, P, H, 2), static_cast<uint32_t>(P)};
        pro.seg[2] = PrologueSegment{inputs, nullptr, nullptr, nullptr, L->shared_gate.su, 0,
                                     xhat(sxh_gate, B, H, 1), batch};
        pro.seg[3] = PrologueSegment{inputs, nullptr, nullptr, nullptr, L->shared_up.su, 0,
                                     xhat(sxh_up, B, H, 1), batch};
        // one row on the decode-GEMV path: routing and prologues in one launch
        if (!(batch == 1 && !mfma && wave_path &&
              launch_route_prologue(ctx, logits, logit_bias, route_expert, route_weight, sort, pro))) {
            launch_route(ctx, logits, logit_bias, batch, route_expert, route_weight, sort);
            launch_prologues(ctx, pro);
        }

        // 4: gate / up projections
        if (mfma) {
            auto expert_mfma = [&](const adi_hip_expert_stack &st, uint32_t rows, uint32_t columns,
                                   size_t words, float *x, float *z) {
                ExpertMfma g{};
                g.trellis = st.trellis;
                g.trellis_stride = words;
                g.gamma = st.wave_gamma_f16;
                g.gamma_stride = gamma_stride;
                g.rows = rows;
                g.columns = columns;
                g.x_hi = hi_of(x);
                g.x_lo = lo_of(x, P * columns);
                g.positions = static_cast<uint32_t>(P);
                g.z = z;
                g.z_split_stride = P * rows;
                return g;
            };
            auto ne_mfma = [&](const adi_hip_ne_matrix &m, float *x, float *z) {
                NeMfma n{};
                n.trellis = m.trellis;
                n.weight_scale = m.weight_scale;
                n.rows = m.rows;
                n.columns = m.columns;
                n.x_hi = hi_of(x);
                n.x_lo = lo_of(x, B * m.columns);
                n.batch = batch;
                n.z = z;
                return n;
            };
            ExpertMfmaJobs gu{};
            gu.expert[0] = expert_mfma(L->gate, I, H, gu_words, xh_gate, z_gate);
            gu.expert[1] = expert_mfma(L->up, I, H, gu_words, xh_up, z_up);
            gu.expert_count = 2;
            gu.expert_book = L->expert_codebook->data;
            gu.slot_info = slot_info;
            gu.max_active = max_active;
            gu.max_positions = batch;
            launch_expert_mfma(ctx, gu);
            NeMfmaJobs sgu{};
            sgu.ne[0] = ne_mfma(L->shared_gate, sxh_gate, sz_gate);
            sgu.ne_count = 1;
            sgu.ne_book = L->shared_gate.codebook->data;
            if (L->shared_up.codebook->data == L->shared_gate.codebook->data) {
                sgu.ne[1] = ne_mfma(L->shared_up, sxh_up, sz_up);
                sgu.ne_count = 2;
                launch_ne_mfma(ctx, sgu);
            } else {
                launch_ne_mfma(ctx, sgu);
                NeMfmaJobs su{};
                su.ne[0] = ne_mfma(L->shared_up, sxh_up, sz_up);
                su.ne_count = 1;
                su.ne_book = L->shared_up.codebook->data;
                launch_ne_mfma(ctx, su);
            }
        } else {
            MoeGemv gu = gate_up_plan();
            if (L->shared_up.codebook->data == L->shared_gate.codebook->data) {
                gu.ne[1] = ne_job(L->shared_up, sxh_up, sz_up);
                gu.ne_count = 2;
                launch_trellis_gemv(ctx, gu);
            } else {
                launch_trellis_gemv(ctx, gu);
                MoeGemv su{};
                su.ne[0] = ne_job(L->shared_up, sxh_up, sz_up);
                su.ne_count = 1;
                su.ne_book = L->shared_up.codebook->data;
                launch_trellis_gemv(ctx, su);
            }
        }

        // the down-projection GEMV (decode path); for one row it builds its
        // x_hat from the gate/up slices itself, so step 5 launches nothing
        MoeGemv dn{};
        if (!mfma) {
            dn = down_plan();
            if (batch == 1 && wave_path && trellis_gemv_can_fuse_swiglu(ctx, dn)) {
                dn.fused_swiglu = 1;
                dn.swiglu = swiglu_plan();
            }
        }

        // 5: SwiGLU and the down prologue
        const float scale_i = hadamard_scale(I);
        if (dn.fused_swiglu != 0) {
            // built inside the down GEMV
        } else if (wave_path) {
            SwigluJobs sj{};
            sj.segments = 2;
            sj.scale = scale_i;
            sj.seg[0] = SwigluSegment{z_gate, z_up, P * I, L->gate.sv_f16, L->up.sv_f16,
                                      L->down.su_f16, nullptr, nullptr, nullptr, position_expert,
                                      xhat(xh_down, P, I, 2), static_cast<uint32_t>(P), sg};
            sj.seg[1] = SwigluSegment{sz_gate, sz_up, B * I, nullptr, nullptr, nullptr,
                                      L->shared_gate.sv, L->shared_up.sv, L->shared_down.su,
                                      nullptr, xhat(sxh_down, B, I, 1), batch, ssg};
            const dim3 grid(ceil_div(P + B, 4));
            switch (I) {
            case 64: launch(ctx, "swiglu", k_swiglu_wave<1>, grid, dim3(256), 0, sj); break;
            case 128: launch(ctx, "swiglu", k_swiglu_wave<2>, grid, dim3(256), 0, sj); break;
            case 256: launch(ctx, "swiglu", k_swiglu_wave<4>, grid, dim3(256), 0, sj); break;
            case 512: launch(ctx, "swiglu", k_swiglu_wave<8>, grid, dim3(256), 0, sj); break;
            case 1024: launch(ctx, "swiglu", k_swiglu_wave<16>, grid, dim3(256), 0, sj); break;
            case 2048: launch(ctx, "swiglu", k_swiglu_wave<32>, grid, dim3(256), 0, sj); break;
            default: launch(ctx, "swiglu", k_swiglu_wave<64>, grid, dim3(256), 0, sj); break;
            }
        } else {
            launch(ctx, "swiglu", k_swiglu<uint16_t>, dim3(static_cast<uint32_t>(P)), dim3(256),
                   2 * I * sizeof(float), static_cast<const float *>(z_gate),
                   static_cast<const float *>(z_up), sg, P * I, I, L->gate.sv_f16, L->up.sv_f16,
                   L->down.su_f16, I, static_cast<const uint32_t *>(position_expert), scale_i,
                   xh_down);
            launch(ctx, "swiglu", k_swiglu<int8_t>, dim3(batch), dim3(256), 2 * I * sizeof(float),
                   static_cast<const float *>(sz_gate), static_cast<const float *>(sz_up), ssg, B * I,
                   I, L->shared_gate.sv, L->shared_up.sv, L->shared_down.su, 0u,
                   static_cast<const uint32_t *>(nullptr), scale_i, sxh_down);
        }

        // 6: down projections
        if (mfma) {
            ExpertMfmaJobs dn{};
            ExpertMfma &g = dn.expert[0];
            g.trellis = L->down.trellis;
            g.trellis_stride = d_words;
            g.gamma = L->down.wave_gamma_f16;
            g.gamma_stride = gamma_stride;
            g.rows = H;
            g.columns = I;
            g.x_hi = hi_of(xh_down);
            g.x_lo = lo_of(xh_down, P * I);
            g.positions = static_cast<uint32_t>(P);
            g.z = z_down;
            g.z_split_stride = P * H;
            dn.expert_count = 1;
            dn.expert_book = L->expert_codebook->data;
            dn.slot_info = slot_info;
            dn.max_active = max_active;
            dn.max_positions = batch;
            launch_expert_mfma(ctx, dn);
            NeMfmaJobs sdn{};
            NeMfma &n = sdn.ne[0];
            n.trellis = L->shared_down.trellis;
            n.weight_scale = L->shared_down.weight_scale;
            n.rows = H;
            n.columns = I;
            n.x_hi = hi_of(sxh_down);
            n.x_lo = lo_of(sxh_down, B * I);
            n.batch = batch;
            n.z = sz_down;
            sdn.ne_count = 1;
            sdn.ne_book = L->shared_down.codebook->data;
            launch_ne_mfma(ctx, sdn);
        } else {
            launch_trellis_gemv(ctx, dn);
        }

        // 7: combine
        if (wave_path) {
            CombineArgs c{z_down, sd, P * H, L->down.sv_f16, route_expert, route_weight,
                          route_to_grouped, sz_down, ssd, B * H, L->shared_down.sv, shared_logit,
                          hadamard_scale(H), outputs};
            switch (H) {
            case 64: launch_combine<1>(ctx, c, batch); break;
            case 128: launch_combine<2>(ctx, c, batch); break;
            case 256: launch_combine<4>(ctx, c, batch); break;
            case 512: launch_combine<8>(ctx, c, batch); break;
            case 1024: launch_combine<16>(ctx, c, batch); break;
            case 2048: launch_combine<32>(ctx, c, batch); break;
            default: launch_combine<64>(ctx, c, batch); break;
            }
        } else {
            launch(ctx, "combine", k_combine, dim3(batch), dim3(256), H * sizeof(float),
                   static_cast<const float *>(z_down), sd, P * H, H, L->down.sv_f16,
                   static_cast<const uint32_t *>(route_expert),
                   static_cast<const float *>(route_weight),
                   static_cast<const uint32_t *>(route_to_grouped),
                   static_cast<const float *>(sz_down), ssd, B * H, L->shared_down.sv,
                   static_cast<const float *>(shared_logit), hadamard_scale(H), outputs);
        }
    }
}

}  // namespace

hipError_t static_scratch_address(void **out) {
    return hipGetSymbolAddress(out, HIP_SYMBOL(scratch));
}

}  // namespace adi_hip

using namespace adi_hip;

extern "C" {

int adi_hip_moe_forward(adi_hip_context *ctx, const adi_hip_moe_layer *L, const float *inputs,
                        uint32_t batch, const float *logit_bias, float *outputs,
                        uint32_t *route_expert_out, float *route_weight_out) {
    return guarded(ctx, [&] {
        moe_forward_body(ctx, L, inputs, batch, logit_bias, outputs, route_expert_out,
                         route_weight_out, nullptr);
    });
}

int adi_hip_moe_forward_static(adi_hip_context *ctx, const adi_hip_moe_layer *L,
                               const float *inputs, uint32_t batch, const float *logit_bias,
                               float *outputs, uint32_t *route_expert_out,
                               float *route_weight_out) {
    return guarded(ctx, [&] {
        require(batch > 0 && batch <= kStaticBatch,
                "MoE batch for the no-allocation entry must be 1..16");
        require(ctx->static_scratch != nullptr, "no-allocation scratch address missing");
        Workspace arena;
        arena.base = ctx->static_scratch;
        arena.capacity = kStaticScratchBytes;
        moe_forward_body(ctx, L, inputs, batch, logit_bias, outputs, route_expert_out,
                         route_weight_out, &arena);
    });
}

}  // extern "C"
