// context.hip -- context lifetime, codebook upload and kernel profiling.
#include "context.hpp"

#include <mutex>

namespace adi_hip {
namespace {

std::mutex g_create_error_mutex;
std::string g_create_error;

// f32 -> f16 bits, round to nearest even with subnormals, the rounding of the
// reference's f32_to_f16 (src/kernels.cpp:336-379).
uint16_t f16_bits(float value) {
    uint32_t bits;
    std::memcpy(&bits, &value, 4);
    const uint16_t sign = static_cast<uint16_t>((bits >> 16) & 0x8000u);
    const uint32_t biased = (bits >> 23) & 0xFFu;
    const uint32_t mantissa = bits & 0x7FFFFFu;
    if (biased == 0xFFu) {
        return static_cast<uint16_t>(sign | 0x7C00u | (mantissa ? ((mantissa >> 13) | 1u) : 0u));
    }
    const int exponent = static_cast<int>(biased) - 112;
    if (exponent >= 31) {
        return static_cast<uint16_t>(sign | 0x7C00u);
    }
    if (exponent <= 0) {
        if (exponent < -10) {
            return sign;
        }
        const uint32_t full = mantissa | 0x800000u;
        const uint32_t shift = static_cast<uint32_t>(14 - exponent);
        uint32_t q = full >> shift;
        const uint32_t rest = full & ((1u << shift) - 1u);
        const uint32_t half = 1u << (shift - 1u);
        if (rest > half || (rest == half && (q & 1u))) {
            ++q;
        }
        return static_cast<uint16_t>(sign | q);
    }
    uint32_t result = (static_cast<uint32_t>(exponent) << 10) | (mantissa >> 13);
    const uint32_t rest = mantissa & 0x1FFFu;
    if (rest > 0x1000u || (rest == 0x1000u && (result & 1u))) {
        ++result;
    }
    return static_cast<uint16_t>(sign | result);
}

bool all_finite(const float *values, size_t count) {
    for (size_t i = 0; i < count; ++i) {
        if (!std::isfinite(values[i])) {
            return false;
        }
    }
    return true;
}

adi_hip_codebook *upload(adi_hip_context *ctx, adi_hip_codebook::Kind kind,
                         const std::vector<uint16_t> &table) {
    auto *book = new adi_hip_codebook{kind, ctx->device, nullptr, table.size() * 2};
    hipError_t error = hipMalloc(&book->data, book->bytes);
    if (error == hipSuccess) {
        error = hipMemcpy(book->data, table.data(), book->bytes, hipMemcpyHostToDevice);
    }
    if (error != hipSuccess) {
        if (book->data != nullptr) {
            (void)hipFree(book->data);
        }
        delete book;
        check_hip(error, "codebook upload");
    }
    return book;
}

}  // namespace

KernelStat &stat_for(adi_hip_context *ctx, const char *name) {
    for (auto &stat : ctx->stats) {
        if (stat.name == name) {
            return stat;
        }
    }
    ctx->stats.push_back(KernelStat{name});
    return ctx->stats.back();
}

}  // namespace adi_hip

using namespace adi_hip;

extern "C" {

int adi_hip_context_create(int device, adi_hip_context **out) {
    auto record = [](const std::string &message) {
        std::lock_guard<std::mutex> lock(g_create_error_mutex);
        g_create_error = message;
    };
    if (out == nullptr) {
        record("adi_hip_context_create: null output pointer");
        return ADI_HIP_INVALID_ARGUMENT;
    }
    *out = nullptr;
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || device < 0 || device >= count) {
        record("adi_hip_context_create: no such HIP device");
        return ADI_HIP_INVALID_ARGUMENT;
    }
    hipDeviceProp_t props;
    if (hipGetDeviceProperties(&props, device) != hipSuccess) {
        record("adi_hip_context_create: hipGetDeviceProperties failed");
        return ADI_HIP_DEVICE_ERROR;
    }
    if (std::string(props.gcnArchName).rfind("gfx950", 0) != 0) {
        record(std::string("adi_hip_context_create: built for gfx950, device is ") +
               props.gcnArchName);
        return ADI_HIP_INVALID_ARGUMENT;
    }
    auto *ctx = new (std::nothrow) adi_hip_context;
    if (ctx == nullptr) {
        record("adi_hip_context_create: host allocation failed");
        return ADI_HIP_OUT_OF_MEMORY;
    }
    ctx->device = device;
    ctx->cu_count = props.multiProcessorCount;
    // each device holds its own copy of the static scratch array: take this
    // device's address with the device current
    int previous = 0;
    hipError_t status = hipGetDevice(&previous);
    if (status == hipSuccess) {
        status = hipSetDevice(device);
    }
    if (status == hipSuccess) {
        status = adi_hip::static_scratch_address(&ctx->static_scratch);
        (void)hipSetDevice(previous);
    }
    if (status != hipSuccess || ctx->static_scratch == nullptr) {
        record(std::string("adi_hip_context_create: hipGetSymbolAddress failed: ") +
               hipGetErrorString(status));
        delete ctx;
        return ADI_HIP_DEVICE_ERROR;
    }
    // the one-launch MoE block's counters, zero before the first call
    status = hipSetDevice(device);
    if (status == hipSuccess) {
        status = hipMalloc(reinterpret_cast<void **>(&ctx->moe_sync),
                           adi_hip::kMoeSyncWords * sizeof(uint32_t));
    }
    if (status == hipSuccess) {
        status = hipMemset(ctx->moe_sync, 0, adi_hip::kMoeSyncWords * sizeof(uint32_t));
    }
    if (status == hipSuccess) {
        status = hipDeviceSynchronize();
    }
    (void)hipSetDevice(previous);
    if (status != hipSuccess) {
        record(std::string("adi_hip_context_create: MoE counters: ") + hipGetErrorString(status));
        if (ctx->moe_sync != nullptr) {
            (void)hipFree(ctx->moe_sync);
        }
        delete ctx;
        return ADI_HIP_DEVICE_ERROR;
    }
    *out = ctx;
    return ADI_HIP_OK;
}

void adi_hip_context_destroy(adi_hip_context *ctx) {
    if (ctx == nullptr) {
        return;
    }
    int previous = 0;
    (void)hipGetDevice(&previous);
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    for (auto &stat : ctx->stats) {
        for (auto &pair : stat.pending) {
            (void)hipEventDestroy(pair.first);
            (void)hipEventDestroy(pair.second);
        }
    }
    if (ctx->moe_sync != nullptr) {
        (void)hipFree(ctx->moe_sync);
    }
    for (adi_hip::Workspace *w : {&ctx->sequence_workspace, &ctx->layer_output, &ctx->decoder_workspace,
                                  &ctx->rope_cache}) {
        if (w->base != nullptr) {
            (void)hipFree(w->base);
        }
    }
    if (ctx->layer_workspace.base != nullptr) {
        (void)hipFree(ctx->layer_workspace.base);
    }
    if (ctx->workspace.base != nullptr) {
        (void)hipFree(ctx->workspace.base);
    }
    (void)hipSetDevice(previous);
    delete ctx;
}

const char *adi_hip_last_error(const adi_hip_context *ctx) {
    if (ctx == nullptr) {
        std::lock_guard<std::mutex> lock(g_create_error_mutex);
        return g_create_error.c_str();
    }
    return const_cast<adi_hip_context *>(ctx)->last_error_cstr();
}

int adi_hip_set_stream(adi_hip_context *ctx, void *stream) {
    return guarded(ctx, [&] { ctx->stream = static_cast<hipStream_t>(stream); });
}

int adi_hip_synchronize(adi_hip_context *ctx) {
    return guarded(ctx, [&] {
        check_hip(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
        if (ctx->moe_sync_pending) {
            // a wait of the one-launch MoE block that ran out leaves its bit
            // here (its outputs are then wrong): report it, reset the words
            ctx->moe_sync_pending = false;
            uint32_t error = 0;
            check_hip(hipMemcpy(&error, ctx->moe_sync + adi_hip::kMoeSyncError, sizeof(error),
                                hipMemcpyDeviceToHost),
                      "MoE counters read");
            if (error != 0) {
                check_hip(hipMemset(ctx->moe_sync, 0, adi_hip::kMoeSyncWords * sizeof(uint32_t)),
                          "MoE counters reset");
                check_hip(hipDeviceSynchronize(), "MoE counters reset");
                fail(ADI_HIP_DEVICE_ERROR,
                     "one-launch MoE block: a cross-block wait ran out (error bits " +
                         std::to_string(error) + "); its outputs are invalid");
            }
        }
    });
}

int adi_hip_set_fused_decode(adi_hip_context *ctx, int enabled) {
    return guarded(ctx, [&] {
        ctx->fused_moe = enabled != 0 && enabled != 2;
        ctx->gemv_up_to_16 = enabled == 2;
    });
}

int adi_hip_set_workspace_limit(adi_hip_context *ctx, size_t bytes) {
    return guarded(ctx, [&] {
        for (adi_hip::Workspace *w : {&ctx->workspace, &ctx->layer_workspace, &ctx->decoder_workspace,
                                      &ctx->sequence_workspace, &ctx->layer_output, &ctx->rope_cache}) {
            w->limit = bytes;
        }
    });
}

int adi_hip_device_alloc(adi_hip_context *ctx, size_t bytes, void **out) {
    return guarded(ctx, [&] {
        require(out != nullptr, "device_alloc: null output");
        *out = nullptr;
        check_hip(hipMalloc(out, bytes == 0 ? 1 : bytes), "hipMalloc");
    });
}

void adi_hip_device_free(adi_hip_context *ctx, void *pointer) {
    if (ctx == nullptr || pointer == nullptr) {
        return;
    }
    int previous = 0;
    if (hipGetDevice(&previous) == hipSuccess) {
        (void)hipSetDevice(ctx->device);
        (void)hipFree(pointer);
        (void)hipSetDevice(previous);
    }
}

int adi_hip_copy_to_device(adi_hip_context *ctx, void *device, const void *host, size_t bytes) {
    return guarded(ctx, [&] {
        require(bytes == 0 || (device != nullptr && host != nullptr), "copy_to_device: null pointer");
        if (bytes == 0) {
            return;
        }
        check_hip(hipMemcpyAsync(device, host, bytes, hipMemcpyHostToDevice, ctx->stream),
                  "hipMemcpyAsync");
        check_hip(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
    });
}

int adi_hip_copy_to_host(adi_hip_context *ctx, void *host, const void *device, size_t bytes) {
    return guarded(ctx, [&] {
        require(bytes == 0 || (device != nullptr && host != nullptr), "copy_to_host: null pointer");
        if (bytes == 0) {
            return;
        }
        check_hip(hipMemcpyAsync(host, device, bytes, hipMemcpyDeviceToHost, ctx->stream),
                  "hipMemcpyAsync");
        check_hip(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
    });
}

int adi_hip_set_reduction_isa(adi_hip_context *ctx, uint32_t lanes) {
    return guarded(ctx, [&] {
        require(lanes == 1 || lanes == 8 || lanes == 16,
                "reduction ISA must be 1 (scalar), 8 (AVX2) or 16 (AVX-512) lanes");
        ctx->isa_lanes = lanes;
    });
}

int adi_hip_codebook_create_expert(adi_hip_context *ctx, const float *tlut,
                                   adi_hip_codebook **out) {
    return guarded(ctx, [&] {
        require(tlut != nullptr && out != nullptr, "expert codebook: null pointer");
        require(all_finite(tlut, 32768 * 8), "expert TLUT holds a non-finite value");
        // Row r of the reachable table is TLUT row 2r, every value rounded
        // through f16 (src/codec_cache.cpp:33-58); the per-state sign of
        // component 0 is applied in the kernels. Stored as two planes of
        // 16384 x 4 f16 (components 0-3, then 4-7) so that one plane, 128 KiB,
        // fits in a CU's LDS.
        std::vector<uint16_t> table(size_t(kExpertRows) * 8);
        for (uint32_t r = 0; r < kExpertRows; ++r) {
            for (uint32_t c = 0; c < 8; ++c) {
                table[size_t(c / 4) * kExpertRows * 4 + size_t(r) * 4 + c % 4] =
                    f16_bits(tlut[size_t(2 * r) * 8 + c]);
            }
        }
        *out = upload(ctx, adi_hip_codebook::expert, table);
    });
}

int adi_hip_codebook_create_ne(adi_hip_context *ctx, const float *tlut,
                               adi_hip_codebook **out) {
    return guarded(ctx, [&] {
        require(tlut != nullptr && out != nullptr, "NE codebook: null pointer");
        require(all_finite(tlut, 512 * 2), "NE TLUT holds a non-finite value");
        // Signed table (src/codec_cache.cpp:85-115): entry row | neg << 9.
        std::vector<uint16_t> table(1024 * 2);
        for (uint32_t index = 0; index < 1024; ++index) {
            const uint32_t row = index & 0x1FFu;
            const uint16_t v0 = f16_bits(tlut[row * 2]);
            const uint16_t v1 = f16_bits(tlut[row * 2 + 1]);
            table[index * 2] = static_cast<uint16_t>((index >> 9) ? (v0 ^ 0x8000u) : v0);
            table[index * 2 + 1] = v1;
        }
        *out = upload(ctx, adi_hip_codebook::ne, table);
    });
}

void adi_hip_codebook_destroy(adi_hip_codebook *codebook) {
    if (codebook == nullptr) {
        return;
    }
    int previous = 0;
    (void)hipGetDevice(&previous);
    (void)hipSetDevice(codebook->device);
    (void)hipDeviceSynchronize();
    (void)hipFree(codebook->data);
    (void)hipSetDevice(previous);
    delete codebook;
}

int adi_hip_profiling_enable(adi_hip_context *ctx, int enabled) {
    return guarded(ctx, [&] {
        check_hip(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
        for (auto &stat : ctx->stats) {
            for (auto &pair : stat.pending) {
                (void)hipEventDestroy(pair.first);
                (void)hipEventDestroy(pair.second);
            }
        }
        ctx->stats.clear();
        ctx->profiling = enabled != 0;
    });
}

int adi_hip_profiling_read(adi_hip_context *ctx, adi_hip_kernel_profile *out,
                           uint32_t capacity, uint32_t *count) {
    return guarded(ctx, [&] {
        check_hip(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
        for (auto &stat : ctx->stats) {
            for (auto &pair : stat.pending) {
                float ms = 0.0f;
                check_hip(hipEventElapsedTime(&ms, pair.first, pair.second), "hipEventElapsedTime");
                stat.total_ms += ms;
                stat.launches += 1;
                (void)hipEventDestroy(pair.first);
                (void)hipEventDestroy(pair.second);
            }
            stat.pending.clear();
        }
        if (count != nullptr) {
            *count = static_cast<uint32_t>(ctx->stats.size());
        }
        for (uint32_t i = 0; i < capacity && i < ctx->stats.size() && out != nullptr; ++i) {
            std::memset(&out[i], 0, sizeof(out[i]));
            std::strncpy(out[i].name, ctx->stats[i].name.c_str(), sizeof(out[i].name) - 1);
            out[i].launches = ctx->stats[i].launches;
            out[i].total_ms = ctx->stats[i].total_ms;
        }
    });
}

}  // extern "C"
