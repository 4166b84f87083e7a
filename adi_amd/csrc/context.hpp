// context.hpp -- the context object behind adi_hip_context and the launch,
// workspace and error plumbing every entry point shares.
#pragma once

#include "common.hpp"

#include <cmath>
#include <exception>
#include <mutex>
#include <new>
#include <string>
#include <thread>
#include <unordered_map>
#include <utility>
#include <vector>

struct adi_hip_codebook {
    enum Kind { expert, ne } kind;
    int device;
    void *data;    // expert: u16[2][16384][4] (component planes); ne: u16[1024][2]
    size_t bytes;
};

namespace adi_hip {

struct KernelStat {
    std::string name;
    uint64_t launches = 0;
    double total_ms = 0.0;
    std::vector<std::pair<hipEvent_t, hipEvent_t>> pending;
};

// Grow-only device arena; reserve() hands out 256-byte aligned slices of one
// allocation, reset per call. `limit` caps its size (adi_hip_set_workspace_limit):
// growth beyond it fails before anything is freed or launched.
struct Workspace {
    void *base = nullptr;
    size_t capacity = 0;
    size_t used = 0;
    size_t limit = SIZE_MAX;
    // set while a stream capture records launches into these slices: growing
    // then would free memory the graph is recording pointers into
    bool frozen = false;

    void ensure(size_t bytes) {
        if (bytes <= capacity) {
            return;
        }
        if (frozen) {
            fail(ADI_HIP_DEVICE_ERROR,
                 "a captured decode step needs more workspace than its planning pass reserved");
        }
        if (bytes > limit) {
            fail(ADI_HIP_OUT_OF_MEMORY, "workspace of " + std::to_string(bytes) +
                                            " bytes exceeds the context's workspace limit of " +
                                            std::to_string(limit) + " bytes");
        }
        if (base != nullptr) {
            check_hip(hipDeviceSynchronize(), "workspace synchronize");
            check_hip(hipFree(base), "workspace free");
            base = nullptr;
            capacity = 0;
        }
        check_hip(hipMalloc(&base, bytes), "workspace allocation");
        capacity = bytes;
    }

    template <typename T>
    T *take(size_t count) {
        const size_t bytes = (count * sizeof(T) + 255) & ~size_t(255);
        if (used + bytes > capacity) {
            fail(ADI_HIP_OUT_OF_MEMORY, "workspace plan exceeded its reservation");
        }
        T *p = reinterpret_cast<T *>(static_cast<char *>(base) + used);
        used += bytes;
        return p;
    }

    static size_t round(size_t bytes) { return (bytes + 255) & ~size_t(255); }
};

}  // namespace adi_hip

struct adi_hip_context {
    int device = 0;
    hipStream_t stream = nullptr;
    uint32_t isa_lanes = 16;
    int cu_count = 256;
    // Message of the last failed call, kept per calling thread: a batcher's
    // submit, cancel and status calls may run on other threads while one
    // thread steps it, and each thread reads back only its own calls'
    // messages. Map nodes are stable, so a returned c_str() stays valid until
    // that thread's next call on the context.
    std::mutex error_mutex;
    std::unordered_map<std::thread::id, std::string> errors;

    void set_error(std::string message) {
        std::lock_guard<std::mutex> lock(error_mutex);
        errors[std::this_thread::get_id()] = std::move(message);
    }
    std::string last_error() {
        std::lock_guard<std::mutex> lock(error_mutex);
        auto it = errors.find(std::this_thread::get_id());
        return it == errors.end() ? std::string() : it->second;
    }
    const char *last_error_cstr() {
        std::lock_guard<std::mutex> lock(error_mutex);
        return errors[std::this_thread::get_id()].c_str();
    }
    adi_hip::Workspace workspace;
    // scratch of the layer-level entries (attention), kept apart from
    // `workspace`, which every projection entry they call resets
    adi_hip::Workspace layer_workspace;
    // scratch of the decoder-layer entry, which calls the attention entries
    adi_hip::Workspace decoder_workspace;
    // scratch of the model-level entries (decode steps, prefill), which call
    // the decoder layers
    adi_hip::Workspace sequence_workspace;
    // the MoE rows of the public decoder-layer entries, added at their end
    adi_hip::Workspace layer_output;
    // RoPE cos/sin of positions 0 .. rope_positions - 1 ([position][cos 32,
    // sin 32] floats), computed on the host and grown on demand
    adi_hip::Workspace rope_cache;
    uint32_t rope_positions = 0;
    // device address of moe.hip's fixed scratch array on this context's
    // device (adi_hip_moe_forward_static), taken once at creation
    void *static_scratch = nullptr;
    // counters and hand-over words of the one-launch batch-1 MoE block
    // (kMoeSyncWords, zero between calls but for the error word), whether a
    // launch since the last synchronize may have set that word, and whether
    // the one-launch path is enabled
    uint32_t *moe_sync = nullptr;
    bool moe_sync_pending = false;
    bool fused_moe = true;
    // with fused_moe off: batches of up to 16 rows still take the decode-GEMV
    // launches (the few-row one-launch block's arithmetic) instead of the MFMA
    bool gemv_up_to_16 = false;
    bool profiling = false;
    // planning pass of a graph capture: every host step of a call runs
    // (checks, workspace and RoPE table growth) but nothing is launched
    bool dry_run = false;

    // every grow-on-demand arena, for the capture's freeze and its check
    // that none was reallocated since
    std::vector<adi_hip::Workspace *> arenas() {
        return {&workspace, &layer_workspace, &decoder_workspace, &sequence_workspace,
                &layer_output, &rope_cache};
    }
    std::vector<adi_hip::KernelStat> stats;
};

namespace adi_hip {

// adi_hip_context::moe_sync: 99 lines of kMoeSyncLine words. Lines 0-45
// hold the one-row MoE block's counters and flags, its logits, the NE
// projection's ticket (43) and the error word (45); lines 46-63 the one-row
// block's nine combine rows (data it leaves behind); lines 64-95 the few-row
// block's counters; lines 96-97 the Gated DeltaNet core's tickets; line 98
// the full-attention decode launch's tickets.
constexpr uint32_t kMoeSyncLine = 1024;
constexpr uint32_t kMoeSyncWords = 99 * kMoeSyncLine;
constexpr uint32_t kMoeSyncError = 45 * kMoeSyncLine;
constexpr uint32_t kMoeSyncNeTicket = 43 * kMoeSyncLine;  // the one-launch NE projection's ticket
constexpr uint32_t kMoeSyncFew = 64 * kMoeSyncLine;       // the few-row MoE block's counters
constexpr uint32_t kMoeSyncLinear = 96 * kMoeSyncLine;    // the Gated DeltaNet core's tickets
constexpr uint32_t kMoeSyncAttention = 98 * kMoeSyncLine; // the full-attention decode launch's tickets

// Selects the context's device for the duration of a call.
class DeviceScope {
  public:
    explicit DeviceScope(int device) {
        check_hip(hipGetDevice(&previous_), "hipGetDevice");
        if (previous_ != device) {
            check_hip(hipSetDevice(device), "hipSetDevice");
        }
        device_ = device;
    }
    ~DeviceScope() {
        if (previous_ != device_) {
            (void)hipSetDevice(previous_);
        }
    }
    DeviceScope(const DeviceScope &) = delete;
    DeviceScope &operator=(const DeviceScope &) = delete;

  private:
    int previous_ = 0;
    int device_ = 0;
};

template <typename F>
int guarded(adi_hip_context *ctx, F &&function) {
    if (ctx == nullptr) {
        return ADI_HIP_INVALID_ARGUMENT;
    }
    try {
        DeviceScope scope(ctx->device);
        function();
        ctx->set_error(std::string());
        return ADI_HIP_OK;
    } catch (const Failure &failure) {
        ctx->set_error(failure.message);
        return failure.status;
    } catch (const std::bad_alloc &) {
        ctx->set_error("host allocation failed");
        return ADI_HIP_OUT_OF_MEMORY;
    } catch (const std::exception &error) {
        ctx->set_error(error.what());
        return ADI_HIP_DEVICE_ERROR;
    }
}

KernelStat &stat_for(adi_hip_context *ctx, const char *name);

// Launches `kernel` on the context stream. With profiling on, the launch
// carries a start and a stop event that the runtime stamps from the kernel's
// own dispatch (hipExtLaunchKernel), so the time is the kernel's execution,
// as a kernel trace reports it, not the gap between two event packets.
template <typename Kernel, typename... Args>
void launch(adi_hip_context *ctx, const char *name, Kernel kernel, dim3 grid,
            dim3 block, size_t lds_bytes, Args... args) {
    if (grid.x == 0 || grid.y == 0 || grid.z == 0 || ctx->dry_run) {
        return;
    }
    if (!ctx->profiling) {
        hipLaunchKernelGGL(kernel, grid, block, lds_bytes, ctx->stream, args...);
        check_hip(hipGetLastError(), name);
        return;
    }
    hipEvent_t start = nullptr, stop = nullptr;
    check_hip(hipEventCreate(&start), "hipEventCreate");
    check_hip(hipEventCreate(&stop), "hipEventCreate");
    hipExtLaunchKernelGGL(kernel, grid, block, static_cast<uint32_t>(lds_bytes), ctx->stream,
                          start, stop, 0, args...);
    check_hip(hipGetLastError(), name);
    stat_for(ctx, name).pending.emplace_back(start, stop);
}

// Raises a kernel's dynamic LDS limit above the 64 KiB default (once per
// kernel; the result is cached by the caller in a function-local static).
inline bool set_lds_limit(const void *kernel, size_t bytes) {
    check_hip(hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                  static_cast<int>(bytes)),
              "hipFuncSetAttribute");
    return true;
}

// The device address of the no-allocation MoE entry's fixed scratch array
// on the current device (defined beside the array in moe.hip).
hipError_t static_scratch_address(void **out);

inline uint32_t ceil_div(uint64_t a, uint64_t b) {
    return static_cast<uint32_t>((a + b - 1) / b);
}

}  // namespace adi_hip
