// batcher.hip -- continuous batching over the model-level entry points
// (ContinuousBatcher::Impl, src/generation.cpp:343-660), token ids in and
// out. The worker loop's iteration is adi_hip_batcher_step; the caller owns
// the thread that drives it.
#include "context.hpp"

#include <atomic>
#include <chrono>
#include <cmath>
#include <deque>
#include <mutex>
#include <random>
#include <unordered_map>
#include <unordered_set>
#include <vector>

namespace adi_hip {
namespace {

constexpr uint32_t kMaxSlots = 256;
constexpr uint32_t kWordGroup = 32;
constexpr uint32_t kNoToken = 0xFFFFFFFFu;  // the samplers' answer for a non-finite row

using Clock = std::chrono::steady_clock;

struct Words {
    uint64_t word[kWordGroup];
};

// The rows' draws reach the device as kernel arguments, in stream order
// with the sampler that reads them.
__global__ __launch_bounds__(64) void k_store_words(uint64_t *dst, Words words, uint32_t count) {
    const uint32_t i = threadIdx.x;
    if (i < count) {
        dst[i] = words.word[i];
    }
}

// Tokenizer::mask_unused_logits (src/tokenizer.cpp:227-234) on rows
// [first, first + rows) of logits[.][vocabulary].
__global__ __launch_bounds__(256) void k_mask_logits(float *logits, uint32_t vocabulary,
                                                     const uint32_t *masked, uint32_t count) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < count) {
        logits[static_cast<size_t>(blockIdx.y) * vocabulary + masked[i]] = -3.40282347e+38f;
    }
}

struct Request {
    std::vector<uint32_t> prompt;
    adi_hip_generation_options options{};
    uint32_t state = ADI_HIP_REQUEST_PENDING;
    uint32_t max_output = 0;
    std::vector<uint32_t> output;
    std::string error;
    bool cancelled = false;
    double prefill_seconds = 0.0;
    double decode_seconds = 0.0;
};

struct Active {
    uint64_t id;
    uint32_t slot;
    uint32_t max_output;
    float temperature;
    float top_p;
    std::mt19937_64 random;
    Clock::time_point decode_started;
};

// One sequence's device state for every layer, in one allocation.
struct Slot {
    void *memory = nullptr;
    std::vector<adi_hip_layer_state> layers;
    std::vector<std::pair<float *, size_t>> zeroed;  // linear states, cleared on admission
    adi_hip_decoder_state state{};
    bool busy = false;
};

double seconds_between(Clock::time_point a, Clock::time_point b) {
    return std::chrono::duration<double>(b - a).count();
}

}  // namespace
}  // namespace adi_hip

using namespace adi_hip;

struct adi_hip_batcher {
    adi_hip_context *ctx = nullptr;
    std::vector<adi_hip_decoder_layer> layers;
    std::vector<adi_hip_head_chunk> heads;
    adi_hip_embedding embedding{};
    adi_hip_model model{};
    uint32_t vocabulary = 0;
    uint32_t context = 0;
    uint32_t max_batch = 0;
    uint32_t ubatch = 0;
    std::unordered_set<uint32_t> stop;
    uint32_t masked_count = 0;
    uint32_t *masked = nullptr;  // device
    float *logits = nullptr;     // device [max_batch][vocabulary]
    uint32_t *tokens = nullptr;  // device [max_batch]
    uint64_t *words = nullptr;   // device [max_batch]
    std::vector<Slot> slots;
    std::vector<Active> active;  // logits row i belongs to active[i]
    // host-forced failures for the failure-handling tests: the next
    // admission, or the next step's sampling, fails as a device error would
    // the decode step recorded as a HIP graph for the rows' slots
    // graph_slots; last_slots and stable_steps track how long the same rows
    // have run
    adi_hip_decode_graph *graph = nullptr;
    std::vector<uint32_t> graph_slots;
    std::vector<uint32_t> last_slots;
    uint32_t stable_steps = 0;
    bool use_graphs = true;
    std::atomic<bool> fail_admission_for_testing{false};
    std::atomic<bool> fail_step_for_testing{false};

    std::mutex mutex;  // guards the fields below
    std::deque<uint64_t> pending;
    std::unordered_map<uint64_t, Request> requests;
    uint64_t next_id = 1;
};

namespace adi_hip {
namespace {

void free_batcher(adi_hip_batcher *b) {
    if (b->graph != nullptr) {
        adi_hip_decode_graph_destroy(b->graph);
        b->graph = nullptr;
    }
    for (Slot &s : b->slots) {
        if (s.memory != nullptr) {
            (void)hipFree(s.memory);
        }
    }
    for (void *p : {static_cast<void *>(b->masked), static_cast<void *>(b->logits),
                    static_cast<void *>(b->tokens), static_cast<void *>(b->words)}) {
        if (p != nullptr) {
            (void)hipFree(p);
        }
    }
    delete b;
}

void mask_rows(adi_hip_batcher *b, uint32_t first, uint32_t rows) {
    if (b->masked_count == 0 || rows == 0) {
        return;
    }
    launch(b->ctx, "mask_logits", k_mask_logits, dim3(ceil_div(b->masked_count, 256), rows),
           dim3(256), 0, b->logits + static_cast<size_t>(first) * b->vocabulary, b->vocabulary,
           static_cast<const uint32_t *>(b->masked), b->masked_count);
}

// Records a request's failure (Impl::fail); the caller holds no lock.
void fail_request(adi_hip_batcher *b, uint64_t id, const std::string &message) {
    std::lock_guard<std::mutex> lock(b->mutex);
    auto it = b->requests.find(id);
    if (it != b->requests.end()) {
        it->second.state = ADI_HIP_REQUEST_FAILED;
        it->second.error = message;
    }
}

// resolved_output_limit (src/generation.cpp:25-44) with 0 as "no limit".
uint32_t output_limit(uint32_t context, size_t prompt, uint32_t requested) {
    if (prompt >= context) {
        fail(ADI_HIP_INVALID_ARGUMENT, "prompt exceeds model context");
    }
    const uint32_t remaining = context - static_cast<uint32_t>(prompt);
    if (requested == 0) {
        return remaining;
    }
    if (requested > remaining) {
        fail(ADI_HIP_INVALID_ARGUMENT, "prompt exceeds model context");
    }
    return requested;
}

// Impl::admit (src/generation.cpp:443-516) of the oldest pending request,
// when a slot is free.
void admit_pending(adi_hip_batcher *b) {
    uint64_t id = 0;
    Request copy;
    {
        std::lock_guard<std::mutex> lock(b->mutex);
        if (b->pending.empty()) {
            return;
        }
        bool free_slot = false;
        for (const Slot &s : b->slots) {
            free_slot = free_slot || !s.busy;
        }
        if (!free_slot) {
            return;
        }
        id = b->pending.front();
        b->pending.pop_front();
        auto it = b->requests.find(id);
        if (it == b->requests.end()) {
            return;  // released while pending
        }
        copy = it->second;
    }
    uint32_t limit = 0;
    try {
        if (copy.cancelled) {
            fail(ADI_HIP_INVALID_ARGUMENT, "generation cancelled");
        }
        if (copy.prompt.empty()) {
            fail(ADI_HIP_INVALID_ARGUMENT, "prompt exceeds model context");
        }
        limit = output_limit(b->context, copy.prompt.size(), copy.options.max_output_tokens);
    } catch (const Failure &f) {
        fail_request(b, id, f.message);
        return;
    }
    uint32_t slot = 0;
    while (b->slots[slot].busy) {
        ++slot;
    }
    Slot &s = b->slots[slot];
    const uint32_t row = static_cast<uint32_t>(b->active.size());
    // Any failure from here on fails this request alone (Impl::admit_pending,
    // src/generation.cpp:520-540): the slot stays free and the loop goes on.
    // The synchronize also reads the one-launch MoE block's error word, so a
    // prompt whose layers ran on invalid MoE outputs is failed here instead
    // of being sampled.
    const auto started = Clock::now();
    try {
        for (const auto &z : s.zeroed) {
            check_hip(hipMemsetAsync(z.first, 0, z.second, b->ctx->stream), "sequence state clear");
        }
        s.state.position = 0;
        int status = adi_hip_prefill(b->ctx, &b->model, copy.prompt.data(),
                                     static_cast<uint32_t>(copy.prompt.size()), b->ubatch, &s.state,
                                     b->logits + static_cast<size_t>(row) * b->vocabulary);
        if (status == ADI_HIP_OK) {
            mask_rows(b, row, 1);
            status = adi_hip_synchronize(b->ctx);
        }
        if (status != ADI_HIP_OK) {
            fail(status, b->ctx->last_error());
        }
        if (b->fail_admission_for_testing.exchange(false)) {
            fail(ADI_HIP_DEVICE_ERROR, "admission failure forced by the host");
        }
    } catch (const Failure &f) {
        fail_request(b, id, f.message);
        return;
    } catch (const std::exception &e) {
        fail_request(b, id, e.what());
        return;
    }
    const auto finished = Clock::now();
    s.busy = true;
    b->active.push_back(Active{id, slot, limit, copy.options.temperature, copy.options.top_p,
                               std::mt19937_64(copy.options.seed), finished});
    std::lock_guard<std::mutex> lock(b->mutex);
    Request &r = b->requests[id];
    r.state = ADI_HIP_REQUEST_RUNNING;
    r.max_output = limit;
    r.prefill_seconds = seconds_between(started, finished);
}

// Destroys the recorded decode step (its rows changed).
void drop_graph(adi_hip_batcher *b) {
    if (b->graph != nullptr) {
        adi_hip_decode_graph_destroy(b->graph);
        b->graph = nullptr;
        b->graph_slots.clear();
    }
}

// Fails every active request with `message` and frees their slots (the
// decode-failure branch of the worker loop, src/generation.cpp:640-652).
void fail_active(adi_hip_batcher *b, const std::string &message) {
    drop_graph(b);
    for (const Active &a : b->active) {
        fail_request(b, a.id, message);
        b->slots[a.slot].busy = false;
    }
    b->active.clear();
}

// sample_token for every active row: the greedy choice or the top-p draw,
// one launch per run of rows with the same temperature and top_p.
void sample_active(adi_hip_batcher *b, std::vector<uint32_t> &chosen) {
    const uint32_t n = static_cast<uint32_t>(b->active.size());
    std::vector<uint64_t> draws(n, 0);
    for (uint32_t i = 0; i < n; ++i) {
        if (b->active[i].temperature > 0.0f) {
            draws[i] = b->active[i].random();  // the one draw of uniform_real_distribution
        }
    }
    for (uint32_t first = 0; first < n; first += kWordGroup) {
        Words w{};
        const uint32_t count = n - first < kWordGroup ? n - first : kWordGroup;
        for (uint32_t i = 0; i < count; ++i) {
            w.word[i] = draws[first + i];
        }
        launch(b->ctx, "store_words", k_store_words, dim3(1), dim3(64), 0, b->words + first, w, count);
    }
    for (uint32_t first = 0; first < n;) {
        uint32_t end = first + 1;
        while (end < n && b->active[end].temperature == b->active[first].temperature &&
               b->active[end].top_p == b->active[first].top_p) {
            ++end;
        }
        const float *rows = b->logits + static_cast<size_t>(first) * b->vocabulary;
        const int status =
            b->active[first].temperature == 0.0f
                ? adi_hip_argmax_rows(b->ctx, rows, end - first, b->vocabulary, b->tokens + first)
                : adi_hip_sample_rows(b->ctx, rows, end - first, b->vocabulary,
                                      b->active[first].temperature, b->active[first].top_p,
                                      b->words + first, b->tokens + first);
        if (status != ADI_HIP_OK) {
            const std::string message = b->ctx->last_error();
            fail_active(b, message);
            fail(status, message);
        }
        first = end;
    }
    chosen.assign(n, 0);
    int status = ADI_HIP_OK;
    if (hipMemcpyAsync(chosen.data(), b->tokens, size_t(n) * 4, hipMemcpyDeviceToHost,
                       b->ctx->stream) != hipSuccess) {
        status = ADI_HIP_DEVICE_ERROR;
    }
    // the synchronize reports a one-launch MoE wait that ran out in the last
    // decode step: its logits are invalid, so every active request fails
    // (their draws are spent) instead of sampling them
    const int synced = adi_hip_synchronize(b->ctx);
    if (status == ADI_HIP_OK && synced != ADI_HIP_OK) {
        status = synced;
    }
    if (status == ADI_HIP_OK && b->fail_step_for_testing.exchange(false)) {
        b->ctx->set_error("decode step failure forced by the host");
        status = ADI_HIP_DEVICE_ERROR;
    }
    if (status != ADI_HIP_OK) {
        const std::string message =
            synced != ADI_HIP_OK || b->ctx->last_error().size() > 0 ? b->ctx->last_error()
                                                                    : std::string("token copy failed");
        fail_active(b, message);
        fail(status, message);
    }
}

// The rest of one loop iteration (src/generation.cpp:568-646): finish or
// keep each active sequence, then one decode step of the survivors.
void step_active(adi_hip_batcher *b) {
    std::vector<uint32_t> chosen;
    sample_active(b, chosen);
    std::vector<Active> next;
    std::vector<uint32_t> next_tokens;
    std::vector<adi_hip_decoder_state> next_states;
    const auto now = Clock::now();
    {
        std::lock_guard<std::mutex> lock(b->mutex);
        for (uint32_t i = 0; i < b->active.size(); ++i) {
            Active &a = b->active[i];
            Request &r = b->requests[a.id];
            const uint32_t token = chosen[i];
            bool done = true;
            if (r.cancelled) {
                r.state = ADI_HIP_REQUEST_FAILED;
                r.error = "generation cancelled";
            } else if (token == kNoToken || token >= b->vocabulary) {
                r.state = ADI_HIP_REQUEST_FAILED;
                r.error = "invalid sampling parameters";
            } else if (b->stop.count(token) != 0) {
                r.state = ADI_HIP_REQUEST_STOP_TOKEN;
            } else {
                r.output.push_back(token);
                if (r.output.size() == a.max_output) {
                    r.state = ADI_HIP_REQUEST_LENGTH;
                } else {
                    done = false;
                }
            }
            if (done) {
                r.decode_seconds = seconds_between(a.decode_started, now);
                b->slots[a.slot].busy = false;
                continue;
            }
            next_tokens.push_back(token);
            next_states.push_back(b->slots[a.slot].state);
            next.push_back(std::move(a));
        }
    }
    // nobody left: row i is still active[i], so the sampled tokens already
    // sit in b->tokens in the order of the rows
    const bool same_rows = next.size() == b->active.size();
    b->active = std::move(next);
    if (b->active.empty()) {
        drop_graph(b);
        return;
    }
    const uint32_t n = static_cast<uint32_t>(b->active.size());
    std::vector<uint32_t> slots(n);
    for (uint32_t i = 0; i < n; ++i) {
        slots[i] = b->active[i].slot;
    }
    int status = ADI_HIP_OK;
    if (same_rows && b->graph != nullptr && slots == b->graph_slots) {
        // the same sequences as the recorded step: replay it
        status = adi_hip_decode_graph_launch(b->graph, next_states.data());
    } else {
        drop_graph(b);
        status = adi_hip_decode_batch(b->ctx, &b->model, next_tokens.data(), n, next_states.data(),
                                      b->logits);
        // record a step once the same rows have run twice in a row: a set
        // of rows that changes every iteration (admissions, finishes) would
        // not replay its recording
        b->stable_steps = same_rows && slots == b->last_slots ? b->stable_steps + 1 : 0;
        b->last_slots = slots;
        if (status == ADI_HIP_OK && b->use_graphs && b->stable_steps >= 1) {
            adi_hip_decoder_state *after = next_states.data();
            if (adi_hip_decode_graph_create(b->ctx, &b->model, n, after, b->tokens, b->logits,
                                            &b->graph) == ADI_HIP_OK) {
                b->graph_slots = slots;
            } else {
                b->graph = nullptr;  // the direct launches serve instead
            }
        }
    }
    if (status != ADI_HIP_OK) {
        const std::string message = b->ctx->last_error();
        drop_graph(b);
        fail_active(b, message);
        fail(status, message);
    }
    for (uint32_t i = 0; i < n; ++i) {
        b->slots[b->active[i].slot].state.position = next_states[i].position;
    }
    mask_rows(b, 0, n);
}

}  // namespace
}  // namespace adi_hip

extern "C" {

int adi_hip_batcher_create(adi_hip_context *ctx, const adi_hip_model *model,
                           const adi_hip_batcher_options *options, adi_hip_batcher **out) {
    return guarded(ctx, [&] {
        require(out != nullptr && model != nullptr && options != nullptr, "batcher: null argument");
        *out = nullptr;
        require(model->layers > 0 && model->layer != nullptr && model->embedding != nullptr &&
                    model->head_chunks > 0 && model->head != nullptr && model->final_norm != nullptr,
                "model descriptor is incomplete");
        require(options->max_batch >= 1 && options->max_batch <= kMaxSlots,
                "batcher max_batch must be in [1, 256]");
        require(options->capacity > 0 && options->capacity <= model->context,
                "batcher capacity must be in [1, the model's context]");
        require(options->prefill_ubatch <= 4096, "prefill_ubatch must be in [1, 4096]");
        auto *b = new adi_hip_batcher;
        try {
            b->ctx = ctx;
            b->layers.assign(model->layer, model->layer + model->layers);
            b->heads.assign(model->head, model->head + model->head_chunks);
            b->embedding = *model->embedding;
            b->model = *model;
            b->model.layer = b->layers.data();
            b->model.head = b->heads.data();
            b->model.embedding = &b->embedding;
            b->vocabulary = b->embedding.rows;
            b->context = options->capacity;
            b->max_batch = options->max_batch;
            b->ubatch = options->prefill_ubatch;
            b->use_graphs = options->direct_steps == 0;
            for (uint32_t i = 0; i < options->stop_count; ++i) {
                require(options->stop_tokens[i] < b->vocabulary, "batcher stop token is out of range");
                b->stop.insert(options->stop_tokens[i]);
            }
            for (uint32_t i = 0; i < options->masked_count; ++i) {
                require(options->masked_tokens[i] < b->vocabulary,
                        "batcher masked token is out of range");
            }
            b->masked_count = options->masked_count;
            if (b->masked_count > 0) {
                check_hip(hipMalloc(&b->masked, size_t(b->masked_count) * 4), "batcher allocation");
                check_hip(hipMemcpy(b->masked, options->masked_tokens, size_t(b->masked_count) * 4,
                                    hipMemcpyHostToDevice),
                          "batcher masked tokens");
            }
            check_hip(hipMalloc(&b->logits, size_t(b->max_batch) * b->vocabulary * 4),
                      "batcher allocation");
            check_hip(hipMalloc(&b->tokens, size_t(b->max_batch) * 4), "batcher allocation");
            check_hip(hipMalloc(&b->words, size_t(b->max_batch) * 8), "batcher allocation");
            const size_t kv = size_t(options->capacity) * 2 * 256 * 4;
            const size_t conv = size_t(8192) * 3 * 4, rec = size_t(32) * 128 * 128 * 4;
            size_t bytes = 0;
            for (const auto &L : b->layers) {
                bytes += L.full_attention != 0 ? 2 * kv : conv + rec;
            }
            b->slots.resize(b->max_batch);
            for (Slot &s : b->slots) {
                check_hip(hipMalloc(&s.memory, bytes), "batcher sequence state allocation");
                char *p = static_cast<char *>(s.memory);
                for (const auto &L : b->layers) {
                    adi_hip_layer_state st{};
                    if (L.full_attention != 0) {
                        st.keys = reinterpret_cast<float *>(p);
                        st.values = reinterpret_cast<float *>(p + kv);
                        st.capacity = options->capacity;
                        p += 2 * kv;
                    } else {
                        st.convolution = reinterpret_cast<float *>(p);
                        st.recurrent = reinterpret_cast<float *>(p + conv);
                        s.zeroed.emplace_back(st.convolution, conv + rec);
                        p += conv + rec;
                    }
                    s.layers.push_back(st);
                }
                s.state.layers = s.layers.data();
            }
        } catch (...) {
            free_batcher(b);
            throw;
        }
        *out = b;
    });
}

void adi_hip_batcher_destroy(adi_hip_batcher *batcher) {
    if (batcher == nullptr) {
        return;
    }
    (void)hipStreamSynchronize(batcher->ctx->stream);
    free_batcher(batcher);
}

int adi_hip_batcher_submit(adi_hip_batcher *b, const uint32_t *prompt, uint32_t count,
                           const adi_hip_generation_options *options, uint64_t *request) {
    if (b == nullptr) {
        return ADI_HIP_INVALID_ARGUMENT;
    }
    return guarded(b->ctx, [&] {
        require(options != nullptr && request != nullptr && (prompt != nullptr || count == 0),
                "batcher: null argument");
        // validate_generation_options (src/generation.cpp:93-110)
        require(options->max_output_tokens <= b->model.context,
                "max_output_tokens exceeds model context");
        const float t = options->temperature, p = options->top_p;
        require(std::isfinite(t) && std::isfinite(p) && t >= 0.0f && !(t > 0.0f && t < 1.0e-4f) &&
                    t <= 2.0f && p > 0.0f && p <= 1.0f,
                "invalid generation options");
        Request r;
        r.prompt.assign(prompt, prompt + count);
        r.options = *options;
        std::lock_guard<std::mutex> lock(b->mutex);
        const uint64_t id = b->next_id++;
        b->requests.emplace(id, std::move(r));
        b->pending.push_back(id);
        *request = id;
    });
}

int adi_hip_batcher_cancel(adi_hip_batcher *b, uint64_t request) {
    if (b == nullptr) {
        return ADI_HIP_INVALID_ARGUMENT;
    }
    std::lock_guard<std::mutex> lock(b->mutex);
    auto it = b->requests.find(request);
    if (it == b->requests.end()) {
        return ADI_HIP_INVALID_ARGUMENT;
    }
    it->second.cancelled = true;
    return ADI_HIP_OK;
}

int adi_hip_batcher_step(adi_hip_batcher *b, uint32_t *remaining) {
    if (b == nullptr) {
        return ADI_HIP_INVALID_ARGUMENT;
    }
    const int status = guarded(b->ctx, [&] {
        admit_pending(b);
        if (!b->active.empty()) {
            step_active(b);
        }
    });
    if (remaining != nullptr) {
        std::lock_guard<std::mutex> lock(b->mutex);
        *remaining = static_cast<uint32_t>(b->pending.size() + b->active.size());
    }
    return status;
}

int adi_hip_batcher_status(adi_hip_batcher *b, uint64_t request, adi_hip_request_status *status,
                           uint32_t *tokens, uint32_t capacity) {
    if (b == nullptr || status == nullptr) {
        return ADI_HIP_INVALID_ARGUMENT;
    }
    std::lock_guard<std::mutex> lock(b->mutex);
    auto it = b->requests.find(request);
    if (it == b->requests.end()) {
        return ADI_HIP_INVALID_ARGUMENT;
    }
    const Request &r = it->second;
    status->state = r.state;
    status->input_tokens = static_cast<uint32_t>(r.prompt.size());
    status->output_tokens = static_cast<uint32_t>(r.output.size());
    status->prefill_seconds = r.prefill_seconds;
    status->decode_seconds = r.decode_seconds;
    for (uint32_t i = 0; tokens != nullptr && i < capacity && i < r.output.size(); ++i) {
        tokens[i] = r.output[i];
    }
    return ADI_HIP_OK;
}

const char *adi_hip_batcher_request_error(adi_hip_batcher *b, uint64_t request) {
    if (b == nullptr) {
        return "";
    }
    std::lock_guard<std::mutex> lock(b->mutex);
    auto it = b->requests.find(request);
    return it == b->requests.end() ? "" : it->second.error.c_str();
}

int adi_hip_batcher_force_failure(adi_hip_batcher *b, int where) {
    if (b == nullptr ||
        (where != ADI_HIP_BATCHER_FAIL_ADMISSION && where != ADI_HIP_BATCHER_FAIL_STEP)) {
        return ADI_HIP_INVALID_ARGUMENT;
    }
    if (where == ADI_HIP_BATCHER_FAIL_ADMISSION) {
        b->fail_admission_for_testing = true;
    } else {
        b->fail_step_for_testing = true;
    }
    return ADI_HIP_OK;
}

int adi_hip_batcher_release(adi_hip_batcher *b, uint64_t request) {
    if (b == nullptr) {
        return ADI_HIP_INVALID_ARGUMENT;
    }
    std::lock_guard<std::mutex> lock(b->mutex);
    auto it = b->requests.find(request);
    if (it == b->requests.end() || it->second.state == ADI_HIP_REQUEST_RUNNING ||
        it->second.state == ADI_HIP_REQUEST_PENDING) {
        return ADI_HIP_INVALID_ARGUMENT;
    }
    b->requests.erase(it);
    return ADI_HIP_OK;
}

}  // extern "C"
