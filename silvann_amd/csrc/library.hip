// library.hip — the library's control entry points: which stream a thread's doors are queued on, the
// remembered launch failure, and the build's name.
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <atomic>
#include <vector>

#include "common.hpp"
#include "../../include/silvann_gfx950_attention.h"

namespace silvann {

// A door runs on its caller's thread, a worker's runner thread bound to its device (reference
// engine/src/engine/launch.cuh:51-60), so the stream is the thread's own. A refused or failed launch is
// remembered for its DEVICE, as the reference family does (amd_rocm_base/sys.cuh:39-62): the thread that
// waits for a worker's answer is not always the thread that launched there.
static thread_local hipStream_t tls_stream = nullptr;
constexpr int kDevicesSeen = 64;
static std::atomic<int> failed[kDevicesSeen];

static void mark_failed() {
    int d = -1;
    if (hipGetDevice(&d) == hipSuccess && d >= 0 && d < kDevicesSeen) failed[d].store(1);
}

hipStream_t stream() { return tls_stream; }

void check_launch(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        fprintf(stderr, "silvann_gfx950: launch of %s failed: %s\n", what, hipGetErrorString(e));
        mark_failed();
    }
}

struct Prof {
    bool on = false;
    std::vector<hipEvent_t> free_events;
    std::vector<std::pair<hipEvent_t, hipEvent_t>> done[kProfKernels];
    hipEvent_t open[kProfKernels] = {};
};
static thread_local Prof tls_prof;

static hipEvent_t prof_event() {
    Prof& P = tls_prof;
    if (!P.free_events.empty()) {
        hipEvent_t e = P.free_events.back();
        P.free_events.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
}

void prof_begin(int kernel) {
    Prof& P = tls_prof;
    if (!P.on) return;
    hipEvent_t e = prof_event();
    if (e && hipEventRecord(e, tls_stream) == hipSuccess) P.open[kernel] = e;
}

void prof_end(int kernel) {
    Prof& P = tls_prof;
    if (!P.on || !P.open[kernel]) return;
    hipEvent_t e = prof_event();
    if (e && hipEventRecord(e, tls_stream) == hipSuccess) P.done[kernel].push_back({P.open[kernel], e});
    P.open[kernel] = nullptr;
}

void refuse(const char* what) {
    fprintf(stderr, "silvann_gfx950: %s refused its operands\n", what);
    mark_failed();
}

static thread_local Deferred tls_deferred;
Deferred& deferred() { return tls_deferred; }

// On unless SILVANN_GFX950_DEFER=0 (read once a process); each thread may switch its own.
static bool defer_default() {
    static const bool on = [] {
        const char* e = getenv("SILVANN_GFX950_DEFER");
        return !(e && strcmp(e, "0") == 0);
    }();
    return on;
}
static thread_local int tls_defer = -1;   // -1: the process default
bool defer_enabled() { return tls_defer < 0 ? defer_default() : tls_defer != 0; }

}  // namespace silvann

SILVANN_EXPORT void silvann_gfx950_set_stream(void* s) {
    silvann::flush_deferred();   // what is recorded runs on the stream it was recorded on
    silvann::tls_stream = (hipStream_t)s;
}
SILVANN_EXPORT void* silvann_gfx950_get_stream(void) { return (void*)silvann::tls_stream; }
SILVANN_EXPORT void silvann_gfx950_flush(void) { silvann::flush_deferred(); }
SILVANN_EXPORT void silvann_gfx950_set_defer(int on) {
    silvann::flush_deferred();
    silvann::tls_defer = on != 0;
}
SILVANN_EXPORT int silvann_gfx950_launch_failed(void) {
    silvann::flush_deferred();
    int d = -1;
    if (hipGetDevice(&d) != hipSuccess || d < 0 || d >= silvann::kDevicesSeen) return 0;
    return silvann::failed[d].exchange(0);
}
static int prof_index(const char* kernel) {
    static const char* names[silvann::kProfKernels] = {"decode_split", "decode_merge", "causal_mfma", "tq_split",
                                                              "cache_write"};
    for (int i = 0; i < silvann::kProfKernels; ++i)
        if (kernel && strcmp(kernel, names[i]) == 0) return i;
    return -1;
}

SILVANN_EXPORT void silvann_gfx950_profile_enable(int on) { silvann::tls_prof.on = on != 0; }

SILVANN_EXPORT int silvann_gfx950_profile_read(const char* kernel, double* total_ms, uint64_t* launches) {
    const int k = prof_index(kernel);
    if (k < 0) return -1;
    silvann::Prof& P = silvann::tls_prof;
    double sum = 0.0;
    uint64_t n = 0;
    for (auto& pr : P.done[k]) {
        float ms = 0.0f;
        if (hipEventSynchronize(pr.second) != hipSuccess) return -1;
        if (hipEventElapsedTime(&ms, pr.first, pr.second) != hipSuccess) return -1;
        sum += ms;
        ++n;
        P.free_events.push_back(pr.first);
        P.free_events.push_back(pr.second);
    }
    P.done[k].clear();
    if (total_ms) *total_ms = sum;
    if (launches) *launches = n;
    return 0;
}

namespace {
struct Row {
    uint32_t index;
    void* fn;
};
}  // namespace

SILVANN_EXPORT uint32_t silvann_gfx950_attention_install(void* nn_doors) {
    if (!nn_doors) return 0;
    const Row rows[] = {
        {SILVANN_GFX950_ROW_ATTENTION_SCORES, (void*)&silvann_gfx950_attention_scores},
        {SILVANN_GFX950_ROW_ATTENTION_MIX, (void*)&silvann_gfx950_attention_mix},
        {SILVANN_GFX950_ROW_ATTENTION_WEIGHTS, (void*)&silvann_gfx950_attention_weights},
        {SILVANN_GFX950_ROW_ATTENTION_RESIDUAL_MIX, (void*)&silvann_gfx950_attention_residual_mix},
        {SILVANN_GFX950_ROW_ATTENTION_MERGE, (void*)&silvann_gfx950_attention_merge},
        {SILVANN_GFX950_ROW_ATTENTION_FINISH, (void*)&silvann_gfx950_attention_finish},
        {SILVANN_GFX950_ROW_ATTENTION_CAUSAL_SCORES, (void*)&silvann_gfx950_attention_causal_scores},
        {SILVANN_GFX950_ROW_ATTENTION_CAUSAL_MIX, (void*)&silvann_gfx950_attention_causal_mix},
        {SILVANN_GFX950_ROW_ATTENTION_WEIGHTS_TQ, (void*)&silvann_gfx950_attention_weights_tq},
        {SILVANN_GFX950_ROW_ATTENTION_RESIDUAL_MIX_TQ, (void*)&silvann_gfx950_attention_residual_mix_tq},
        {SILVANN_GFX950_ROW_ATTENTION_SCORES_GROUPED, (void*)&silvann_gfx950_attention_scores_grouped},
        {SILVANN_GFX950_ROW_ATTENTION_SOFTMAX_ROWS, (void*)&silvann_gfx950_attention_softmax_rows},
        {SILVANN_GFX950_ROW_ATTENTION_CAUSAL_SCORES_GROUPED, (void*)&silvann_gfx950_attention_causal_scores_grouped},
        {SILVANN_GFX950_ROW_ATTENTION_CAUSAL_SOFTMAX, (void*)&silvann_gfx950_attention_causal_softmax},
        {SILVANN_GFX950_ROW_ATTENTION_SOFTMAX_SINK, (void*)&silvann_gfx950_attention_softmax_sink},
        {SILVANN_GFX950_ROW_ATTENTION_WEIGHTS_ROWS, (void*)&silvann_gfx950_attention_weights_rows},
        {SILVANN_GFX950_ROW_ATTENTION_RESIDUAL_MIX_ROWS, (void*)&silvann_gfx950_attention_residual_mix_rows},
        {SILVANN_GFX950_ROW_ATTENTION_WEIGHTS_TQ_ROWS, (void*)&silvann_gfx950_attention_weights_tq_rows},
        {SILVANN_GFX950_ROW_ATTENTION_RESIDUAL_MIX_TQ_ROWS, (void*)&silvann_gfx950_attention_residual_mix_tq_rows},
        {SILVANN_GFX950_ROW_ATTENTION_SCORES_GROUPED_ROWS, (void*)&silvann_gfx950_attention_scores_grouped_rows},
        {SILVANN_GFX950_ROW_ATTENTION_SOFTMAX_LENS, (void*)&silvann_gfx950_attention_softmax_lens},
        {SILVANN_GFX950_ROW_ATTENTION_MIX_ROWS, (void*)&silvann_gfx950_attention_mix_rows},
        {SILVANN_GFX950_ROW_ROPE_ROWS, (void*)&silvann_gfx950_rope_rows},
        {SILVANN_GFX950_ROW_ATTENTION_DECODE_PAGED, (void*)&silvann_gfx950_attention_decode_paged},
        {SILVANN_GFX950_ROW_ATTENTION_CAUSAL_PAGED, (void*)&silvann_gfx950_attention_causal_paged},
        {SILVANN_GFX950_ROW_ATTENTION_RESIDUAL_TQ, (void*)&silvann_gfx950_attention_residual_tq},
        {SILVANN_GFX950_ROW_ATTENTION_CAUSAL_RESIDUAL_PAGED, (void*)&silvann_gfx950_attention_causal_residual_paged},
        {SILVANN_GFX950_ROW_ATTENTION_CACHE_WRITE_PAGED, (void*)&silvann_gfx950_attention_cache_write_paged},
    };
    uint32_t size;
    memcpy(&size, nn_doors, sizeof size);
    const uint64_t slots = size >= 8 ? (size - 8) / sizeof(void*) : 0;
    void** table = (void**)((char*)nn_doors + 8);
    uint32_t n = 0;
    for (const Row& r : rows)
        if (r.index < slots) {
            table[r.index] = r.fn;
            ++n;
        }
    return n;
}

SILVANN_EXPORT const char* silvann_gfx950_version(void) {
    return "gfx950 decode-splitk-mfma16 causal-mfma32 tq-mfma16 cache-writer doors-28 deferred-chains v1";
}
