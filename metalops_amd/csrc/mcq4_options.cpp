// Snapshot of the library's MCQ4_* switches (see mcq4_options.h).  A reload
// publishes a new immutable snapshot through an atomic pointer; the old one is
// kept alive (a few hundred bytes per reload) so that a launch running on
// another thread never reads freed memory.
#include <algorithm>
#include <atomic>
#include <mutex>
#include <stdlib.h>
#include <string.h>
#include <string>

#include "mcq4_options.h"
#include "../../include/mcq4.h"

namespace {

const char *const kNames[] = {
    // q4_0 path
    "MCQ4_XCD_LOCAL",       // 0: split-K partials through memory / the reduction kernel
    "MCQ4_GEMM_PATH",       // sync | async | 6 | 7 | 8: force one prefill kernel
    "MCQ4_GEMM6_SPLIT",     // K splits of the prefill GEMM
    "MCQ4_GEMM8_SPLIT",     // 1 | 2: K splits of the few-tile prefill GEMM
    "MCQ4_GEMV_PATH",       // off: M == 1 through the batched decode kernels
    "MCQ4_GEMV_SPAN",       // 0: no span kernels (strip kernels instead); 1: the split form wherever it fits
    "MCQ4_GEMVM_SPLIT",     // 1 | 2 | 4 | 8: K splits of the batched decode GEMV
    "MCQ4_GEMVM_HOIST",     // 0: batched decode GEMV rebuilds -S per item even with one batch per wave
    "MCQ4_DECODE_PATH",     // direct: the register-load decode kernel
    "MCQ4_GEMM2_BM",        // 128 | 256: row tile of the fallback prefill kernel
    "MCQ4_SPLIT_FOREIGN",   // mask: split-K splits treated as run on another XCD (recompute path)
    "MCQ4_SPLIT_SPIN",      // polls of a split flag before the split is recomputed (default 256; 0: at once)
    // per-group INT4 / INT8 path
    "MCQ4_I4_PATH",         // generic: the general kernel for everything
    "MCQ4_I4_RMS_FUSE",     // 0: fused RMSNorm + INT4 at M = 1 runs as two kernels
    "MCQ4_I4_GEMV1",        // 0 | 1 | 4: async-copy decode GEMV routing
    "MCQ4_I4_SPW1",         // steps per wave of the async-copy decode GEMV
    "MCQ4_I4_GEMM6",        // 0: the barrier-free prefill kernel
    "MCQ4_I4_GEMM7",        // 0: no 256 x 256-tile prefill kernel; 1: that kernel whatever the grid
};
constexpr int kN = sizeof(kNames) / sizeof(kNames[0]);

struct Snapshot {
    std::string value[kN];
    bool set[kN];
};

std::atomic<const Snapshot *> g_snap{nullptr};
std::mutex g_mu;

const Snapshot *load() {
    Snapshot *s = new Snapshot;
    for (int i = 0; i < kN; ++i) {
        const char *v = getenv(kNames[i]);
        s->set[i] = v != nullptr;
        s->value[i] = v ? v : "";
    }
    return s;
}

}  // namespace

namespace mcq4 {
const char *opt(const char *name) {
    const Snapshot *s = g_snap.load(std::memory_order_acquire);
    if (!s) {
        std::lock_guard<std::mutex> lk(g_mu);
        s = g_snap.load(std::memory_order_acquire);
        if (!s) {
            s = load();
            g_snap.store(s, std::memory_order_release);
        }
    }
    for (int i = 0; i < kN; ++i)
        if (strcmp(kNames[i], name) == 0) return s->set[i] ? s->value[i].c_str() : nullptr;
    return nullptr;
}
uint32_t split_foreign_mask() {
    const char *v = opt("MCQ4_SPLIT_FOREIGN");
    return v ? (uint32_t)strtoul(v, nullptr, 0) : 0u;
}
uint32_t split_spin() {
    const char *v = opt("MCQ4_SPLIT_SPIN");
    return v ? (uint32_t)std::min<unsigned long>(strtoul(v, nullptr, 0), 1u << 20) : 256u;
}
}  // namespace mcq4

extern "C" int mcq4_reload_options(void) {
    std::lock_guard<std::mutex> lk(g_mu);
    g_snap.store(load(), std::memory_order_release);   // the previous snapshot is leaked on purpose
    return MCQ4_OK;
}
