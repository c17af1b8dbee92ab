// Per-kernel GPU timing behind pelica_attn_prof_enable / pelica_attn_prof_read.
#include <atomic>
#include <mutex>
#include <vector>

#include "../../include/pelica_attn.h"
#include "attn_prof.hpp"

namespace pelica {
namespace {

struct Rec {
    int kind;
    hipEvent_t start, stop;
    bool closed;
};

std::atomic<bool> g_on{false};
std::mutex g_mu;
std::vector<Rec> g_recs;
std::vector<hipEvent_t> g_free;  // events kept for reuse
constexpr size_t kMaxRecs = 1 << 14;

hipEvent_t take_event() {
    if (!g_free.empty()) {
        hipEvent_t e = g_free.back();
        g_free.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
}

}  // namespace

bool prof_enabled() { return g_on.load(std::memory_order_relaxed); }

int prof_begin(int kind, hipStream_t st) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(st, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) return -1;
    std::lock_guard<std::mutex> lk(g_mu);
    if (g_recs.size() >= kMaxRecs) return -1;
    Rec r{kind, take_event(), take_event(), false};
    if (!r.start || !r.stop || hipEventRecord(r.start, st) != hipSuccess) {
        if (r.start) g_free.push_back(r.start);
        if (r.stop) g_free.push_back(r.stop);
        return -1;
    }
    g_recs.push_back(r);
    return (int)g_recs.size() - 1;
}

void prof_end(int h, hipStream_t st) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (h < 0 || (size_t)h >= g_recs.size()) return;
    g_recs[h].closed = hipEventRecord(g_recs[h].stop, st) == hipSuccess;
}

}  // namespace pelica

extern "C" {

int pelica_attn_prof_enable(int on) {
    std::lock_guard<std::mutex> lk(pelica::g_mu);
    for (auto& r : pelica::g_recs) {
        pelica::g_free.push_back(r.start);
        pelica::g_free.push_back(r.stop);
    }
    pelica::g_recs.clear();
    pelica::g_on.store(on != 0, std::memory_order_relaxed);
    return PELICA_ATTN_OK;
}

int pelica_attn_prof_read(PelicaAttnProfRecord* out, int max_records) {
    std::lock_guard<std::mutex> lk(pelica::g_mu);
    int n = 0;
    int rc = 0;
    for (auto& r : pelica::g_recs) {
        if (out && n < max_records && r.closed) {
            float ms = 0.f;
            if (hipEventSynchronize(r.stop) != hipSuccess || hipEventElapsedTime(&ms, r.start, r.stop) != hipSuccess)
                rc = PELICA_ATTN_EHIP;
            out[n].kernel = r.kind;
            out[n].ms = ms;
            ++n;
        }
        pelica::g_free.push_back(r.start);
        pelica::g_free.push_back(r.stop);
    }
    pelica::g_recs.clear();
    return rc ? rc : n;
}

}  // extern "C"
