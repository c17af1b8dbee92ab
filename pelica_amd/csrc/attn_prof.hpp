// Per-kernel GPU timing (the counterpart of the reference's PELICA_PROF
// timestamp queries, src/moe.rs:1761-1833, src/oss.rs:1164-1242): when
// enabled, every kernel the library launches is bracketed by HIP events on
// its stream; pelica_attn_prof_read() waits for them and reports the times.
// Launches on a capturing stream are not timed.
#pragma once
#include <hip/hip_runtime.h>

namespace pelica {

enum ProfKernel { kProfDecodeSplit = 1, kProfDecodeCombine = 2, kProfPrefill = 3, kProfMerge = 4, kProfQkv = 5 };

bool prof_enabled();
// opens a record (start event) for `kind` on `st`; returns a handle or -1
int prof_begin(int kind, hipStream_t st);
// closes it (stop event)
void prof_end(int handle, hipStream_t st);

struct ProfScope {
    int h;
    hipStream_t st;
    ProfScope(int kind, hipStream_t s) : h(prof_enabled() ? prof_begin(kind, s) : -1), st(s) {}
    ~ProfScope() {
        if (h >= 0) prof_end(h, st);
    }
};

}  // namespace pelica
