// Cost of a dependent small kernel after a large one (the decode split
// kernel + combine launch shape): a "big" kernel reads 64 MB (256
// workgroups x 256 KB) and writes 1 MB of partials; a "small" kernel of 256
// workgroups reads 8 partials per thread and writes them out.  Graph of 64
// steps (big; big + small; big + small + small), per-step time from HIP
// events.  The partials are stored with the default policy, sc1 (written
// through to the coherence point, nothing left dirty in L2), nt, or sc0 nt.
// Built twice: as is, and with kernel arguments preloaded into SGPRs
// (-mllvm -amdgpu-kernarg-preload-count=16).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <vector>

#define CK(x)                                                                              \
    do {                                                                                   \
        hipError_t e_ = (x);                                                               \
        if (e_ != hipSuccess) {                                                            \
            std::printf("HIP error %s at line %d\n", hipGetErrorString(e_), __LINE__);     \
            return 1;                                                                      \
        }                                                                                  \
    } while (0)

typedef float f4 __attribute__((ext_vector_type(4)));
typedef unsigned u4 __attribute__((ext_vector_type(4)));

template <int AUX>  // store policy of the partials: -1 default, else buffer-store cache bits
__global__ __launch_bounds__(256) void big(const f4* __restrict__ src, f4* __restrict__ part, int per_wg) {
    const f4* s = src + (size_t)blockIdx.x * per_wg;
    f4 acc = {0, 0, 0, 0};
    for (int i = threadIdx.x; i < per_wg; i += 256) acc += __builtin_nontemporal_load(s + i);
    if constexpr (AUX < 0) {
        part[blockIdx.x * 256 + threadIdx.x] = acc;
    } else {
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4, acc),
                                               __builtin_amdgcn_make_buffer_rsrc(part, 0, 0x7fffffff, 0x00020000),
                                               (blockIdx.x * 256 + threadIdx.x) * 16, 0, AUX);
    }
}

__global__ __launch_bounds__(256) void small_k(const f4* __restrict__ part, f4* __restrict__ out, int n) {
    f4 a = {0, 0, 0, 0};
#pragma unroll
    for (int j = 0; j < 8; ++j) a += part[((blockIdx.x * 8 + j) * 256 + threadIdx.x) % n];
    out[blockIdx.x * 256 + threadIdx.x] = a;
}

template <int AUX>
static int run(const char* what, hipStream_t st, const f4* src, f4* part, f4* out) {
    const int nwg = 256, per_wg = 16384, copies = 24;
    for (int mode = 0; mode < 3; ++mode) {
        hipGraph_t g;
        hipGraphExec_t ge;
        CK(hipStreamBeginCapture(st, hipStreamCaptureModeGlobal));
        for (int i = 0; i < 64; ++i) {
            hipLaunchKernelGGL(big<AUX>, dim3(nwg), dim3(256), 0, st, src + (size_t)(i % copies) * nwg * per_wg, part, per_wg);
            for (int k = 0; k < mode; ++k) hipLaunchKernelGGL(small_k, dim3(256), dim3(256), 0, st, part, out, nwg * 256);
        }
        CK(hipStreamEndCapture(st, &g));
        CK(hipGraphInstantiate(&ge, g, nullptr, nullptr, 0));
        hipEvent_t e0, e1;
        CK(hipEventCreate(&e0));
        CK(hipEventCreate(&e1));
        for (int w = 0; w < 3; ++w) CK(hipGraphLaunch(ge, st));
        std::vector<float> ts;
        for (int rep = 0; rep < 10; ++rep) {
            CK(hipEventRecord(e0, st));
            CK(hipGraphLaunch(ge, st));
            CK(hipEventRecord(e1, st));
            CK(hipEventSynchronize(e1));
            float ms;
            CK(hipEventElapsedTime(&ms, e0, e1));
            ts.push_back(ms * 1000.f / 64);
        }
        std::sort(ts.begin(), ts.end());
        std::printf("%-22s big%s: median %.2f us per step (min %.2f)\n", what,
                    mode == 0 ? "          " : mode == 1 ? " + small  " : " + 2 small", ts[5], ts[0]);
        CK(hipGraphExecDestroy(ge));
        CK(hipGraphDestroy(g));
    }
    return 0;
}

int main(int argc, char** argv) {
    const char* build = argc > 1 ? argv[1] : "";
    const int nwg = 256, per_wg = 16384, copies = 24;
    f4 *src, *part, *out;
    CK(hipMalloc(&src, (size_t)copies * nwg * per_wg * 16));
    CK(hipMemset(src, 0, (size_t)copies * nwg * per_wg * 16));
    CK(hipMalloc(&part, nwg * 256 * 16));
    CK(hipMalloc(&out, nwg * 256 * 16));
    hipStream_t st;
    CK(hipStreamCreate(&st));
    char name[64];
    std::snprintf(name, sizeof name, "%s stores default", build);
    if (run<-1>(name, st, src, part, out)) return 1;
    std::snprintf(name, sizeof name, "%s stores sc1", build);
    if (run<16>(name, st, src, part, out)) return 1;
    std::snprintf(name, sizeof name, "%s stores nt", build);
    if (run<2>(name, st, src, part, out)) return 1;
    std::snprintf(name, sizeof name, "%s stores sc0 nt", build);
    if (run<3>(name, st, src, part, out)) return 1;
    return 0;
}
