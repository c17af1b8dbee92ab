// The Qwen3 32-sequence draft-verify decode's K/V read alone (ragged lengths
// 512..16384, the bench's seeded draw; cache rows of 4 kv heads x 128 f16 =
// 1 KB; K and V: 502 MB), no arithmetic: 256 workgroups of 4 waves, each wave
// one 64-key block (K and V, 32 KB) in flight, loaded straight into LDS
// (buffer_load_dwordx4 ... lds, nt), the next block requested when it has
// landed.  Patterns: the stream-K list of one-head blocks split evenly over
// the workgroups (the decode kernel's), and whole-row blocks (all 4 heads of
// 64 keys) with wave = head or wave = 16 rows.  20 launches over 2 copies
// in a HIP graph, HIP events.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <vector>

#define CK(x) do { hipError_t e_ = (x); if (e_ != hipSuccess) { std::printf("HIP error %s at line %d\n", hipGetErrorString(e_), __LINE__); return 1; } } while (0)
// seq_lengths(C5) of pelica_amd/workloads.py
static const int LENS[32] = {7688, 10990, 3836, 6142, 13714, 2346, 7849, 5266, 3722, 13448, 7332, 11011, 12086, 12427, 14022, 16327, 6562, 2079, 4161, 13567, 12236, 6662, 8487, 3775, 8378, 8008, 8817, 6915, 6722, 7703, 3261, 1731};
struct Blk { int row0, nrow, head; };  // head -1: all four heads (whole rows)
__device__ __forceinline__ void dma(__amdgpu_buffer_rsrc_t r, uint32_t off, void* lds) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, off, 0, 0, 2);
}
// MODE 0: list of one-head blocks, wave w takes list items w, w+4, ... of the workgroup's range
// MODE 1: list of whole-row blocks (4 heads); wave w reads head w of every block of the range
// MODE 2: as 1, but wave w reads rows 16w..16w+15 of the block, whole 1 KB rows per instruction
template <int MODE>
__global__ __launch_bounds__(256) void probe(const char* k, const char* v, uint32_t nbytes, const Blk* list, int n, float* sink) {
    __shared__ __attribute__((aligned(16))) char lds[4][32768];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc((void*)k, 0, (int)nbytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc((void*)v, 0, (int)nbytes, 0x00020000);
    const int b0 = (int)((long long)n * blockIdx.x / gridDim.x), b1 = (int)((long long)n * (blockIdx.x + 1) / gridDim.x);
    char* my = lds[wave];
    for (int b = (MODE == 0 ? b0 + wave : b0); b < b1; b += (MODE == 0 ? 4 : 1)) {
        const Blk B = list[b];
        #pragma unroll
        for (int j = 0; j < 16; ++j) {
            uint32_t off;
            if (MODE == 2) {
                const int row = 16 * wave + j;
                off = row < B.nrow ? (uint32_t)(B.row0 + row) * 1024u + 16u * lane : 0xFFFFFFF0u;
            } else {
                const int h = MODE == 0 ? B.head : wave;
                const int row = 4 * j + lane / 16;
                off = row < B.nrow ? (uint32_t)(B.row0 + row) * 1024u + 256u * h + 16u * (lane % 16) : 0xFFFFFFF0u;
            }
            dma(rk, off, my + 1024 * j);
            dma(rv, off, my + 16384 + 1024 * j);
        }
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    }
    __syncthreads();
    if (threadIdx.x == 0) sink[blockIdx.x] = (float)lds[0][0];
}
int main() {
    size_t rows = 0; for (int s = 0; s < 32; ++s) rows += LENS[s];
    const size_t bytes = rows * 1024;
    const int copies = 2;
    char *k, *v; float* sink;
    CK(hipMalloc(&k, bytes * copies)); CK(hipMalloc(&v, bytes * copies)); CK(hipMalloc(&sink, 4096));
    CK(hipMemset(k, 1, bytes * copies)); CK(hipMemset(v, 1, bytes * copies));
    std::vector<Blk> l0, l1;
    int row0 = 0;
    for (int s = 0; s < 32; ++s) {
        for (int h = 0; h < 4; ++h) for (int r = 0; r < LENS[s]; r += 64) l0.push_back({row0 + r, std::min(64, LENS[s] - r), h});
        for (int r = 0; r < LENS[s]; r += 64) l1.push_back({row0 + r, std::min(64, LENS[s] - r), -1});
        row0 += LENS[s];
    }
    Blk *d0, *d1;
    CK(hipMalloc(&d0, l0.size() * sizeof(Blk))); CK(hipMalloc(&d1, l1.size() * sizeof(Blk)));
    CK(hipMemcpy(d0, l0.data(), l0.size() * sizeof(Blk), hipMemcpyHostToDevice));
    CK(hipMemcpy(d1, l1.data(), l1.size() * sizeof(Blk), hipMemcpyHostToDevice));
    hipStream_t st; CK(hipStreamCreate(&st));
    const char* names[3] = {"one-head blocks, list split over 256 wgs (stream-K pattern)", "whole-row blocks, wave = head", "whole-row blocks, wave = 16 rows, 1 KB per instruction"};
    for (int rep = 0; rep < 2; ++rep)
    for (int mode = 0; mode < 3; ++mode) {
        hipGraph_t g; hipGraphExec_t ge;
        CK(hipStreamBeginCapture(st, hipStreamCaptureModeGlobal));
        for (int i = 0; i < 20; ++i) {
            const char* kk = k + (i % copies) * bytes; const char* vv = v + (i % copies) * bytes;
            if (mode == 0) hipLaunchKernelGGL(probe<0>, dim3(256), dim3(256), 0, st, kk, vv, (uint32_t)bytes, d0, (int)l0.size(), sink);
            if (mode == 1) hipLaunchKernelGGL(probe<1>, dim3(256), dim3(256), 0, st, kk, vv, (uint32_t)bytes, d1, (int)l1.size(), sink);
            if (mode == 2) hipLaunchKernelGGL(probe<2>, dim3(256), dim3(256), 0, st, kk, vv, (uint32_t)bytes, d1, (int)l1.size(), sink);
        }
        CK(hipStreamEndCapture(st, &g));
        CK(hipGraphInstantiate(&ge, g, nullptr, nullptr, 0));
        hipEvent_t e0, e1; CK(hipEventCreate(&e0)); CK(hipEventCreate(&e1));
        CK(hipGraphLaunch(ge, st));
        std::vector<float> ts;
        for (int r = 0; r < 5; ++r) {
            CK(hipEventRecord(e0, st)); CK(hipGraphLaunch(ge, st)); CK(hipEventRecord(e1, st)); CK(hipEventSynchronize(e1));
            float ms; CK(hipEventElapsedTime(&ms, e0, e1)); ts.push_back(ms * 1000.f / 20);
        }
        std::sort(ts.begin(), ts.end());
        printf("%-60s %.1f us per launch = %.2f TB/s (%zu MB)\n", names[mode], ts[2], 2.0 * bytes / (ts[2] * 1e-6) / 1e12, 2 * bytes >> 20);
    }
    return 0;
}
