// The gpt-oss 32K decode's K/V read alone (32768 cache rows of 8 kv heads x
// 64 f16 = 1 KB, K and V: 64 MB), with the split kernel's access pattern and
// no arithmetic: 256 workgroups (128 key splits x 2 groups of 4 kv heads) of
// 8 waves; wave (head, phase) takes 64-key blocks phase, phase + 2 of its
// split; a load brings 8 keys x 128 B of one head (16 B a lane) straight
// into LDS (buffer_load_dwordx4 ... lds, nt), as decode_kernel does.
// 48 launches over 16 rotating copies (1 GiB) in a HIP graph, HIP events.
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

constexpr int kRows = 32768, kRowBytes = 1024;

__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, uint32_t off, void* lds) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, off, 0, 0, 2);
}
__device__ __forceinline__ void wait_all() { __builtin_amdgcn_s_waitcnt(0x0F70); }  // vmcnt(0)
__device__ __forceinline__ char* kb_lds(char (*lds)[16384], int wave) { return lds[wave]; }
__device__ __forceinline__ char* kb_lds_k(char* w, int j) { return w + 1024 * j; }

// MODE 0: both blocks of a wave requested at once (into the same LDS buffer)
// MODE 1: the second block requested after the first has landed (the kernel's dependency)
// MODE 2: whole 1 KB rows, one key per load: a workgroup takes 128 keys of all 8 heads
// MODE 3: one kv head per XCD: workgroup i (on XCD i % 8) reads head i % 8 of keys
//         [1024 (i / 8), +1024), its 8 waves two 64-key blocks each (8 keys x 128 B per load)
template <int MODE>
__global__ __launch_bounds__(512) void c3read(const char* k, const char* v, unsigned* sink) {
    __shared__ __attribute__((aligned(16))) char lds[8][16384];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc((void*)k, 0, kRows * kRowBytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc((void*)v, 0, kRows * kRowBytes, 0x00020000);
    char* kb = lds[wave];
    char* vb = kb + 8192;
    if (MODE == 3) {
        const int head = blockIdx.x & 7, key0 = (blockIdx.x >> 3) * 1024;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int kb = key0 + 64 * (wave + 8 * i);
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const uint32_t off = (uint32_t)(kb + 8 * j + lane / 8) * kRowBytes + head * 128 + 16 * (lane % 8);
                dma16(rk, off, kb_lds_k(kb_lds(lds, wave), j));
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const uint32_t off = (uint32_t)(kb + 8 * j + lane / 8) * kRowBytes + head * 128 + 16 * (lane % 8);
                dma16(rv, off, kb_lds(lds, wave) + 8192 + 1024 * j);
            }
            wait_all();
        }
    } else if (MODE == 2) {
        const int key0 = blockIdx.x * 128 + wave * 16;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const uint32_t off = (uint32_t)(key0 + j) * kRowBytes + 16 * lane;
            dma16(rk, off, kb + 512 * (j & 7));
            dma16(rv, off, vb + 512 * (j & 7));
        }
        wait_all();
    } else {
        const int split = blockIdx.x >> 1, hg = blockIdx.x & 1;
        const int head = hg * 4 + (wave & 3), phase = wave >> 2;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int key0 = split * 256 + 64 * (phase + 2 * i);
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const uint32_t off = (uint32_t)(key0 + 8 * j + lane / 8) * kRowBytes + head * 128 + 16 * (lane % 8);
                dma16(rk, off, kb + 1024 * j);
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const uint32_t off = (uint32_t)(key0 + 8 * j + lane / 8) * kRowBytes + head * 128 + 16 * (lane % 8);
                dma16(rv, off, vb + 1024 * j);
            }
            if (MODE == 1) wait_all();
        }
        wait_all();
    }
    __syncthreads();
    if (threadIdx.x == 0 && lds[0][0] == 123) sink[0] = 1;
}

int main() {
    const size_t bytes = (size_t)kRows * kRowBytes;
    const int copies = 16;
    char *k, *v;
    unsigned* sink;
    CK(hipMalloc(&k, bytes * copies));
    CK(hipMalloc(&v, bytes * copies));
    CK(hipMemset(k, 1, bytes * copies));
    CK(hipMemset(v, 1, bytes * copies));
    CK(hipMalloc(&sink, 64));
    hipStream_t st;
    CK(hipStreamCreate(&st));
    const char* names[4] = {"split pattern, both blocks requested at once", "split pattern, second block after the first landed",
                            "whole 1 KB rows, one key per load", "one kv head per XCD, second block after the first"};
    for (int rep = 0; rep < 2; ++rep)
        for (int mode = 0; mode < 4; ++mode) {
            hipGraph_t g;
            hipGraphExec_t ge;
            CK(hipStreamBeginCapture(st, hipStreamCaptureModeGlobal));
            for (int i = 0; i < 48; ++i) {
                const char* kk = k + (i % copies) * bytes;
                const char* vv = v + (i % copies) * bytes;
                if (mode == 0) hipLaunchKernelGGL(c3read<0>, dim3(256), dim3(512), 0, st, kk, vv, sink);
                if (mode == 1) hipLaunchKernelGGL(c3read<1>, dim3(256), dim3(512), 0, st, kk, vv, sink);
                if (mode == 2) hipLaunchKernelGGL(c3read<2>, dim3(256), dim3(512), 0, st, kk, vv, sink);
                if (mode == 3) hipLaunchKernelGGL(c3read<3>, dim3(256), dim3(512), 0, st, kk, vv, sink);
            }
            CK(hipStreamEndCapture(st, &g));
            CK(hipGraphInstantiate(&ge, g, nullptr, nullptr, 0));
            CK(hipGraphLaunch(ge, st));
            hipEvent_t e0, e1;
            CK(hipEventCreate(&e0));
            CK(hipEventCreate(&e1));
            std::vector<double> t;
            for (int r = 0; r < 3; ++r) {
                CK(hipEventRecord(e0, st));
                CK(hipGraphLaunch(ge, st));
                CK(hipEventRecord(e1, st));
                CK(hipEventSynchronize(e1));
                float ms;
                CK(hipEventElapsedTime(&ms, e0, e1));
                t.push_back(ms * 1000.0 / 48);
            }
            std::sort(t.begin(), t.end());
            std::printf("%-55s %6.2f us per 64 MB = %.2f TB/s\n", names[mode], t[1], 2.0 * bytes / (t[1] * 1e-6) / 1e12);
            CK(hipGraphExecDestroy(ge));
            CK(hipGraphDestroy(g));
        }
    return 0;
}
