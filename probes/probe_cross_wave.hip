// Cross-wave co-execution: two waves on one SIMD, one issuing only MFMAs
// (v_mfma_f32_32x32x16_f16, 4 accumulator chains) and the other only
// vector ops of the prefill softmax's kind; against each alone (one wave per
// SIMD).  Kernel time (HIP events) and shader cycles of each wave.
#include <hip/hip_runtime.h>

#include <cstdio>
typedef float f16v __attribute__((ext_vector_type(16)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
#define VALU8 "v_fma_f32 %0, %0, %1, %2\n v_fma_f32 %1, %1, %2, %3\n v_exp_f32 %2, %2\n v_exp_f32 %3, %3\n v_fma_f32 %4, %4, %5, %6\n v_fma_f32 %5, %5, %6, %7\n v_cvt_pk_f16_f32 %6, %6, %7\n v_dot2c_f32_f16 %7, %6, %6\n"
// ROLE per wave: 0 = MFMA loop (4 chains, 2000 trips x 8), 1 = VALU loop (2000 trips x 64 ops), 2 = idle
template <int CFG>  // CFG 0: 4 waves MFMA; 1: 4 waves VALU; 2: 8 waves, waves 0-3 MFMA, 4-7 VALU; 3: 8 waves, 0-3 VALU, 4-7 MFMA
__global__ void k(float* out, unsigned long long* st, float s) {
    const int wave = threadIdx.x >> 6;
    int role = CFG == 0 ? 0 : CFG == 1 ? 1 : CFG == 2 ? (wave < 4 ? 0 : 1) : (wave < 4 ? 1 : 0);
    role = __builtin_amdgcn_readfirstlane(role);
    h8 a, b;
    for (int i = 0; i < 8; ++i) { a[i] = (_Float16)(s + threadIdx.x * 0.01f + i); b[i] = (_Float16)(s - i); }
    f16v c0 = {}, c1 = {}, c2 = {}, c3 = {};
    float x0 = s + threadIdx.x, x1 = x0 + 1, x2 = x0 + 2, x3 = x0 + 3, x4 = x0 + 4, x5 = x0 + 5, x6 = x0 + 6, x7 = x0 + 7;
    unsigned long long t0 = __builtin_amdgcn_s_memtime();
    if (role == 0) {
#pragma unroll 1
        for (int it = 0; it < 2000; ++it)
            asm volatile("v_mfma_f32_32x32x16_f16 %0, %4, %5, %0\n v_mfma_f32_32x32x16_f16 %1, %4, %5, %1\n v_mfma_f32_32x32x16_f16 %2, %4, %5, %2\n v_mfma_f32_32x32x16_f16 %3, %4, %5, %3\n v_mfma_f32_32x32x16_f16 %0, %4, %5, %0\n v_mfma_f32_32x32x16_f16 %1, %4, %5, %1\n v_mfma_f32_32x32x16_f16 %2, %4, %5, %2\n v_mfma_f32_32x32x16_f16 %3, %4, %5, %3\n" : "+v"(c0), "+v"(c1), "+v"(c2), "+v"(c3) : "v"(a), "v"(b));
    } else {
#pragma unroll 1
        for (int it = 0; it < 2000; ++it)
            asm volatile(VALU8 VALU8 VALU8 VALU8 VALU8 VALU8 VALU8 VALU8 : "+v"(x0), "+v"(x1), "+v"(x2), "+v"(x3), "+v"(x4), "+v"(x5), "+v"(x6), "+v"(x7));
    }
    unsigned long long t1 = __builtin_amdgcn_s_memtime();
    float r = x0 + x1 + x2 + x3 + x4 + x5 + x6 + x7; for (int i = 0; i < 16; ++i) r += c0[i] + c1[i] + c2[i] + c3[i];
    out[blockIdx.x * blockDim.x + threadIdx.x] = r;
    if ((threadIdx.x & 63) == 0) st[blockIdx.x * 8 + wave] = t1 - t0;
}
template <int C> void run(const char* name, int W, float* out, unsigned long long* st) {
    hipEvent_t e0, e1; (void)hipEventCreate(&e0); (void)hipEventCreate(&e1);
    hipLaunchKernelGGL(k<C>, dim3(256), dim3(64 * W), 0, 0, out, st, 0.f);
    (void)hipEventRecord(e0, 0);
    hipLaunchKernelGGL(k<C>, dim3(256), dim3(64 * W), 0, 0, out, st, 0.f);
    (void)hipEventRecord(e1, 0); (void)hipEventSynchronize(e1);
    float ms; (void)hipEventElapsedTime(&ms, e0, e1);
    unsigned long long h[256 * 8]; (void)hipMemcpy(h, st, sizeof h, hipMemcpyDeviceToHost);
    double lo = 0, hi = 0; for (int i = 0; i < 256; ++i) { for (int w = 0; w < 4; ++w) lo += h[i * 8 + w]; if (W == 8) for (int w = 4; w < 8; ++w) hi += h[i * 8 + w]; }
    std::printf("%-40s kernel %.1f us; waves 0-3 %.0f cycles, waves 4-7 %.0f cycles\n", name, ms * 1000, lo / 1024, W == 8 ? hi / 1024 : 0.0);
}
int main() { float* out; unsigned long long* st; (void)hipMalloc(&out, 256 * 512 * 4); (void)hipMalloc(&st, 256 * 8 * 8);
  run<0>("MFMA waves alone (1/SIMD)", 4, out, st); run<1>("VALU waves alone (1/SIMD)", 4, out, st);
  run<2>("MFMA (older) + VALU (younger) per SIMD", 8, out, st); run<3>("VALU (older) + MFMA (younger) per SIMD", 8, out, st); return 0; }
