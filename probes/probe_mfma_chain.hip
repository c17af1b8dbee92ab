// Dependent-MFMA latency: v_mfma_f32_32x32x16_f16 on 1, 2 or 4 independent
// accumulator chains (8 MFMAs per trip, round robin), one wave per SIMD;
// shader cycles per MFMA of wave 0.  One chain at the pipe's rate means a
// dependent MFMA (srcC = the previous result) issues right behind it.
#include <hip/hip_runtime.h>

#include <cstdio>
typedef float f16v __attribute__((ext_vector_type(16)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
// NCH independent accumulator chains, 8 MFMAs per trip in round-robin order; one wave per SIMD
template <int NCH>
__global__ void k(float* out, unsigned long long* st, float s) {
    h8 a, b;
    for (int i = 0; i < 8; ++i) { a[i] = (_Float16)(s + threadIdx.x * 0.01f + i); b[i] = (_Float16)(s - i); }
    f16v c0 = {}, c1 = {}, c2 = {}, c3 = {};
    unsigned long long t0 = __builtin_amdgcn_s_memtime();
#pragma unroll 1
    for (int it = 0; it < 2000; ++it) {
        if (NCH == 1) asm volatile("v_mfma_f32_32x32x16_f16 %0, %1, %2, %0\n v_mfma_f32_32x32x16_f16 %0, %1, %2, %0\n v_mfma_f32_32x32x16_f16 %0, %1, %2, %0\n v_mfma_f32_32x32x16_f16 %0, %1, %2, %0\n v_mfma_f32_32x32x16_f16 %0, %1, %2, %0\n v_mfma_f32_32x32x16_f16 %0, %1, %2, %0\n v_mfma_f32_32x32x16_f16 %0, %1, %2, %0\n v_mfma_f32_32x32x16_f16 %0, %1, %2, %0\n" : "+v"(c0) : "v"(a), "v"(b));
        if (NCH == 2) asm volatile("v_mfma_f32_32x32x16_f16 %0, %2, %3, %0\n v_mfma_f32_32x32x16_f16 %1, %2, %3, %1\n v_mfma_f32_32x32x16_f16 %0, %2, %3, %0\n v_mfma_f32_32x32x16_f16 %1, %2, %3, %1\n v_mfma_f32_32x32x16_f16 %0, %2, %3, %0\n v_mfma_f32_32x32x16_f16 %1, %2, %3, %1\n v_mfma_f32_32x32x16_f16 %0, %2, %3, %0\n v_mfma_f32_32x32x16_f16 %1, %2, %3, %1\n" : "+v"(c0), "+v"(c1) : "v"(a), "v"(b));
        if (NCH == 4) asm volatile("v_mfma_f32_32x32x16_f16 %0, %4, %5, %0\n v_mfma_f32_32x32x16_f16 %1, %4, %5, %1\n v_mfma_f32_32x32x16_f16 %2, %4, %5, %2\n v_mfma_f32_32x32x16_f16 %3, %4, %5, %3\n v_mfma_f32_32x32x16_f16 %0, %4, %5, %0\n v_mfma_f32_32x32x16_f16 %1, %4, %5, %1\n v_mfma_f32_32x32x16_f16 %2, %4, %5, %2\n v_mfma_f32_32x32x16_f16 %3, %4, %5, %3\n" : "+v"(c0), "+v"(c1), "+v"(c2), "+v"(c3) : "v"(a), "v"(b));
    }
    unsigned long long t1 = __builtin_amdgcn_s_memtime();
    float r = 0; for (int i = 0; i < 16; ++i) r += c0[i] + c1[i] + c2[i] + c3[i];
    out[blockIdx.x * blockDim.x + threadIdx.x] = r;
    if (threadIdx.x == 0) st[blockIdx.x] = t1 - t0;
}
template <int N> void run(float* out, unsigned long long* st) {
    hipLaunchKernelGGL(k<N>, dim3(256), dim3(256), 0, 0, out, st, 0.f);
    (void)hipDeviceSynchronize();
    unsigned long long h[256]; (void)hipMemcpy(h, st, sizeof h, hipMemcpyDeviceToHost);
    double c = 0; for (int i = 0; i < 256; ++i) c += h[i];
    std::printf("%d chain(s): %.2f cycles per MFMA\n", N, c / 256 / 16000);
}
int main() { float* out; unsigned long long* st; (void)hipMalloc(&out, 256 * 256 * 4); (void)hipMalloc(&st, 256 * 8); run<1>(out, st); run<2>(out, st); run<4>(out, st); return 0; }
