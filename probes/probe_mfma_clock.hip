// What one v_mfma_f32_32x32x16_f16 costs, what s_memtime counts, and how two
// waves on one SIMD share the matrix core when both issue MFMAs back to
// back.  256 workgroups of W waves (W = 4: one wave per SIMD; W = 8: two);
// each wave runs 2000 trips of 8 MFMAs on 4 independent accumulators and
// stamps s_memtime and s_memrealtime (100 MHz) around them, with its
// hardware id; the kernel is timed with HIP events.
#include <hip/hip_runtime.h>

#include <cstdio>

typedef float f16v __attribute__((ext_vector_type(16)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));

__global__ void mfma_loop(float* out, unsigned long long* st, float s) {
    h8 a, b;
    for (int i = 0; i < 8; ++i) {
        a[i] = (_Float16)(s + threadIdx.x * 0.01f + i);
        b[i] = (_Float16)(s - i);
    }
    f16v c0 = {}, c1 = {}, c2 = {}, c3 = {};
    const unsigned long long t0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
#pragma unroll 1
    for (int it = 0; it < 2000; ++it) {
        asm volatile(
            "v_mfma_f32_32x32x16_f16 %0, %4, %5, %0\n v_mfma_f32_32x32x16_f16 %1, %4, %5, %1\n"
            "v_mfma_f32_32x32x16_f16 %2, %4, %5, %2\n v_mfma_f32_32x32x16_f16 %3, %4, %5, %3\n"
            "v_mfma_f32_32x32x16_f16 %0, %4, %5, %0\n v_mfma_f32_32x32x16_f16 %1, %4, %5, %1\n"
            "v_mfma_f32_32x32x16_f16 %2, %4, %5, %2\n v_mfma_f32_32x32x16_f16 %3, %4, %5, %3\n"
            : "+v"(c0), "+v"(c1), "+v"(c2), "+v"(c3)
            : "v"(a), "v"(b));
    }
    const unsigned long long t1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
    float r = 0;
    for (int i = 0; i < 16; ++i) r += c0[i] + c1[i] + c2[i] + c3[i];
    out[blockIdx.x * blockDim.x + threadIdx.x] = r;
    if ((threadIdx.x & 63) == 0) {
        const int w = blockIdx.x * (blockDim.x / 64) + threadIdx.x / 64;
        st[4 * w] = t1 - t0;
        st[4 * w + 1] = r1 - r0;
        st[4 * w + 2] = r0;
        st[4 * w + 3] = __builtin_amdgcn_s_getreg((4 << 0) | (0 << 6) | (31 << 11));  // HW_ID
    }
}

int main() {
    float* out;
    unsigned long long* st;
    if (hipMalloc(&out, 256 * 512 * 4) != hipSuccess || hipMalloc(&st, 256 * 8 * 32) != hipSuccess) return 1;
    static unsigned long long h[256 * 32];
    for (int W : {4, 8}) {
        hipEvent_t e0, e1;
        (void)hipEventCreate(&e0);
        (void)hipEventCreate(&e1);
        hipLaunchKernelGGL(mfma_loop, dim3(256), dim3(64 * W), 0, 0, out, st, 0.f);
        (void)hipEventRecord(e0, 0);
        hipLaunchKernelGGL(mfma_loop, dim3(256), dim3(64 * W), 0, 0, out, st, 0.f);
        (void)hipEventRecord(e1, 0);
        if (hipEventSynchronize(e1) != hipSuccess) return 1;
        float ms;
        (void)hipEventElapsedTime(&ms, e0, e1);
        (void)hipMemcpy(h, st, sizeof(unsigned long long) * 4 * 256 * W, hipMemcpyDeviceToHost);
        double cyc = 0, rt = 0;
        for (int i = 0; i < 256 * W; ++i) {
            cyc += h[4 * i];
            rt += h[4 * i + 1];
        }
        cyc /= 256 * W;
        rt /= 256 * W;
        for (int w = 0; w < W; ++w)
            std::printf("  workgroup 0 wave %d: starts %+lld x 10 ns after wave 0, runs %llu x 10 ns, HW_ID 0x%llx\n", w,
                        (long long)(h[4 * w + 2] - h[2]), h[4 * w + 1], h[4 * w + 3]);
        const double flops = 256.0 * W * 2000 * 8 * 32768;
        std::printf("%d wave(s) per SIMD: per wave %.0f s_memtime cycles in %.1f us -> %.2f GHz, %.2f cycles per MFMA "
                    "of the wave; kernel %.3f ms = %.0f TFLOP/s\n",
                    W / 4, cyc, rt / 100.0, cyc / (rt * 10.0), cyc / 16000.0, ms, flops / (ms * 1e-3) / 1e12);
    }
    return 0;
}
