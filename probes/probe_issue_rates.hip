// Issue cost of the vector instructions of the prefill softmax for one wave
// alone on its SIMD (256 workgroups of 4 waves): shader cycles (s_memtime)
// per wave instruction, 8 independent chains, 256 x 64 instructions per
// wave.  exp_f32 vs exp_f16 (plain and SDWA halves), fma_f32, fma_mix (f32
// in, f16 half out), cvt_pk_f16_f32.
#include <hip/hip_runtime.h>
#include <cstdio>
#define REP8(x) x x x x x x x x
template <int K>
__global__ __launch_bounds__(256) void bench(float* out, unsigned long long* cyc, float a) {
    float r0 = a + threadIdx.x, r1 = r0 + 1, r2 = r0 + 2, r3 = r0 + 3, r4 = r0 + 4, r5 = r0 + 5, r6 = r0 + 6, r7 = r0 + 7;
    unsigned long long t0 = __builtin_amdgcn_s_memtime();
    for (int it = 0; it < 256; ++it) {
        if (K == 0) asm volatile(REP8("v_exp_f32 %0, %0\n v_exp_f32 %1, %1\n v_exp_f32 %2, %2\n v_exp_f32 %3, %3\n v_exp_f32 %4, %4\n v_exp_f32 %5, %5\n v_exp_f32 %6, %6\n v_exp_f32 %7, %7\n") : "+v"(r0), "+v"(r1), "+v"(r2), "+v"(r3), "+v"(r4), "+v"(r5), "+v"(r6), "+v"(r7));
        if (K == 1) asm volatile(REP8("v_exp_f16_sdwa %0, %0 dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:WORD_1\n v_exp_f16_sdwa %1, %1 dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:WORD_1\n v_exp_f16_sdwa %2, %2 dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:WORD_1\n v_exp_f16_sdwa %3, %3 dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:WORD_1\n v_exp_f16_sdwa %4, %4 dst_sel:WORD_0 dst_unused:UNUSED_PRESERVE src0_sel:WORD_0\n v_exp_f16_sdwa %5, %5 dst_sel:WORD_0 dst_unused:UNUSED_PRESERVE src0_sel:WORD_0\n v_exp_f16_sdwa %6, %6 dst_sel:WORD_0 dst_unused:UNUSED_PRESERVE src0_sel:WORD_0\n v_exp_f16_sdwa %7, %7 dst_sel:WORD_0 dst_unused:UNUSED_PRESERVE src0_sel:WORD_0\n") : "+v"(r0), "+v"(r1), "+v"(r2), "+v"(r3), "+v"(r4), "+v"(r5), "+v"(r6), "+v"(r7));
        if (K == 2) asm volatile(REP8("v_exp_f16 %0, %0\n v_exp_f16 %1, %1\n v_exp_f16 %2, %2\n v_exp_f16 %3, %3\n v_exp_f16 %4, %4\n v_exp_f16 %5, %5\n v_exp_f16 %6, %6\n v_exp_f16 %7, %7\n") : "+v"(r0), "+v"(r1), "+v"(r2), "+v"(r3), "+v"(r4), "+v"(r5), "+v"(r6), "+v"(r7));
        if (K == 3) asm volatile(REP8("v_fma_f32 %0, %0, %1, %2\n v_fma_f32 %1, %1, %2, %3\n v_fma_f32 %2, %2, %3, %4\n v_fma_f32 %3, %3, %4, %5\n v_fma_f32 %4, %4, %5, %6\n v_fma_f32 %5, %5, %6, %7\n v_fma_f32 %6, %6, %7, %0\n v_fma_f32 %7, %7, %0, %1\n") : "+v"(r0), "+v"(r1), "+v"(r2), "+v"(r3), "+v"(r4), "+v"(r5), "+v"(r6), "+v"(r7));
        if (K == 4) asm volatile(REP8("v_fma_mixlo_f16 %0, %1, %2, %3 op_sel_hi:[0,0,0]\n v_fma_mixhi_f16 %1, %2, %3, %4 op_sel_hi:[0,0,0]\n v_fma_mixlo_f16 %2, %3, %4, %5 op_sel_hi:[0,0,0]\n v_fma_mixhi_f16 %3, %4, %5, %6 op_sel_hi:[0,0,0]\n v_fma_mixlo_f16 %4, %5, %6, %7 op_sel_hi:[0,0,0]\n v_fma_mixhi_f16 %5, %6, %7, %0 op_sel_hi:[0,0,0]\n v_fma_mixlo_f16 %6, %7, %0, %1 op_sel_hi:[0,0,0]\n v_fma_mixhi_f16 %7, %0, %1, %2 op_sel_hi:[0,0,0]\n") : "+v"(r0), "+v"(r1), "+v"(r2), "+v"(r3), "+v"(r4), "+v"(r5), "+v"(r6), "+v"(r7));
        if (K == 5) asm volatile(REP8("v_cvt_pk_f16_f32 %0, %1, %2\n v_cvt_pk_f16_f32 %1, %2, %3\n v_cvt_pk_f16_f32 %2, %3, %4\n v_cvt_pk_f16_f32 %3, %4, %5\n v_cvt_pk_f16_f32 %4, %5, %6\n v_cvt_pk_f16_f32 %5, %6, %7\n v_cvt_pk_f16_f32 %6, %7, %0\n v_cvt_pk_f16_f32 %7, %0, %1\n") : "+v"(r0), "+v"(r1), "+v"(r2), "+v"(r3), "+v"(r4), "+v"(r5), "+v"(r6), "+v"(r7));
    }
    unsigned long long t1 = __builtin_amdgcn_s_memtime();
    out[blockIdx.x * 256 + threadIdx.x] = r0 + r1 + r2 + r3 + r4 + r5 + r6 + r7;
    if (threadIdx.x == 0) cyc[blockIdx.x] = t1 - t0;
}
template <int K> void run(const char* name, float* out, unsigned long long* cyc) {
    hipLaunchKernelGGL(bench<K>, dim3(256), dim3(256), 0, 0, out, cyc, 0.f);
    hipLaunchKernelGGL(bench<K>, dim3(256), dim3(256), 0, 0, out, cyc, 0.f);
    (void)hipDeviceSynchronize();
    unsigned long long h[256];
    (void)hipMemcpy(h, cyc, sizeof h, hipMemcpyDeviceToHost);
    unsigned long long s = 0; for (int i = 0; i < 256; ++i) s += h[i];
    // wave 0 of each workgroup: 256 x 64 instructions
    printf("%-16s %.2f shader cycles per wave instruction (one wave per SIMD)\n", name, (double)s / 256 / (256 * 64));
}
int main() {
    float* out; unsigned long long* cyc;
    (void)hipMalloc(&out, 256 * 512 * 4); (void)hipMalloc(&cyc, 256 * 8);
    run<0>("exp_f32", out, cyc); run<1>("exp_f16_sdwa", out, cyc); run<2>("exp_f16", out, cyc);
    run<3>("fma_f32", out, cyc); run<4>("fma_mix", out, cyc); run<5>("cvt_pk_f16_f32", out, cyc);
    return 0;
}
