// MFMA / vector-ALU co-execution within one wave alone on its SIMD (256
// workgroups of 4 waves): per loop trip the wave issues 4
// v_mfma_f32_32x32x16_f16 (independent accumulators, in arch VGPRs or in
// AGPRs) interleaved with 32 vector ops of the prefill softmax's kind (fma,
// exp, f16 pack, dot2); shader cycles (s_memtime) per trip, against the
// MFMAs alone and the vector ops alone.
#include <hip/hip_runtime.h>
#include <cstdio>
typedef float f16v __attribute__((ext_vector_type(16)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
#define MF_V(acc) "v_mfma_f32_32x32x16_f16 " acc ", %[a], %[b], " acc "\n"
#define VALU8 "v_fma_f32 %[x0], %[x0], %[x1], %[x2]\n v_fma_f32 %[x1], %[x1], %[x2], %[x3]\n v_exp_f32 %[x2], %[x2]\n v_exp_f32 %[x3], %[x3]\n v_fma_f32 %[x4], %[x4], %[x5], %[x6]\n v_fma_f32 %[x5], %[x5], %[x6], %[x7]\n v_cvt_pk_f16_f32 %[x6], %[x6], %[x7]\n v_dot2c_f32_f16 %[x7], %[x6], %[x6]\n"
template <int MODE, int NV>  // MODE 0: MFMA only (VGPR acc), 1: MFMA VGPR + VALU, 2: MFMA AGPR + VALU, 3: VALU only, 4: MFMA only AGPR
__global__ __launch_bounds__(256) void bench(float* out, unsigned long long* cyc, float s) {
    h8 a, b;
    for (int i = 0; i < 8; ++i) { a[i] = (_Float16)(s + threadIdx.x + i); b[i] = (_Float16)(s - i); }
    f16v c0 = {}, c1 = {}, c2 = {}, c3 = {};
    float x0 = s + threadIdx.x, x1 = x0 + 1, x2 = x0 + 2, x3 = x0 + 3, x4 = x0 + 4, x5 = x0 + 5, x6 = x0 + 6, x7 = x0 + 7;
    unsigned long long t0 = __builtin_amdgcn_s_memtime();
    for (int it = 0; it < 512; ++it) {
#define BODY(MF) \
        asm volatile(MF("%[c0]") VALU8 MF("%[c1]") VALU8 MF("%[c2]") VALU8 MF("%[c3]") VALU8 \
            : [c0] "+" CC(c0), [c1] "+" CC(c1), [c2] "+" CC(c2), [c3] "+" CC(c3), [x0] "+v"(x0), [x1] "+v"(x1), [x2] "+v"(x2), [x3] "+v"(x3), [x4] "+v"(x4), [x5] "+v"(x5), [x6] "+v"(x6), [x7] "+v"(x7) : [a] "v"(a), [b] "v"(b));
        if constexpr (MODE == 0 || MODE == 4) {
            if constexpr (MODE == 0) asm volatile(MF_V("%[c0]") MF_V("%[c1]") MF_V("%[c2]") MF_V("%[c3]") : [c0] "+v"(c0), [c1] "+v"(c1), [c2] "+v"(c2), [c3] "+v"(c3) : [a] "v"(a), [b] "v"(b));
            else asm volatile(MF_V("%[c0]") MF_V("%[c1]") MF_V("%[c2]") MF_V("%[c3]") : [c0] "+a"(c0), [c1] "+a"(c1), [c2] "+a"(c2), [c3] "+a"(c3) : [a] "v"(a), [b] "v"(b));
        } else if constexpr (MODE == 1) {
#define CC(x) "v"(x)
            BODY(MF_V)
#undef CC
        } else if constexpr (MODE == 2) {
#define CC(x) "a"(x)
            BODY(MF_V)
#undef CC
        } else {
            asm volatile(VALU8 VALU8 VALU8 VALU8 : [x0] "+v"(x0), [x1] "+v"(x1), [x2] "+v"(x2), [x3] "+v"(x3), [x4] "+v"(x4), [x5] "+v"(x5), [x6] "+v"(x6), [x7] "+v"(x7));
        }
    }
    unsigned long long t1 = __builtin_amdgcn_s_memtime();
    float r = x0 + x1 + x2 + x3 + x4 + x5 + x6 + x7;
    for (int i = 0; i < 16; ++i) r += c0[i] + c1[i] + c2[i] + c3[i];
    out[blockIdx.x * 256 + threadIdx.x] = r;
    if (threadIdx.x == 0) cyc[blockIdx.x] = t1 - t0;
}
template <int MODE> void run(const char* name, float* out, unsigned long long* cyc) {
    hipLaunchKernelGGL((bench<MODE, 8>), dim3(256), dim3(256), 0, 0, out, cyc, 0.f);
    hipLaunchKernelGGL((bench<MODE, 8>), dim3(256), dim3(256), 0, 0, out, cyc, 0.f);
    (void)hipDeviceSynchronize();
    unsigned long long h[256];
    (void)hipMemcpy(h, cyc, sizeof h, hipMemcpyDeviceToHost);
    unsigned long long s = 0; for (int i = 0; i < 256; ++i) s += h[i];
    printf("%-28s %.1f cycles per trip (4 MFMA + 32 vector ops, one wave per SIMD)\n", name, (double)s / 256 / 512);
}
int main() {
    float* out; unsigned long long* cyc;
    (void)hipMalloc(&out, 256 * 512 * 4); (void)hipMalloc(&cyc, 256 * 8);
    run<0>("mfma only, vgpr acc", out, cyc); run<4>("mfma only, agpr acc", out, cyc); run<3>("valu only", out, cyc);
    run<1>("mfma vgpr acc + valu", out, cyc); run<2>("mfma agpr acc + valu", out, cyc);
    return 0;
}
