// LDS read throughput on gfx950 by instruction: ds_read_b128 (16 B a lane,
// conflict-free), ds_read_b64, and ds_read_b64_tr_b16 at the prefill's V^T
// operand pattern (XOR-swizzled rows); one workgroup of W waves per CU
// (256 workgroups), 16 reads in flight per wave, shader cycles of wave 0.
#include <hip/hip_runtime.h>

#include <cstdio>
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef __fp16 fp16x4_lds __attribute__((__vector_size__(4 * sizeof(__fp16))));
typedef unsigned u4 __attribute__((ext_vector_type(4)));
// MODE 0: ds_read_b128, lane l reads 16 B at l*16 (1 KB per instruction);
// MODE 1: ds_read_b64_tr_b16 at the prefill's V pattern; MODE 2: ds_read_b64
template <int MODE>
__global__ void k(float* out, unsigned long long* st) {
    __shared__ __attribute__((aligned(16))) char lds[65536];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int i = threadIdx.x; i < 65536 / 16; i += blockDim.x) ((u4*)lds)[i] = u4{(unsigned)i, 1, 2, 3};
    __syncthreads();
    u4 acc = {0, 0, 0, 0};
    unsigned long long t0 = __builtin_amdgcn_s_memtime();
#pragma unroll 1
    for (int it = 0; it < 1000; ++it) {
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int base = ((it * 16 + j) & 31) * 2048;
            if (MODE == 0) acc ^= *(const u4*)(lds + base + lane * 16);
            if (MODE == 2) { auto v = *(const unsigned long long*)(lds + base + lane * 8); acc.x ^= (unsigned)v; acc.y ^= (unsigned)(v >> 32); }
            if (MODE == 1) {
                // lanes of 16-lane group G: key 4*(G&1)... same shape as the prefill: 4 rows of 16 B, rows 128 B apart
                const int G = lane >> 4, r4 = (lane & 15) >> 2, q4 = lane & 3;
                const int key = 4 * (G >> 1) + r4, dim = 16 * (G & 1) + 4 * q4;
                const int p = dim >> 3;
                const int off = base + key * 128 + ((p ^ ((key & 3) << 1)) << 4) + ((dim & 7) << 1);
                typedef __attribute__((address_space(3))) fp16x4_lds lds_t;
                fp16x4_lds r = __builtin_amdgcn_ds_read_tr16_b64_v4f16((lds_t*)(__attribute__((address_space(3))) void*)(lds + off));
                auto v = __builtin_bit_cast(unsigned long long, r); acc.x ^= (unsigned)v; acc.y ^= (unsigned)(v >> 32);
            }
        }
    }
    unsigned long long t1 = __builtin_amdgcn_s_memtime();
    out[blockIdx.x * blockDim.x + threadIdx.x] = (float)(acc.x ^ acc.y ^ acc.z ^ acc.w);
    if (threadIdx.x == 0) st[blockIdx.x] = t1 - t0;
}
template <int M> void run(const char* name, int W, float* out, unsigned long long* st) {
    hipLaunchKernelGGL(k<M>, dim3(256), dim3(64 * W), 0, 0, out, st);
    (void)hipDeviceSynchronize();
    unsigned long long h[256]; (void)hipMemcpy(h, st, sizeof h, hipMemcpyDeviceToHost);
    double c = 0; for (int i = 0; i < 256; ++i) c += h[i]; c /= 256;
    const double bytes = (M == 0 ? 1024.0 : 512.0) * 16000 * W;
    std::printf("%-22s %d waves/CU: %.2f cycles per wave instruction, %.1f B/cycle per CU\n", name, W, c / 16000, bytes / c);
}
int main() { float* out; unsigned long long* st; (void)hipMalloc(&out, 256 * 1024 * 4); (void)hipMalloc(&st, 256 * 8);
  for (int W : {4, 8}) { run<0>("ds_read_b128", W, out, st); run<2>("ds_read_b64", W, out, st); run<1>("ds_read_b64_tr_b16", W, out, st); } return 0; }
