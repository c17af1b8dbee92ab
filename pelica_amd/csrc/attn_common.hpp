// Shared device helpers of the gfx950 attention kernels: MFMA operand types,
// 64-lane reductions, exp2, f16 packing, LDS transpose reads.
//
// Operand layouts of v_mfma_f32_16x16x32_f16 (checked on the device):
//   A[16 x 32]: lane l holds row l%16, k = 8*(l/16) .. +7
//   B[32 x 16]: lane l holds column l%16, k = 8*(l/16) .. +7
//   C[16 x 16]: lane l holds column l%16, rows 4*(l/16) .. +3
// ds_read_b64_tr_b16 within each 16-lane group: lane i receives element i%4
// of the 4-element rows addressed by lanes 4r + i/4, r = 0..3.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace pelica {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef __fp16 fp16x4_lds __attribute__((__vector_size__(4 * sizeof(__fp16))));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

__device__ __forceinline__ float4v mfma16(const half8& a, const half8& b, const float4v& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// 2^x on the transcendental unit (v_exp_f32); 2^-inf = 0.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// max / sum over the four 16-lane groups (lanes l, l^16, l^32, l^48)
__device__ __forceinline__ float group4_max(float x) {
    auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

__device__ __forceinline__ float group4_sum(float x) {
    auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// Transposing LDS read: 4 f16 (see the layout note above).
__device__ __forceinline__ half4 lds_read_tr(const _Float16* p) {
    typedef __attribute__((address_space(3))) fp16x4_lds lds_t;
    fp16x4_lds r = __builtin_amdgcn_ds_read_tr16_b64_v4f16(
        (lds_t*)(__attribute__((address_space(3))) void*)(p));
    return __builtin_bit_cast(half4, r);
}

__device__ __forceinline__ half8 cat8(const half4& a, const half4& b) {
    return half8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}

__device__ __forceinline__ half8 load16(const void* p) {
    return __builtin_bit_cast(half8, *reinterpret_cast<const u32x4*>(p));
}

// Workgroup barrier for LDS data only: waits for this wave's own LDS
// operations (lgkmcnt(0)), not for vector-memory loads — __syncthreads()'s
// fence would also wait for every in-flight buffer_load ... lds (vmcnt(0)),
// draining a prefetch pipeline; kernels that stream tiles into LDS wait for
// those explicitly.  The empty asm keeps the compiler from moving memory
// accesses across the barrier.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt, expcnt untouched (max)
    __asm__ volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    __asm__ volatile("" ::: "memory");
}

// 16 bytes per lane from a buffer resource straight into LDS at
// lds_base + 16 * lane (buffer_load_dwordx4 ... lds, base in M0).  Callers
// wait for these loads (s_waitcnt vmcnt) before the barrier that publishes
// the tile.  `NT` sets the non-temporal bit (streamed data no one re-reads).
template <bool NT = false>
__device__ __forceinline__ void lds_dma16(__amdgpu_buffer_rsrc_t rsrc, uint32_t voffset, void* lds_base) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (__attribute__((address_space(3))) void*)lds_base, 16, voffset, 0,
                                             0, NT ? 2 : 0);
}

// The same load issued from inline asm, so the compiler does not track it.
// A tracked LDS DMA makes the compiler put s_waitcnt vmcnt(0) before any
// later LDS read it cannot prove disjoint (the transposing ds_read_b64_tr_b16
// reads always), which drains the whole prefetch ring — the next tiles'
// loads included — in every loop iteration.  For loads issued inside a tile
// loop: the kernel's own vmcnt waits and barriers order each tile's loads
// before its reads, and every load is waited for before the loop ends, so
// later LDS writes never race one.  Not for loads issued ahead of loads
// the compiler waits for (queries): vmcnt counts in issue order, and the
// compiler's count would not include these.  M0 is saved and restored.
template <bool NT = false>
__device__ __forceinline__ void lds_dma16_untracked(__amdgpu_buffer_rsrc_t rsrc, uint32_t voffset, void* lds_base) {
    const uint32_t m = __builtin_amdgcn_readfirstlane(
        (uint32_t)(size_t)(__attribute__((address_space(3))) char*)lds_base);
    uint32_t saved;
    if constexpr (NT)
        __asm__ volatile(
            "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\ts_nop 0\n\t"
            "buffer_load_dwordx4 %2, %3, 0 offen nt lds\n\ts_mov_b32 m0, %0"
            : "=&s"(saved)
            : "s"(m), "v"(voffset), "s"(rsrc));
    else
        __asm__ volatile(
            "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\ts_nop 0\n\t"
            "buffer_load_dwordx4 %2, %3, 0 offen lds\n\ts_mov_b32 m0, %0"
            : "=&s"(saved)
            : "s"(m), "v"(voffset), "s"(rsrc));
}

// Keys of sequence s: seq_len[s] clipped to kv_len (the bound every launch
// and workspace is sized from), or kv_len without a per-sequence table.
__device__ __forceinline__ int seq_keys(const int32_t* seq_len, int s, int kv_len) {
    return seq_len ? min(seq_len[s], kv_len) : kv_len;
}

// Split x into f16 hi + lo with x ~= hi + lo to ~2^-22 relative.
__device__ __forceinline__ void split_f16(float x, _Float16& hi, _Float16& lo) {
    hi = (_Float16)x;
    lo = (_Float16)(x - (float)hi);
}

}  // namespace pelica
