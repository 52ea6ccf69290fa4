// Device-side helpers for the gfx950 DVAttn kernels: vector types, per-dtype
// conversions and MFMA wrappers, wave-level shuffles and the query rotation.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "dv_common.h"

namespace dv {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(8))) _Float16 f16x8;
typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4;
typedef __attribute__((ext_vector_type(2))) uint32_t u32x2;
typedef __attribute__((ext_vector_type(4))) short i16x4;

#define DV_INF __builtin_inff()

// ---- per-dtype traits -------------------------------------------------------

template <int DT> struct Tr;

template <> struct Tr<kBF16> {
    using raw = uint16_t;
    static constexpr int kBytes = 2;
    __device__ static inline float tof(uint16_t v) { return __uint_as_float((uint32_t)v << 16); }
    __device__ static inline uint16_t fromf(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }
    // D = A(16x32) * B(32x16) + C; A/B hold 8 bf16 per lane (k = (lane/16)*8 + 0..7).
    __device__ static inline f32x4 mma(u32x4 a, u32x4 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                       __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
    }
};

template <> struct Tr<kF16> {
    using raw = uint16_t;
    static constexpr int kBytes = 2;
    __device__ static inline float tof(uint16_t v) { return (float)__builtin_bit_cast(_Float16, v); }
    __device__ static inline uint16_t fromf(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }
    __device__ static inline f32x4 mma(u32x4 a, u32x4 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                      __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
    }
};

template <> struct Tr<kF32> {
    using raw = float;
    static constexpr int kBytes = 4;
    __device__ static inline float tof(float v) { return v; }
    __device__ static inline float fromf(float f) { return f; }
    // D = A(16x4) * B(4x16) + C; one fp32 per lane (k = lane/16).
    __device__ static inline f32x4 mma1(float a, float b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
    }
};

template <int DT>
__device__ inline uint32_t pack2(float lo, float hi) {
    return (uint32_t)Tr<DT>::fromf(lo) | ((uint32_t)Tr<DT>::fromf(hi) << 16);
}

// A VALU read of an MFMA result needs software wait states after the MFMA that
// wrote it (11-19 for the 8- and 16-pass XDL ops).  The compiler provides them
// inside a block but was seen to miss them where a branch leads straight to a
// loop-carried copy of the accumulators (the copy read stale elements).  This
// barrier depends on all eight accumulators, so it follows the last MFMA that
// writes them, and puts 24 wait states before any later instruction.
__device__ inline void mfma_settle(f32x4 (&o)[8]) {
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7"
                 : "+v"(o[0]), "+v"(o[1]), "+v"(o[2]), "+v"(o[3]), "+v"(o[4]), "+v"(o[5]), "+v"(o[6]), "+v"(o[7]));
}

// ---- memory helpers ---------------------------------------------------------

// 16-byte loads from global memory (address space 1, so the compiler emits
// global_load_dwordx4 rather than flat loads).
typedef __attribute__((address_space(1))) const u32x4 gu32x4;
typedef __attribute__((address_space(1))) const f32x4 gf32x4;
__device__ inline u32x4 ld16(const void* p) { return *(gu32x4*)(p); }
__device__ inline f32x4 ld16f(const void* p) { return *(gf32x4*)(p); }

// Transposed LDS read (gfx950 ds_read_b64_tr_b16).  Within each 16-lane block,
// result lane i, element j = the 16-bit word (i % 4) at the address supplied by
// block lane (i / 4 + 4 * j).
__device__ inline u32x2 lds_read_tr16(const unsigned char* p) {
    typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
    i16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p));
    return __builtin_bit_cast(u32x2, v);
}

__device__ inline void compiler_fence() { asm volatile("" ::: "memory"); }

// ---- direct-to-LDS loads ------------------------------------------------------

__device__ inline uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)((__attribute__((address_space(3))) const void*)(p));
}

// 16 bytes per lane from global memory straight into LDS at m0 + 16 * lane
// (global_load_lds_dwordx4).  lds_base must be wave-uniform.  The compiler does
// not track these loads: completion is awaited with wait_vmcnt.  An SALU write of
// m0 needs one wait state before an LDS-DMA instruction reads it (the compiler's
// hazard recognizer inserts the same s_nop for its own global_load_lds); without
// it the first lanes of the load can use the previous m0.
__device__ inline void dma16(const void* gptr, uint32_t lds_base) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(gptr), "s"(lds_base)
                 : "memory", "m0");
}

// Wait until at most N vector-memory operations of this wave are outstanding.
template <int N>
__device__ inline void wait_vmcnt() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Wait until this wave's LDS operations are complete.
__device__ inline void lds_wait() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// ---- wave-level helpers -----------------------------------------------------

__device__ inline float shfl_xor_f(float v, int mask) { return __shfl_xor(v, mask, kWave); }
__device__ inline int shfl_i(int v, int src) { return __shfl(v, src, kWave); }
__device__ inline uint64_t ballot(bool b) { return __ballot(b); }

// ---- query rotation ---------------------------------------------------------
// Rotated value of the run of N consecutive dims [d0, d0+N) of one query row,
// restating src/rope.cuh:18-51: for e < R/2: x[e]*c[e] - x[e+R/2]*s[e];
// for R/2 <= e < R: x[e]*c[e-R/2] + x[e-R/2]*s[e-R/2]; e >= R copied.  c/s are
// the first R/2 entries of the cos/sin row.  Products and the sum are separate
// fp32 roundings (no FMA contraction); the result is rounded to the storage type.
template <int DT, int N>
__device__ inline void rotate_run(const typename Tr<DT>::raw* __restrict__ qrow,
                                  const float* __restrict__ crow, const float* __restrict__ srow,
                                  int R, int d0, typename Tr<DT>::raw (&res)[N]) {
#pragma clang fp contract(off)
    using raw = typename Tr<DT>::raw;
    const int half = R >> 1;
    if (d0 >= R) {
#pragma unroll
        for (int e = 0; e < N; ++e) res[e] = qrow[d0 + e];
        return;
    }
    if (half % N == 0) {
        // the whole run sits in one half of the rotary block
        const bool first = d0 < half;
        const int pd = first ? d0 + half : d0 - half;
        const int ci = first ? d0 : d0 - half;
#pragma unroll
        for (int e = 0; e < N; ++e) {
            const float x = Tr<DT>::tof(qrow[d0 + e]);
            const float xp = Tr<DT>::tof(qrow[pd + e]);
            const float c = crow[ci + e];
            const float s = srow[ci + e];
            float y;
            if (first) {
                const float a = x * c;
                const float b = xp * s;
                y = a - b;
            } else {
                const float a = x * c;
                const float b = xp * s;
                y = a + b;
            }
            res[e] = Tr<DT>::fromf(y);
        }
        return;
    }
#pragma unroll 1
    for (int e = 0; e < N; ++e) {
        const int d = d0 + e;
        if (d >= R) {
            res[e] = qrow[d];
        } else if (d < half) {
            const float a = Tr<DT>::tof(qrow[d]) * crow[d];
            const float b = Tr<DT>::tof(qrow[d + half]) * srow[d];
            res[e] = Tr<DT>::fromf(a - b);
        } else {
            const float a = Tr<DT>::tof(qrow[d]) * crow[d - half];
            const float b = Tr<DT>::tof(qrow[d - half]) * srow[d - half];
            res[e] = Tr<DT>::fromf(a + b);
        }
    }
}

}  // namespace dv
