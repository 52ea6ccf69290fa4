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

typedef __attribute__((ext_vector_type(2))) float f32x2;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;
typedef __attribute__((ext_vector_type(2))) _Float16 f16x2;

// Two floats rounded to the 16-bit storage type (round to nearest even), lo in
// bits 0-15: one v_cvt_pk_bf16_f32 / v_cvt_pk_f16_f32.
template <int DT>
__device__ inline uint32_t pack2(float lo, float hi) {
    static_assert(DT == kBF16 || DT == kF16, "16-bit storage types only");
    const f32x2 v = {lo, hi};
    if constexpr (DT == kBF16) return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
    else return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2));
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
// Non-temporal (streaming) 16-byte load, for K/V rows read once per call.
__device__ inline f32x4 ld16f_nt(const void* p) { return __builtin_nontemporal_load((gf32x4*)(p)); }

// Transposed LDS read (gfx950 ds_read_b64_tr_b16).  Within each 16-lane block,
// result lane i, element j = the 16-bit word (i % 4) at the address supplied by
// block lane (i / 4 + 4 * j).
__device__ inline u32x2 lds_read_tr16(const unsigned char* p) {
    typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
    i16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p));
    return __builtin_bit_cast(u32x2, v);
}

// The same at an LDS byte address (lets the compiler fold constant offsets into
// the instruction).
__device__ inline u32x2 lds_read_tr16_at(uint32_t addr) {
    typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
    i16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(uintptr_t)addr);
    return __builtin_bit_cast(u32x2, v);
}
__device__ inline u32x4 lds_read16_at(uint32_t addr) {
    typedef __attribute__((address_space(3))) const u32x4 lds_u32x4;
    return *(lds_u32x4*)(uintptr_t)addr;
}

__device__ inline void compiler_fence() { asm volatile("" ::: "memory"); }

// threadIdx.x behind an empty asm statement: per-lane values derived from it are
// recomputed where they are used instead of being hoisted out of loops and held
// in registers across them.
__device__ inline int opaque_tid() {
    int t = threadIdx.x;
    asm volatile("" : "+v"(t));
    return t;
}

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
// The load is non-temporal (nt): every K/V row and query row staged this way
// is read once per call, and streaming reads with nt reach ~7.0 TB/s on MI355X
// against ~6.3 TB/s with the default policy (measured with a plain full-chip
// read); the decode's paged read rate rose from 5.7 to 6.5 TB/s with it.
__device__ inline void dma16(const void* gptr, uint32_t lds_base) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off nt" ::"v"(gptr), "s"(lds_base)
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


// Max / sum over the four 16-lane rows of a wave (lanes n, n+16, n+32, n+48),
// every lane receiving the result, with the gfx950 row-swap permutes (VALU;
// no LDS round trip).  permlane16_swap(v, v) returns rows (0,0,2,2) and (1,1,3,3)
// of v, permlane32_swap(v, v) rows (0,1,0,1) and (2,3,2,3); the sum is formed as
// (r0 + r1) + (r2 + r3) in every lane.
__device__ inline float rows4_max(float v) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    const float m = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(m), __float_as_uint(m), false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ inline float rows4_sum(float v) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    const float s = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(s), __float_as_uint(s), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}
__device__ inline int shfl_i(int v, int src) { return __shfl(v, src, kWave); }
__device__ inline uint64_t ballot(bool b) { return __ballot(b); }

// ---- online softmax ---------------------------------------------------------

// The running max is raised only when a row's new max exceeds it by more than
// this many base-2 units; below that, probabilities exp2(x - m) may reach 2^8,
// which fp32 accumulators and the 16-bit P operand hold with the same relative
// precision as values below 1.  The result is mathematically the same softmax.
constexpr float kMaxSlack = 8.0f;

// One online-softmax step over a 32-key stage for the rows of a lane column.
// s0 / s1: raw scores of keys 0-15 / 16-31 (lane (g, n) holds keys g*4 + i of
// row n); mask: visible keys (bit k = key k); l2scale: softmax scale / ln 2
// (p = exp2(score * l2scale - m)).  Updates the running max m, sum l and the
// accumulators o (rescaled when m is raised); returns the unnormalised p of the
// lane's 8 keys (keys g*4 + i, then 16 + g*4 + i).
//
// The common case -- every key visible and no score over the slack -- needs no
// row reduction: a wave in which any lane holds a score over the slack (or a
// row with no key yet, m = -inf) takes the exact path, which raises the max to
// the rows' maximum.  The accumulators are rescaled at one site, so the register
// allocator keeps them in place across the paths.
//
// kSum = false leaves the row sum to the caller (p_operands, for the 16-bit
// kernels).
template <bool kSum = true>
__device__ inline void softmax32(f32x4 (&o)[8], float& m, float& l, const f32x4& s0, const f32x4& s1,
                                 uint32_t mask, float l2scale, float (&pr)[8]) {
    const bool full = mask == 0xffffffffu && l2scale > 0.0f;
    bool exact = true;  // wave-uniform
    float mx;           // the row's scaled max, on the exact path
    if (full) {
        const float nm = -m;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            pr[i] = __builtin_fmaf(s0[i], l2scale, nm);
            pr[4 + i] = __builtin_fmaf(s1[i], l2scale, nm);
        }
        const float lmx =
            fmaxf(fmaxf(fmaxf(pr[0], pr[1]), fmaxf(pr[2], pr[3])), fmaxf(fmaxf(pr[4], pr[5]), fmaxf(pr[6], pr[7])));
        exact = ballot(lmx > kMaxSlack) != 0;
        // max of the raw scores, scaled once
        if (exact)
            mx = rows4_max(fmaxf(fmaxf(fmaxf(s0[0], s0[1]), fmaxf(s0[2], s0[3])),
                                 fmaxf(fmaxf(s1[0], s1[1]), fmaxf(s1[2], s1[3])))) *
                 l2scale;
    } else {
        // bit g*4 + i (+16) of the mask: the per-lane shift sits behind an empty
        // asm so the eight bit masks are not precomputed and held in registers
        uint32_t mg = mask >> (((opaque_tid() & 63) >> 4) * 4);
        asm volatile("" : "+v"(mg));
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            pr[i] = ((mg >> i) & 1u) ? s0[i] * l2scale : -DV_INF;
            pr[4 + i] = ((mg >> (16 + i)) & 1u) ? s1[i] * l2scale : -DV_INF;
        }
        mx = rows4_max(
            fmaxf(fmaxf(fmaxf(pr[0], pr[1]), fmaxf(pr[2], pr[3])), fmaxf(fmaxf(pr[4], pr[5]), fmaxf(pr[6], pr[7]))));
    }
    if (exact) {
        // raise the running max where some row exceeds it by more than the slack
        if (ballot(mx > m + kMaxSlack)) {
            const float mnew = fmaxf(m, mx);
            const float alpha = mnew == -DV_INF ? 1.0f : __builtin_amdgcn_exp2f(m - mnew);
            l *= alpha;
#pragma unroll
            for (int c = 0; c < 8; ++c) o[c] *= alpha;
            m = mnew;
        }
        const float mm = m == -DV_INF ? 0.0f : m;  // p = 0 while the row has no visible key
        if (full) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                pr[i] = __builtin_fmaf(s0[i], l2scale, -mm);
                pr[4 + i] = __builtin_fmaf(s1[i], l2scale, -mm);
            }
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) pr[i] -= mm;
        }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) pr[i] = __builtin_amdgcn_exp2f(pr[i]);
    if (kSum) {
        float ps = pr[0];
#pragma unroll
        for (int i = 1; i < 8; ++i) ps += pr[i];
        l += ps;
    }
}

// P^T operands of a lane's 8 probabilities, and their row-sum contribution.
// bf16: one operand; the normaliser sums the rounded weights (v_dot2 with ones,
// products exact), so the output is a convex combination of V rows -- a softmax
// concentrated on one key returns that row exactly, where an fp32 normaliser
// would leave the weight's 2^-9 rounding error.  fp16: the rounding residual
// p - fp16(p) goes into a second operand (hi + lo carries ~22 bits, one more
// P V MFMA per slice), so fp16 outputs keep the fp32-P accuracy their 1e-3
// tolerance needs; the normaliser is the fp32 sum.
struct POperand {
    u32x4 hi, lo;  // lo: fp16 only
};

template <int DT>
__device__ inline float dot2_ones(uint32_t x, float c) {
    if constexpr (DT == kBF16)
        return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, x), __builtin_bit_cast(bf16x2, 0x3f803f80u),
                                               c, false);
    else
        return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, x), __builtin_bit_cast(f16x2, 0x3c003c00u), c, false);
}

template <int DT>
__device__ inline POperand p_operands(const float (&pr)[8], float& l) {
    // the packed words are handled as scalars: taking them as elements of the
    // vector operand was compiled into four dot products of the first element
    uint32_t w[4], r[4] = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = pack2<DT>(pr[2 * i], pr[2 * i + 1]);
    if constexpr (DT == kBF16) {
        float ps = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) ps = dot2_ones<DT>(w[i], ps);
        l += ps;
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const f16x2 h = __builtin_bit_cast(f16x2, w[i]);
            r[i] = pack2<DT>(pr[2 * i] - (float)h[0], pr[2 * i + 1] - (float)h[1]);
        }
        float ps = pr[0];
#pragma unroll
        for (int i = 1; i < 8; ++i) ps += pr[i];
        l += ps;
    }
    return POperand{u32x4{w[0], w[1], w[2], w[3]}, u32x4{r[0], r[1], r[2], r[3]}};
}

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

// ---- split partials -----------------------------------------------------------
//
// A partial slot holds, for each of its nrows query rows (row j of the slot:
// one query head of one KV head or token), the piece's normalised output and
// its base-2 log-sum-exp:
//   fp32 and fp16 calls: values float[nrows][kHeadDim], lse float[nrows] after them;
//   bf16 calls: values fp16[nrows][kHeadDim] scaled per row by 2^k, the
//   exponents k int[nrows] right after the fp16 values, lse at the same float
//   offset as above (the slot keeps its fp32 size; half of it is left unused).
// The scale puts a row's largest finite magnitude in [2^14, 2^15), so every
// stored value is within 2^-11 of that magnitude of the exact normalised
// output: a quarter of the relative rounding (2^-9) the piece already applied
// to the probabilities when it packed them to bf16 for P V, and 1/16 of the
// output's own bf16 rounding.  Infinite values stay infinite, NaN stays NaN.
// Half the bytes of fp32 partials are written and read again by the merge.
template <int DT> constexpr bool kHalfPartials = DT == kBF16;

// Scale exponent of a row whose largest finite |value| is amax (0 for an empty
// or zero row): amax * 2^k in [2^14, 2^15), at most 2^100 so that the factor
// stays finite for rows of tiny values.
__device__ inline int partial_exp(float amax) {
    const int k = 15 - __builtin_amdgcn_frexp_expf(amax);  // amax = m * 2^e, m in [0.5, 1)
    return k < 100 ? k : 100;
}

// Lane (g, n) holds dims c*16 + g*4 + e (c < 8, e < 4) of slot row j in o
// (unnormalised; inv = 1 / row sum); the four lanes of a row are n + 16g, and
// every lane of the wave takes part (cross-lane maximum).  g == 0 also writes
// the row's lse.
template <int DT>
__device__ inline void store_partial(float* sbase, int nrows, int j, int g, const f32x4 (&o)[8], float inv,
                                     float lse) {
    if constexpr (kHalfPartials<DT>) {
        float amax = 0.0f;
#pragma unroll
        for (int c = 0; c < 8; ++c) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float a = __builtin_fabsf(o[c][e]);
                amax = fmaxf(amax, a < DV_INF ? a : 0.0f);
            }
        }
        const int k = partial_exp(rows4_max(amax) * inv);
        const float sc = __builtin_amdgcn_ldexpf(inv, k);
        uint16_t* h = reinterpret_cast<uint16_t*>(sbase) + j * kHeadDim;
#pragma unroll
        for (int c = 0; c < 8; ++c)
            *reinterpret_cast<u32x2*>(h + c * 16 + g * 4) =
                u32x2{pack2<kF16>(o[c][0] * sc, o[c][1] * sc), pack2<kF16>(o[c][2] * sc, o[c][3] * sc)};
        if (g == 0) {
            reinterpret_cast<int*>(sbase)[nrows * (kHeadDim / 2) + j] = k;
            sbase[nrows * kHeadDim + j] = lse;
        }
    } else {
        float* v = sbase + j * kHeadDim;
#pragma unroll
        for (int c = 0; c < 8; ++c) *reinterpret_cast<f32x4*>(v + c * 16 + g * 4) = o[c] * inv;
        if (g == 0) sbase[nrows * kHeadDim + j] = lse;
    }
}

// Pieces whose loads are in flight together in a merge: segments of up to
// kMergeBatch pieces take one round, longer ones rounds of kMergeBatchLong (a
// merge kernel lasts as long as its segment with the most pieces, and every
// round is a dependent memory round trip).
constexpr int kMergeBatch = 8;
constexpr int kMergeBatchLong = 16;

// Merge of the pieces [base, base + cnt) of one segment (slots of slot_floats
// floats from part) for slot row j of nrows, NQ runs of eight dims starting at
// d[q]: the base-2-LSE-weighted sum of the pieces' normalised outputs
// (paged_kernel_v21.cuh:325-364), with B pieces' loads in flight per round
// (merge_runs: B = kMergeBatch up to kMergeBatch pieces, else kMergeBatchLong).
// res[q][e] = merged value of dim d[q] + e; 0 when no piece has a visible key.
// The result depends on the pieces and on B (the running max is raised once
// per round).
// merge_acc_b: the accumulation -- the running base-2 max m_out, the weight
// sum wsum_out and the weighted sum acc over the pieces (-inf, 0 and zeros for
// none); merge_runs_b normalises it.
template <int DT, int NQ, int B>
__device__ inline void merge_acc_b(const float* part, long long slot_floats, int nrows, int j, const int (&d)[NQ],
                                   int base, int cnt, float& m_out, float& wsum_out, float (&acc)[NQ][8]) {
    float m = -DV_INF, wsum = 0.0f;
#pragma unroll
    for (int q = 0; q < NQ; ++q)
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[q][e] = 0.0f;
    for (int k0 = 0; k0 < cnt; k0 += B) {
        float lse[B];
        int kx[B];
        u32x4 h[B][NQ];
        f32x4 v0[B][NQ], v1[B][NQ];
#pragma unroll
        for (int i = 0; i < B; ++i) {
            const bool in = k0 + i < cnt;
            const float* sp = part + (long long)(base + (in ? k0 + i : k0)) * slot_floats;
            lse[i] = in ? sp[nrows * kHeadDim + j] : -DV_INF;
            if constexpr (kHalfPartials<DT>) {
                kx[i] = reinterpret_cast<const int*>(sp)[nrows * (kHeadDim / 2) + j];
#pragma unroll
                for (int q = 0; q < NQ; ++q) h[i][q] = ld16(reinterpret_cast<const uint16_t*>(sp) + j * kHeadDim + d[q]);
            } else {
#pragma unroll
                for (int q = 0; q < NQ; ++q) {
                    v0[i][q] = ld16f(sp + j * kHeadDim + d[q]);
                    v1[i][q] = ld16f(sp + j * kHeadDim + d[q] + 4);
                }
            }
        }
        float bm = m;
#pragma unroll
        for (int i = 0; i < B; ++i) bm = fmaxf(bm, lse[i]);
        if (bm == -DV_INF) continue;
        const float sc = exp2f(m - bm);  // m == -inf -> 0
        wsum *= sc;
#pragma unroll
        for (int q = 0; q < NQ; ++q)
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[q][e] *= sc;
#pragma unroll
        for (int i = 0; i < B; ++i) {
            const float wgt = exp2f(lse[i] - bm);  // empty piece (-inf) -> 0
            wsum += wgt;
            if constexpr (kHalfPartials<DT>) {
                const float w = __builtin_amdgcn_ldexpf(wgt, -kx[i]);
                // halves taken by shifts: a bit cast of a vector element to
                // f16x2 was compiled as a cast of element 0 for every element
#pragma unroll
                for (int q = 0; q < NQ; ++q) {
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        const uint32_t hw = h[i][q][t];
                        acc[q][2 * t] = __builtin_fmaf(w, Tr<kF16>::tof((uint16_t)(hw & 0xffffu)), acc[q][2 * t]);
                        acc[q][2 * t + 1] = __builtin_fmaf(w, Tr<kF16>::tof((uint16_t)(hw >> 16)), acc[q][2 * t + 1]);
                    }
                }
            } else {
#pragma unroll
                for (int q = 0; q < NQ; ++q) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        acc[q][e] = __builtin_fmaf(wgt, v0[i][q][e], acc[q][e]);
                        acc[q][4 + e] = __builtin_fmaf(wgt, v1[i][q][e], acc[q][4 + e]);
                    }
                }
            }
        }
        m = bm;
    }
    m_out = m;
    wsum_out = wsum;
}

template <int DT, int NQ, int B>
__device__ inline void merge_runs_b(const float* part, long long slot_floats, int nrows, int j, const int (&d)[NQ],
                                    int base, int cnt, float (&res)[NQ][8]) {
    float m, wsum, acc[NQ][8];
    merge_acc_b<DT, NQ, B>(part, slot_floats, nrows, j, d, base, cnt, m, wsum, acc);
    const float inv = wsum > 0.0f ? 1.0f / wsum : 0.0f;
#pragma unroll
    for (int q = 0; q < NQ; ++q)
#pragma unroll
        for (int e = 0; e < 8; ++e) res[q][e] = acc[q][e] * inv;
}

template <int DT, int NQ>
__device__ inline void merge_runs(const float* part, long long slot_floats, int nrows, int j, const int (&d)[NQ],
                                  int base, int cnt, float (&res)[NQ][8]) {
    if (cnt <= kMergeBatch)
        merge_runs_b<DT, NQ, kMergeBatch>(part, slot_floats, nrows, j, d, base, cnt, res);
    else
        merge_runs_b<DT, NQ, kMergeBatchLong>(part, slot_floats, nrows, j, d, base, cnt, res);
}

// Eight merged values stored to the output (16-bit: one 16-byte store).
template <int DT>
__device__ inline void store_run8(typename Tr<DT>::raw* o, const float (&v)[8]) {
    if constexpr (DT == kF32) {
        *reinterpret_cast<f32x4*>(o) = f32x4{v[0], v[1], v[2], v[3]};
        *reinterpret_cast<f32x4*>(o + 4) = f32x4{v[4], v[5], v[6], v[7]};
    } else {
        *reinterpret_cast<u32x4*>(o) =
            u32x4{pack2<DT>(v[0], v[1]), pack2<DT>(v[2], v[3]), pack2<DT>(v[4], v[5]), pack2<DT>(v[6], v[7])};
    }
}

}  // namespace dv
