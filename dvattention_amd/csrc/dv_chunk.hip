// gfx950 multi-query ("chunk") attention with fused query RoPE: S >= 2 query
// tokens per sequence that share one K/V stream (chunked prefill, speculative
// verification).  Same operator semantics as the decode kernel
// (src/kernels/paged_kernel_v21.cuh:17-374 and kernel_v21.cuh:17-367 in the
// reference repository, which re-read K/V once per query token: grid.y = W*S,
// paged_kernel_v21.cuh:391); here each K/V row is read once per block of 16
// tokens.
//
//  * Workgroup = eight waves, two per SIMD, on one (sequence, 16-token block,
//    KV head) and a contiguous range of its visible keys.  Wave w owns tokens
//    2w and 2w+1: two 16-row query tiles (16 heads each), so a K/V stage read
//    from LDS feeds 32 query rows per wave and 256 per workgroup.
//  * K/V pages stream through an 8-stage LDS ring filled by direct-to-LDS loads
//    (global_load_lds_dwordx4, non-temporal): 32 keys x 256 B of K and of V per
//    stage, one eighth issued by each wave, seven stages ahead of the one
//    computed, completion tracked with vmcnt and one workgroup barrier per stage.
//  * Per stage and tile: S^T = K Q^T on 16x16x32 MFMA (8 per tile), online
//    softmax per query row, O^T += V^T P^T (8 MFMA per tile, 16 for fp16: see
//    p_operands); the K and V^T operands of a stage are read from LDS once per
//    wave and kept in registers for both tiles.
//  * MFMA / VALU overlap inside the wave: the two tiles (A = 0, B = 1) run half
//    a stage apart.  Each half-stage issues one tile's MFMAs (S of B and P V of
//    B's previous stage, or P V of A and S of A's next stage) while the other
//    tile's softmax runs on the VALU, so the two use disjoint registers and the
//    matrix core has work during the softmax; the second wave on the SIMD fills
//    what one wave's dependences leave idle.
//  * Rows are causal-masked per token (key l visible iff l <= locations[f,w,s]).
//  * The balanced split / LSE merge is the decode kernel's (equal key chunks per
//    workgroup, fp32 partial slots, dv_merge_chunk).
#include "dv_chunk.h"

namespace dv {
namespace chunk {

// Workgroup barrier that is also a compiler memory and scheduling barrier: no
// LDS access or MFMA moves across it.
__device__ inline void wg_barrier() {
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_barrier" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
}

// swizzled 16-byte piece positions inside a 256-byte key row
__device__ inline int swz_k(int key, int piece) { return piece ^ (key & 15); }
__device__ inline int swz_v(int key, int piece) { return piece ^ ((key & 7) << 1); }

// Issue this wave's eighth of stage `st` (keys [kb0, kb0+32) of the range): key
// rows 4*wave .. 4*wave+3 of K and of V, lane -> (row lane/16, 16-byte piece).
template <int KVM, bool P2>
__device__ inline void issue_stage(const DecodeParams& p, const Range& r, const int* pages, uint32_t ring,
                                   int st, int kb0) {
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int pos = lane & 15;
    const uint32_t sbase = ring + (uint32_t)(st % kStages) * kStageBytes;
    const int kl = wv * 4 + (lane >> 4);
    const int gk = swz_k(kl, pos), gv = swz_v(kl, pos);
    const uint32_t koff = (uint32_t)(wv * 4) * 256;
    const unsigned char* ka;
    const unsigned char* va;
    if (KVM == kKvPaged && P2 && r.pages_ok && kb0 + kStep <= r.b) {
        // interior stage of a range whose pages are all valid: no visibility
        // test and no zero rows
        const uint32_t pos_l = (uint32_t)(r.off + kb0 + kl);
        const int pg = pages[(pos_l >> p.bs_shift) - r.lp0];
        const uint32_t rowidx = (((uint32_t)pg << p.bs_shift) + (pos_l & ((1u << p.bs_shift) - 1u))) *
                                    (uint32_t)p.Hkv + (uint32_t)r.hkv;
        const unsigned long long boff = (unsigned long long)rowidx << 8;
        ka = r.k + boff + gk * 16;
        va = r.v + boff + gv * 16;
    } else {
        const long long row = row_of<KVM, P2>(p, r, pages, kb0 + kl);
        ka = row >= 0 ? r.k + row + gk * 16 : zrow + gk * 16;
        va = row >= 0 ? r.v + row + gv * 16 : zrow + gv * 16;
    }
    dma16(ka, __builtin_amdgcn_readfirstlane(sbase + koff));
    dma16(va, __builtin_amdgcn_readfirstlane(sbase + kKvBytes + koff));
}

struct Tile {
    f32x4 o[8];
    float m, l;
    // -max(m, -FLT_MAX), the exponent offset of every stage: kept beside m and
    // updated only where m changes (sm_raise), not recomputed per stage
    float nm;
};

// Query tiles of this wave's tokens tok0 .. tok0 + ntile - 1 of group gr for
// view f, staged through LDS (the K/V ring is idle between view ranges): raw
// q rows arrive by direct-to-LDS loads, each lane rotates whole (d, d + R/2)
// pairs in place (src/rope.cuh:18-51 and :67-114: first R/2 cos/sin entries of
// the token's full-width row, or its half-width varlen row; separately rounded
// fp32 products and sum, rounded to the storage type; dims >= R untouched),
// then lane (g, n) reads Q[n][c*32 + g*8 + 0..7] of every tile.  Wave-private
// LDS region: 8 KiB.
template <int DT, int QM, int RM>
__device__ inline void stage_q_tiles(const DecodeParams& p, unsigned char* qreg, float* csreg, const Grp& gr,
                                     int tok0, int ntile, int f, int hkv, u32x4 (&qB)[kTiles][4]) {
#pragma clang fp contract(off)
    using raw = typename Tr<DT>::raw;
    const int lane = opaque_tid() & 63;
    const int g = lane >> 4, n = lane & 15;
    const uint32_t qbase = lds_addr(qreg);
    for (int t = 0; t < ntile; ++t) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int hn = i * 4 + (lane >> 4);
            const int h = hkv * kGqa + hn;
            const raw* q = reinterpret_cast<const raw*>(p.q) + q_row<QM, RM>(p, gr, tok0 + t, h, f);
            dma16(q + (lane & 15) * 8, __builtin_amdgcn_readfirstlane(qbase + (uint32_t)(t * 4096 + i * 1024)));
        }
    }
    const int half = p.R >> 1;
    if (QM != kQPre) {
        for (int t = 0; t < ntile; ++t) {
            const long long row = (long long)f * tok_axis<RM>(p) + gr.lin + tok0 + t;
            const long long co = QM == kQRotHalf ? row * half : row * p.R;
            csreg[t * 128 + lane] = lane < half ? p.cosv[co + lane] : 0.0f;
            csreg[t * 128 + 64 + lane] = lane < half ? p.sinv[co + lane] : 0.0f;
        }
    }
    wait_vmcnt<0>();
    compiler_fence();
    if (QM != kQPre && half > 0) {
        const int hn = lane >> 2, q4 = lane & 3;
        for (int t = 0; t < ntile; ++t) {
            raw* x = reinterpret_cast<raw*>(qreg + t * 4096 + hn * 256);
            const float* cs = csreg + t * 128;
            const float* sn = cs + 64;
            if ((half & 7) == 0) {
                for (int j0 = q4 * 8; j0 < half; j0 += 32) {
                    const u32x4 a = *reinterpret_cast<const u32x4*>(x + j0);
                    const u32x4 b = *reinterpret_cast<const u32x4*>(x + j0 + half);
                    u32x4 ya, yb;
#pragma unroll
                    for (int e2 = 0; e2 < 4; ++e2) {
                        uint32_t pa = 0, pb = 0;
#pragma unroll
                        for (int hl = 0; hl < 2; ++hl) {
                            const int e = e2 * 2 + hl;
                            const float x1 = Tr<DT>::tof((raw)((a[e2] >> (16 * hl)) & 0xffffu));
                            const float x2 = Tr<DT>::tof((raw)((b[e2] >> (16 * hl)) & 0xffffu));
                            const float c = cs[j0 + e], sv = sn[j0 + e];
                            const float a1 = x1 * c, b1 = x2 * sv;
                            const float a2 = x2 * c, b2 = x1 * sv;
                            pa |= (uint32_t)Tr<DT>::fromf(a1 - b1) << (16 * hl);
                            pb |= (uint32_t)Tr<DT>::fromf(a2 + b2) << (16 * hl);
                        }
                        ya[e2] = pa;
                        yb[e2] = pb;
                    }
                    *reinterpret_cast<u32x4*>(x + j0) = ya;
                    *reinterpret_cast<u32x4*>(x + j0 + half) = yb;
                }
            } else {
                for (int j = q4; j < half; j += 4) {
                    const float x1 = Tr<DT>::tof(x[j]), x2 = Tr<DT>::tof(x[j + half]);
                    const float c = cs[j], sv = sn[j];
                    const float a1 = x1 * c, b1 = x2 * sv;
                    const float a2 = x2 * c, b2 = x1 * sv;
                    x[j] = Tr<DT>::fromf(a1 - b1);
                    x[j + half] = Tr<DT>::fromf(a2 + b2);
                }
            }
        }
        compiler_fence();
    }
#pragma unroll
    for (int t = 0; t < kTiles; ++t)
        if (t < ntile)
#pragma unroll
            for (int cc = 0; cc < 4; ++cc)
                qB[t][cc] = *reinterpret_cast<const u32x4*>(qreg + t * 4096 + n * 256 + (cc * 32 + g * 8) * 2);
    compiler_fence();
}

// frag / view_vis: the views' tensors and visible key counts (dv_stream.h)

// K operand of one stage (A of S^T = K Q^T): lo[cc] holds key n, hi[cc] key
// 16 + n, dims cc*32 + g*8 .. +8 (lane (g, n)).  The K swizzle only flips
// address bits 6-7 of the row base, so slice cc is at kbase ^ (64 cc).
struct KOp {
    u32x4 lo[4], hi[4];
};

// V^T operand of one stage (A of O^T += V^T P^T), 16-dim slice cc: block lane
// sl -> key g*4 + sl/4 (and + 16), dims cc*16 + (sl%4)*4 (transposing reads);
// the V swizzle only flips address bits 5-7, so slice cc is at vbase ^ (32 cc).
struct VOp {
    u32x4 v[8];
};

__device__ inline void read_k(const unsigned char* kt, KOp& k) {
    const int lane = threadIdx.x & 63;
    const int g = lane >> 4, n = lane & 15;
    const uint32_t kbase = lds_addr(kt) + (uint32_t)(n * 256 + 16 * (g ^ (n & 3)) + 64 * (n >> 2));
#pragma unroll
    for (int cc = 0; cc < 4; ++cc) {
        k.lo[cc] = lds_read16_at(kbase ^ (uint32_t)(64 * cc));
        k.hi[cc] = lds_read16_at((kbase ^ (uint32_t)(64 * cc)) + 16 * 256);
    }
}

__device__ inline void read_v(const unsigned char* vt, VOp& v) {
    const int lane = threadIdx.x & 63;
    const int g = lane >> 4, sl = lane & 15;
    const int k0 = g * 4 + (sl >> 2);
    const uint32_t vbase =
        lds_addr(vt) + (uint32_t)(k0 * 256 + 16 * ((sl & 3) >> 1) + (sl & 1) * 8 + 32 * (k0 & 7));
#pragma unroll
    for (int cc = 0; cc < 8; ++cc) {
        const u32x2 a0 = lds_read_tr16_at(vbase ^ (uint32_t)(32 * cc));
        const u32x2 a1 = lds_read_tr16_at((vbase ^ (uint32_t)(32 * cc)) + 16 * 256);
        v.v[cc] = u32x4{a0[0], a0[1], a1[0], a1[1]};
    }
}

// Scores of one tile: s0 keys 0-15, s1 keys 16-31 (S^T, lane (g, n): keys
// g*4 + i of head n).
template <int DT>
__device__ inline void qk_tile(const KOp& k, const u32x4 (&q)[4], f32x4& s0, f32x4& s1) {
    s0 = f32x4{0.f, 0.f, 0.f, 0.f};
    s1 = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int cc = 0; cc < 4; ++cc) {
        s0 = Tr<DT>::mma(k.lo[cc], q[cc], s0);
        s1 = Tr<DT>::mma(k.hi[cc], q[cc], s1);
    }
}

// O^T += V^T P^T for one tile.
template <int DT>
__device__ inline void pv_tile(const VOp& v, const POperand& pB, Tile& t) {
#pragma unroll
    for (int cc = 0; cc < 8; ++cc) t.o[cc] = Tr<DT>::mma(v.v[cc], pB.hi, t.o[cc]);
    if constexpr (DT == kF16) {
#pragma unroll
        for (int cc = 0; cc < 8; ++cc) t.o[cc] = Tr<DT>::mma(v.v[cc], pB.lo, t.o[cc]);
    }
}

// Visibility of the 32 keys of the stage starting at kb0: the range end, and,
// when some page of the sub-range is missing, page validity (a scalar branch
// around a few instructions; the loop itself is not duplicated).
template <int KVM, bool P2>
__device__ inline uint32_t stage_mask(const DecodeParams& p, const Range& r, const int* pages, int sbnd, int kb0) {
    const int nin = sbnd - kb0;
    uint32_t m = nin >= 32 ? 0xffffffffu : ((1u << nin) - 1u);
    if (!r.pages_ok) {
        const int lane = threadIdx.x & 63;
        const bool kv_ok = row_of<KVM, P2>(p, r, pages, kb0 + (lane & 31)) >= 0;
        m &= (uint32_t)ballot(kv_ok && lane < 32);
    }
    return m;
}

// Scores of invisible keys set to -inf (mask bit k = key k; lane (g, n) holds
// keys g*4 + i and 16 + g*4 + i): a partially visible stage only, so full
// stages spend nothing on masks.
__device__ inline void mask_scores(f32x4& s0, f32x4& s1, uint32_t mask) {
    const int lane = threadIdx.x & 63;
    const uint32_t mg = mask >> ((lane >> 4) * 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        s0[i] = ((mg >> i) & 1u) ? s0[i] : -DV_INF;
        s1[i] = ((mg >> (16 + i)) & 1u) ? s1[i] : -DV_INF;
    }
}

// Online softmax of two tiles over one 32-key stage, in two straight-line
// parts so that the MFMAs of the other tile group can be interleaved with it
// (a branch ends the scheduling region).  Scores of invisible keys are -inf
// already (mask_scores).  Part 1: base-2 exponents against the running max
// (lane (g, n) holds keys g*4 + i and 16 + g*4 + i of head n); returns the
// lane's largest, so the caller can ask whether some row exceeds its max by
// more than kMaxSlack or has no max yet -- then sm_raise (rare) raises the max
// to the rows' maximum, rescales the accumulators and recomputes the
// exponents.  Part 2 (sm_finish): the probabilities, the row sums and the P^T
// operands.  Same arithmetic as softmax32 + p_operands.
__device__ inline float sm_exponents(const Tile& t, const f32x4& s0, const f32x4& s1, float l2, float (&pr)[8]) {
    // a row with no max yet (m = -inf) subtracts -FLT_MAX instead (t.nm): a
    // visible key's exponent is then huge (the row takes sm_raise) and an
    // invisible key's stays -inf, where -inf - (-inf) would be NaN
    const float nm = t.nm;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        pr[i] = __builtin_fmaf(s0[i], l2, nm);
        pr[4 + i] = __builtin_fmaf(s1[i], l2, nm);
    }
    // shaped for three-operand maxima: max3(max3(0,1,2), max3(3,4,5), max(6,7)),
    // four instructions where a balanced pairwise tree compiled to five
    const float a = fmaxf(fmaxf(pr[0], pr[1]), pr[2]), b = fmaxf(fmaxf(pr[3], pr[4]), pr[5]);
    return fmaxf(fmaxf(a, b), fmaxf(pr[6], pr[7]));
}

__device__ inline void sm_raise(Tile& t, const f32x4& s0, const f32x4& s1, float l2, float (&pr)[8]) {
    float sc[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        sc[i] = s0[i] * l2;
        sc[4 + i] = s1[i] * l2;
    }
    const float mx = rows4_max(
        fmaxf(fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3])), fmaxf(fmaxf(sc[4], sc[5]), fmaxf(sc[6], sc[7]))));
    if (ballot(mx > t.m + kMaxSlack)) {
        const float mnew = fmaxf(t.m, mx);
        const float alpha = mnew == -DV_INF ? 1.0f : __builtin_amdgcn_exp2f(t.m - mnew);
        t.l *= alpha;
#pragma unroll
        for (int c = 0; c < 8; ++c) t.o[c] *= alpha;
        t.m = mnew;
        t.nm = -fmaxf(mnew, -3.402823466e38f);
    }
    const float mm = t.m == -DV_INF ? 0.0f : t.m;  // p = 0 while the row has no visible key
#pragma unroll
    for (int i = 0; i < 8; ++i) pr[i] = sc[i] - mm;
}

template <int DT>
__device__ inline POperand sm_finish(Tile& t, float (&pr)[8]) {
#pragma unroll
    for (int i = 0; i < 8; ++i) pr[i] = __builtin_amdgcn_exp2f(pr[i]);
    return p_operands<DT>(pr, t.l);
}

// Register tie: the values are complete at this point in program order (the
// compiler may not move their computation past it, e.g. across a workgroup
// barrier into the next half-stage).  Only the words the P V MFMAs read are
// tied: bf16 has no residual operand, and tying its (zero) lo made the
// compiler rebuild and copy four zero registers every half-stage.
template <int DT>
__device__ inline void settle(POperand& a) {
    asm volatile("" : "+v"(a.hi));
    if constexpr (DT == kF16) asm volatile("" : "+v"(a.lo));
}

// Keys [sa, sbnd) of the current view for this wave's two tiles (A = tile 0,
// B = tile 1): the stage loop.  Ring slot i % kStages holds stage i.  Per
// stage i, in every wave:
//   H1(i): MFMA O_B += V(i-1) P_B(i-1) beside A's exponents; MFMA S_B(i) =
//          K(i) Q_B^T and read V(i) beside A's probabilities
//   own loads of stage i+1 landed; workgroup barrier
//   H2(i): read K(i+1); MFMA O_A += V(i) P_A(i) beside B's exponents; MFMA
//          S_A(i+1) = K(i+1) Q_A^T and the loads of stage i+kAhead beside B's
//          probabilities
// so each wave's instruction stream alternates MFMAs of one tile with the
// softmax of the other, and the two waves of a SIMD issue both at once.  A
// slot is refilled (stage i+kAhead into the slot of stage i-1) only after the
// barrier of stage i+1, which every wave reaches having completed its reads of
// every stage <= i (the V reads of H1 are waited for before the barrier).  One
// K and one V^T operand set live in registers: K(i+1) is read after the MFMAs
// of K(i) are issued, V(i) after those of V(i-1).  A's accumulators are
// rescaled in H1 and written by MFMAs issued in H2 (and B's the other way
// round), so a softmax never touches registers an MFMA of the same half-stage
// writes; mfma_settle before each softmax covers the MFMA -> VALU dependence
// across the half-stage boundary.  Invisible keys get -inf scores only on a
// partially visible stage (a uniform branch between the interleaved regions).
template <int DT, int KVM, bool P2>
__device__ inline void stream_range(const DecodeParams& p, const Range& r, const int* pages, unsigned char* smem,
                                    int sa, int sbnd, const int (&vis_t)[kTiles], const u32x4 (&qB)[kTiles][4],
                                    Tile (&tl)[kTiles]) {
    const uint32_t ring = lds_addr(smem);
    const int nsteps = (sbnd - sa + kStep - 1) / kStep;
    const float l2 = p.l2scale;
    // prologue: stages 0 .. kAhead-1 (past the end: rows of zeros)
#pragma unroll
    for (int st = 0; st < kAhead; ++st) issue_stage<KVM, P2>(p, r, pages, ring, st, sa + st * kStep);
    wait_vmcnt<kDmaPerStage * (kAhead - 1)>();  // own share of stage 0 landed
    wg_barrier();

    KOp kop;
    VOp vop;
#pragma unroll
    for (int cc = 0; cc < 8; ++cc) vop.v[cc] = u32x4{0u, 0u, 0u, 0u};  // the first P V adds 0 * 0
    f32x4 sa0, sa1, sb0, sb1;
    POperand pa = {}, pb = {};
    read_k(smem, kop);
    qk_tile<DT>(kop, qB[0], sa0, sa1);

    for (int i = 0; i < nsteps; ++i) {
        const int kb0 = sa + i * kStep;
        const unsigned char* slot = smem + (i % kStages) * kStageBytes;
        const uint32_t okm = stage_mask<KVM, P2>(p, r, pages, sbnd, kb0);
        const uint32_t mka = okm & token_mask(vis_t[0], kb0), mkb = okm & token_mask(vis_t[1], kb0);
        float pr[8];
        // ---- H1(i)
        if (mka != 0xffffffffu) mask_scores(sa0, sa1, mka);
        mfma_settle(tl[0].o);
        pv_tile<DT>(vop, pb, tl[1]);  // zero at i = 0
        float lmx = sm_exponents(tl[0], sa0, sa1, l2, pr);
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
            __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);  // VALU
        }
        if (ballot(lmx > kMaxSlack)) sm_raise(tl[0], sa0, sa1, l2, pr);
        qk_tile<DT>(kop, qB[1], sb0, sb1);
        read_v(slot + kKvBytes, vop);
        pa = sm_finish<DT>(tl[0], pr);
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
            __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // LDS read
            __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);  // VALU
        }
        settle<DT>(pa);
        lds_wait();
        wait_vmcnt<kDmaPerStage * (kAhead - 2)>();  // own share of stage i + 1 landed
        wg_barrier();
        // ---- H2(i) (stage i + 1 has landed even past the end -- rows of zeros --
        // so K and S_A of the next stage need no branch; the last ones go unused)
        read_k(smem + ((i + 1) % kStages) * kStageBytes, kop);
        if (mkb != 0xffffffffu) mask_scores(sb0, sb1, mkb);
        mfma_settle(tl[1].o);
        pv_tile<DT>(vop, pa, tl[0]);
        lmx = sm_exponents(tl[1], sb0, sb1, l2, pr);
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // LDS read
            __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);  // VALU
        }
        if (ballot(lmx > kMaxSlack)) sm_raise(tl[1], sb0, sb1, l2, pr);
        qk_tile<DT>(kop, qB[0], sa0, sa1);
        pb = sm_finish<DT>(tl[1], pr);
        // the loads of stage i + kAhead (into the slot of stage i - 1, free since
        // the barrier), their address arithmetic beside the MFMAs
        issue_stage<KVM, P2>(p, r, pages, ring, i + kAhead, sa + (i + kAhead) * kStep);
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
            __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);  // VALU
        }
        settle<DT>(pb);
    }
    // P V of B's last stage
    mfma_settle(tl[1].o);
    pv_tile<DT>(vop, pb, tl[1]);
#pragma unroll
    for (int t = 0; t < kTiles; ++t) mfma_settle(tl[t].o);
    wait_vmcnt<0>();  // the trailing zero-row stages land before the ring is reused
    __syncthreads();
}

// One workgroup: keys [v0, v1) of row group rg for KV head hkv.
template <int DT, int QM, int KVM, bool P2, int RM>
__device__ void chunk_piece(const DecodeParams& p, unsigned char* smem, int* pages, int rg, int hkv, long long v0,
                            long long v1, bool final_out, int slot) {
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int g = lane >> 4, n = lane & 15;
    const Grp gr = group_of<RM>(p, rg);
    const int w = gr.w;
    const int tok0 = wv * kTiles;  // this wave's first token of the group
    const int ntile = gr.ntok - tok0 < kTiles ? (gr.ntok - tok0 > 0 ? gr.ntok - tok0 : 0) : kTiles;

    Tile tl[kTiles];
#pragma unroll
    for (int t = 0; t < kTiles; ++t) {
#pragma unroll
        for (int c = 0; c < 8; ++c) tl[t].o[c] = f32x4{0.f, 0.f, 0.f, 0.f};
        tl[t].m = -DV_INF;
        tl[t].l = 0.0f;
        tl[t].nm = 3.402823466e38f;
    }

    long long P = 0, off = 0;
    for (int f = 0; f < p.F && P < v1; ++f) {
        // visible keys of this view for the block (union) and per tile
        const int vis_blk = group_view_vis<KVM, RM>(p, f, gr);
        int vis_t[kTiles];
#pragma unroll
        for (int t = 0; t < kTiles; ++t)  // wave-uniform: the stage masks and their branches stay scalar
            vis_t[t] = __builtin_amdgcn_readfirstlane(t < ntile ? view_vis<KVM>(p, f, loc_of<RM>(p, f, gr, tok0 + t)) : 0);
        const long long a = v0 > P ? v0 : P;
        const long long bnd = v1 < P + vis_blk ? v1 : P + vis_blk;
        if (a < bnd) {
            u32x4 qB[kTiles][4] = {};
            // the ring is idle here (previous range drained): stage the query tiles in it
            stage_q_tiles<DT, QM, RM>(p, smem + wv * (kTiles * 4096),
                                      reinterpret_cast<float*>(smem + kWaves * kTiles * 4096 + wv * kTiles * 512), gr,
                                      tok0, ntile, f, hkv, qB);
            __syncthreads();
            Range r;
            r.w = w;
            r.hkv = hkv;
            if (KVM == kKvPaged) {
                r.k = reinterpret_cast<const unsigned char*>(p.kc);
                r.v = reinterpret_cast<const unsigned char*>(p.vc);
                r.off = off;
                r.bstride = 0;
                r.L = 0;
            } else {
                const FragDesc& fd = frag<KVM>(p, f);
                r.k = reinterpret_cast<const unsigned char*>(fd.k);
                r.v = reinterpret_cast<const unsigned char*>(fd.v);
                r.off = 0;
                r.bstride = fd.bstride * w;
                r.L = fd.L;
            }
            const int la = (int)(a - P), lb = (int)(bnd - P);
            // sub-ranges whose page ids fit the LDS page cache
            const int span = KVM == kKvPaged ? (p.bs_shift >= 0 ? (kPageCap - 2) << p.bs_shift : (kPageCap - 2) * p.bs)
                                             : (1 << 30);
            for (int sa = la; sa < lb; sa += span) {
                const int sbnd = sa + span < lb ? sa + span : lb;
                r.b = sbnd;
                r.pages_ok = true;
                if (KVM == kKvPaged) {
                    const uint32_t p0 = (uint32_t)(off + sa), p1 = (uint32_t)(off + sbnd - 1);
                    const uint32_t lpl = p.bs_shift >= 0 ? (p1 >> p.bs_shift) : p1 / (uint32_t)p.bs;
                    r.lp0 = p.bs_shift >= 0 ? (p0 >> p.bs_shift) : p0 / (uint32_t)p.bs;
                    __syncthreads();
                    // every page this thread loaded for the sub-range is valid
                    const bool ok = fill_page_cache(p, p.bt + (long long)w * p.maxB, pages, r.lp0, lpl);
                    r.pages_ok = __syncthreads_and(ok) != 0;
                }
                stream_range<DT, KVM, P2>(p, r, pages, smem, sa, sbnd, vis_t, qB, tl);
            }
        }
        P += vis_blk;
        off += p.fl[f];
    }

    // epilogue: per tile, normalise and write the output or a partial slot
    {
    const int lane = opaque_tid() & 63;
    const int g = lane >> 4, n = lane & 15;
#pragma unroll
    for (int t = 0; t < kTiles; ++t) {
        if (t >= ntile) continue;
        const float lt = rows4_sum(tl[t].l);
        const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
        const int h = hkv * kGqa + n;
        if (final_out) {
            using raw = typename Tr<DT>::raw;
            raw* o = reinterpret_cast<raw*>(p.out) + out_row<RM>(p, gr, tok0 + t, h);
#pragma unroll
            for (int c = 0; c < 8; ++c) {
                const u32x2 pk = {pack2<DT>(tl[t].o[c][0] * inv, tl[t].o[c][1] * inv),
                                  pack2<DT>(tl[t].o[c][2] * inv, tl[t].o[c][3] * inv)};
                *reinterpret_cast<u32x2*>(o + c * 16 + g * 4) = pk;
            }
        } else {
            const int tb = wv * kTiles + t;  // token within the block
            store_partial<DT>(p.part + (long long)slot * p.slot_floats, kTokBlk * kGqa, tb * kGqa + n, g, tl[t].o,
                              inv, lt > 0.0f ? tl[t].m + log2f(lt) : -DV_INF);
        }
    }
    }
}

// P2: paged with a power-of-two block_size (shift and mask instead of a
// division in the stage loop's row addressing).
template <int DT, int QM, int KVM, bool P2, int RM>
__global__ __launch_bounds__(kThreads) void dv_chunk(const DecodeParams p) {
    extern __shared__ __align__(16) unsigned char smem_raw[];
    // the ring starts at a 256-byte aligned LDS address (the XOR addressing of
    // the MFMA operands needs address bits 0-7 of every tile base clear)
    unsigned char* smem = smem_raw + ((256u - (lds_addr(smem_raw) & 255u)) & 255u);
    int* pages = reinterpret_cast<int*>(smem + kRingBytes);
    long long* s_scan = reinterpret_cast<long long*>(smem + kRingBytes + kPageCap * 4);  // kWaves entries
    long long* s_pref = s_scan + kWaves;
    const int NHG = p.Hkv;  // one KV head per workgroup

    run_schedule(p, NHG, s_pref, s_scan, [&](int rg) { return group_visible<KVM, RM>(p, rg); },
                 [&](int rg, int hg, long long v0, long long v1, bool fin, int slot, long long) {
                     chunk_piece<DT, QM, KVM, P2, RM>(p, smem, pages, rg, hg, v0, v1, fin, slot);
                 });
}

size_t lds_bytes(int nrows) {
    return 256 + (size_t)kRingBytes + (size_t)kPageCap * 4 + (size_t)(kWaves + nrows + 1) * sizeof(long long);
}

// ---- varlen row groups ----------------------------------------------------------
//
// Token t of a varlen call belongs to the first sequence i with
// t < cu_seqlens_q[i + 1], or to sequence 0 when there is none (the decode
// path's rule, varlen_paged_kernel_v21.cuh:40-47).  With M_i the running
// maximum of cu_seqlens_q[1 .. i + 1], sequence i's tokens are therefore
// [max(0, M_{i-1}), min(T, M_i)) (M_{-1} = 0), and the tokens from M_{W-1} on
// form one more run, of sequence 0 -- also for tables that are not
// non-decreasing.  Each run is cut into groups of kTokBlk tokens.  One
// workgroup writes entry g = {first token, tokens, sequence, 0} for every
// group, and {0, 0, 0, 0} for the entries from the group count up to gmax
// (the host's bound T / kTokBlk + W + 1: a run of n tokens makes at most
// n / kTokBlk + 1 groups).
constexpr int kVgThreads = 1024;

__device__ inline int block_scan_excl(int v, int* s_part, bool is_max) {
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int ident = is_max ? INT_MIN : 0;
    int incl = v;
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
        const int o = __shfl_up(incl, d, kWave);
        if (lane >= d) incl = is_max ? (o > incl ? o : incl) : incl + o;
    }
    if (lane == 63) s_part[wv] = incl;
    __syncthreads();
    int before = ident;
    for (int i = 0; i < wv; ++i) before = is_max ? (s_part[i] > before ? s_part[i] : before) : before + s_part[i];
    const int excl_lane = __shfl_up(incl, 1, kWave);
    const int mine = lane == 0 ? ident : excl_lane;
    __syncthreads();
    return is_max ? (mine > before ? mine : before) : before + mine;
}

__global__ __launch_bounds__(kVgThreads) void dv_varlen_groups(const int* cu, int W, int T, int gmax, int4* groups) {
    __shared__ int s_m[kVarlenChunkMaxW];       // M_i
    __shared__ int s_base[kVarlenChunkMaxW + 2];  // first group of run i (runs 0 .. W), then the total
    __shared__ int s_part[kVgThreads / kWave];
    const int tid = threadIdx.x;
    // running maximum of cu[1 .. W], each thread over a contiguous block of sequences
    const int per = (W + kVgThreads - 1) / kVgThreads;
    const int i0 = tid * per < W ? tid * per : W, i1 = i0 + per < W ? i0 + per : W;
    int mx = INT_MIN;
    for (int i = i0; i < i1; ++i) {
        const int c = cu[i + 1];
        mx = c > mx ? c : mx;
        s_m[i] = mx;
    }
    const int before = block_scan_excl(mx, s_part, true);
    for (int i = i0; i < i1; ++i) s_m[i] = s_m[i] > before ? s_m[i] : before;
    __syncthreads();
    // run i (i < W: sequence i; i == W: the tokens past M_{W-1}) = [a, b)
    auto run = [&](int i, int& a, int& b) {
        a = i == 0 ? 0 : (s_m[i - 1] > 0 ? s_m[i - 1] : 0);
        b = i == W ? T : (s_m[i] < T ? s_m[i] : T);
    };
    const int per1 = (W + 1 + kVgThreads - 1) / kVgThreads;
    const int j0 = tid * per1 < W + 1 ? tid * per1 : W + 1, j1 = j0 + per1 < W + 1 ? j0 + per1 : W + 1;
    int cnt = 0;
    for (int i = j0; i < j1; ++i) {
        int a, b;
        run(i, a, b);
        const int c = b > a ? (b - a + kTokBlk - 1) / kTokBlk : 0;
        s_base[i] = c;
        cnt += c;
    }
    int acc = block_scan_excl(cnt, s_part, false);
    for (int i = j0; i < j1; ++i) {
        const int c = s_base[i];
        s_base[i] = acc;
        acc += c;
    }
    if (tid == kVgThreads - 1) s_base[W + 1] = acc;
    __syncthreads();
    const int total = s_base[W + 1];
    for (int gi = tid; gi < gmax; gi += kVgThreads) {
        int4 e = {0, 0, 0, 0};
        if (gi < total) {
            // the last run whose first group is <= gi (it has groups: the next run's first is larger)
            int lo = 0, hi = W;
            while (lo < hi) {
                const int mid = (lo + hi + 1) >> 1;
                if (s_base[mid] <= gi) lo = mid;
                else hi = mid - 1;
            }
            int a, b;
            run(lo, a, b);
            const int t0 = a + (gi - s_base[lo]) * kTokBlk;
            e.x = t0;
            e.y = b - t0 < kTokBlk ? b - t0 : kTokBlk;
            e.z = lo == W ? 0 : lo;
        }
        groups[gi] = e;
    }
}

template <int DT, int QM, int KVM, bool P2, int RM>
hipError_t launch1(DecodeParams p, int device, int cus, long long cap, hipStream_t stream) {
    static std::atomic<unsigned long long> attr_done{0};
    hipError_t ea = once_per_device(attr_done, device, [] {
        return hipFuncSetAttribute(reinterpret_cast<const void*>(&dv_chunk<DT, QM, KVM, P2, RM>),
                                   hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds_bytes(kMaxRows));
    });
    if (ea != hipSuccess) return ea;
    const size_t lds = lds_bytes(p.nrows);
    long long nwg = cus;  // one eight-wave workgroup per CU (LDS ring 96 KiB)
    if (nwg > cap) nwg = cap;
    p.nwg = nwg < 1 ? 1 : (int)nwg;
    hipLaunchKernelGGL((dv_chunk<DT, QM, KVM, P2, RM>), dim3(p.nwg), dim3(kThreads), lds, stream, p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((dv_merge_chunk<DT, RM>), dim3(p.nrows * p.Hkv * kTokBlk), dim3(256), 0, stream, p);
    return hipGetLastError();
}

template <int DT, int QM, int KVM, int RM>
hipError_t launch(DecodeParams p, int device, int cus, long long cap, hipStream_t stream) {
    if constexpr (DT == kF32) {
        return launch_chunk32(QM, KVM, RM, p, device, cus, cap, stream);
    } else {
        if constexpr (KVM == kKvPaged)
            if (p.bs_shift >= 0) return launch1<DT, QM, KVM, true, RM>(p, device, cus, cap, stream);
        return launch1<DT, QM, KVM, false, RM>(p, device, cus, cap, stream);
    }
}

}  // namespace chunk

namespace {
int chunk_cus(int device) { return device_cu_count(device); }

// Workspace of the chunk path for `groups` row groups: partial slots, merge
// directory, and (varlen) the group table.
struct ChunkWs {
    size_t part, dir, vgroups, total;
};

ChunkWs chunk_ws(long long groups, int Hkv, int device, bool varlen) {
    const long long rows = groups < kMaxRows ? groups : kMaxRows;
    const long long nseg = rows * Hkv;
    const long long slot_floats = (long long)chunk::kTokBlk * kGqa * (kHeadDim + 1);
    ChunkWs l;
    l.part = ((size_t)((chunk_cus(device) + nseg) * slot_floats * 4) + 255) & ~(size_t)255;
    l.dir = ((size_t)(nseg * 2 * 4) + 255) & ~(size_t)255;
    l.vgroups = varlen ? (size_t)groups * 16 : 0;
    l.total = l.part + l.dir + l.vgroups;
    return l;
}

long long varlen_gmax(int T, int W) { return (long long)T / chunk::kTokBlk + W + 1; }

// The chunk launches over `groups` row groups, kMaxRows at a time.
template <int RM>
hipError_t launch_groups(int dtype, int qmode, int kvmode, DecodeParams p, long long groups_total,
                         long long max_keys_per_group, const ChunkWs& l, void* workspace, hipStream_t stream) {
    int device = 0;
    hipError_t e = hipGetDevice(&device);
    if (e != hipSuccess) return e;
    const int cus = chunk_cus(device);
    p.hpw = 1;
    p.slot_floats = chunk::kTokBlk * kGqa * (kHeadDim + 1);
    p.part = reinterpret_cast<float*>(workspace);
    p.dir = reinterpret_cast<int*>(reinterpret_cast<unsigned char*>(workspace) + l.part);
    p.piece_cost = chunk::kPieceCost;
    // odd workgroups (odd XCD of each pair) take shorter chunks, as in the decode
    // split; 30 per mille measured best on configuration 5
    static const int skew = env_per_mille("DVATTN_CHUNK_SKEW_PM", 30);
    p.skew_pm = skew;
    for (long long g0 = 0; g0 < groups_total; g0 += kMaxRows) {
        p.row_begin = (int)g0;
        p.nrows = (int)(groups_total - g0 < kMaxRows ? groups_total - g0 : kMaxRows);
        const long long cap = ((long long)p.nrows * p.Hkv * max_keys_per_group + p.min_keys - 1) / p.min_keys;
        if (RM == kRowVarlen) {
            if (dtype == kBF16 && qmode == kQRotHalf && kvmode == kKvPaged)
                e = chunk::launch<kBF16, kQRotHalf, kKvPaged, RM>(p, device, cus, cap, stream);
            else if (dtype == kF16 && qmode == kQRotHalf && kvmode == kKvPaged)
                e = chunk::launch<kF16, kQRotHalf, kKvPaged, RM>(p, device, cus, cap, stream);
            else if (dtype == kF32 && qmode == kQRotHalf && kvmode == kKvPaged)
                e = chunk::launch<kF32, kQRotHalf, kKvPaged, RM>(p, device, cus, cap, stream);
            else
                e = hipErrorInvalidValue;
        } else {
            if (dtype == kBF16 && qmode == kQRotFull && kvmode == kKvPaged)
                e = chunk::launch<kBF16, kQRotFull, kKvPaged, RM>(p, device, cus, cap, stream);
            else if (dtype == kF16 && qmode == kQRotFull && kvmode == kKvPaged)
                e = chunk::launch<kF16, kQRotFull, kKvPaged, RM>(p, device, cus, cap, stream);
            else if (dtype == kBF16 && qmode == kQPre && kvmode == kKvContig)
                e = chunk::launch<kBF16, kQPre, kKvContig, RM>(p, device, cus, cap, stream);
            else if (dtype == kF16 && qmode == kQPre && kvmode == kKvContig)
                e = chunk::launch<kF16, kQPre, kKvContig, RM>(p, device, cus, cap, stream);
            else if (dtype == kF32 && qmode == kQRotFull && kvmode == kKvPaged)
                e = chunk::launch<kF32, kQRotFull, kKvPaged, RM>(p, device, cus, cap, stream);
            else if (dtype == kF32 && qmode == kQPre && kvmode == kKvContig)
                e = chunk::launch<kF32, kQPre, kKvContig, RM>(p, device, cus, cap, stream);
            else
                e = hipErrorInvalidValue;
        }
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}
}  // namespace

size_t chunk_workspace_bytes(int W, int S, int Hkv, int device) {
    if (W <= 0 || S <= 0 || Hkv <= 0) return 0;
    const long long groups = (long long)W * ((S + chunk::kTokBlk - 1) / chunk::kTokBlk);
    return chunk_ws(groups, Hkv, device, false).total;
}

hipError_t launch_chunk(int dtype, int qmode, int kvmode, const DecodeParams& base, long long max_keys_per_group,
                        void* workspace, size_t ws_bytes, hipStream_t stream) {
    if (base.W <= 0 || base.S <= 0 || base.Hkv <= 0) return hipSuccess;
    int device = 0;
    hipError_t e = hipGetDevice(&device);
    if (e != hipSuccess) return e;
    const long long groups = (long long)base.W * ((base.S + chunk::kTokBlk - 1) / chunk::kTokBlk);
    const ChunkWs l = chunk_ws(groups, base.Hkv, device, false);
    if (ws_bytes < l.total) return hipErrorInvalidValue;
    return launch_groups<kRowWS>(dtype, qmode, kvmode, base, groups, max_keys_per_group, l, workspace, stream);
}

size_t varlen_chunk_workspace_bytes(int T, int W, int Hkv, int device) {
    if (T <= 0 || W <= 0 || Hkv <= 0) return 0;
    return chunk_ws(varlen_gmax(T, W), Hkv, device, true).total;
}

hipError_t launch_varlen_chunk(int dtype, const DecodeParams& base, long long max_keys_per_group, void* workspace,
                               size_t ws_bytes, hipStream_t stream) {
    if (base.T <= 0 || base.W <= 0 || base.Hkv <= 0) return hipSuccess;
    if (base.W > kVarlenChunkMaxW) return hipErrorInvalidValue;
    int device = 0;
    hipError_t e = hipGetDevice(&device);
    if (e != hipSuccess) return e;
    const long long gmax = varlen_gmax(base.T, base.W);
    const ChunkWs l = chunk_ws(gmax, base.Hkv, device, true);
    if (ws_bytes < l.total) return hipErrorInvalidValue;
    DecodeParams p = base;
    int4* groups = reinterpret_cast<int4*>(reinterpret_cast<unsigned char*>(workspace) + l.part + l.dir);
    p.vgroups = reinterpret_cast<const int*>(groups);
    hipLaunchKernelGGL(chunk::dv_varlen_groups, dim3(1), dim3(chunk::kVgThreads), 0, stream, base.cu_q, base.W,
                       base.T, (int)gmax, groups);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    return launch_groups<kRowVarlen>(dtype, kQRotHalf, kKvPaged, p, gmax, max_keys_per_group, l, workspace, stream);
}

}  // namespace dv
