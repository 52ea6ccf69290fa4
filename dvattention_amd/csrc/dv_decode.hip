// gfx950 decode attention with fused query RoPE (paged / varlen / contiguous views).
//
// Restates the operator semantics of src/kernels/paged_kernel_v21.cuh:17-374,
// src/kernels/varlen_paged_kernel_v21.cuh:17-371 and src/kernels/kernel_v21.cuh:17-367
// (reference repository) with an MI355X-first design:
//
//  * One wave owns one KV head and its 16 query heads of one query row, for a
//    contiguous range of that row's visible keys.  A workgroup holds up to four
//    such waves (four KV heads of the same row and key range), so a token's K/V
//    rows for those heads are fetched together.
//  * Scores are computed transposed on MFMA, S^T = K Q^T (16 keys x 16 heads per
//    16x16x32 bf16/f16 MFMA, 4 per 16 keys), so every lane owns one query head:
//    the online softmax needs only two cross-lane reductions per 32 keys and no
//    layout change.  The output is accumulated transposed too, O^T += V^T P^T,
//    with P^T taken straight from the score registers and V^T read from a
//    wave-private LDS tile with the gfx950 transposing LDS read.
//  * The query of each view is rotated once per (row, view) in registers while
//    it is loaded (no rotated-query round trip through HBM).
//  * Work balance: every workgroup computes the same schedule from locations /
//    fragment_lengths: all (row, KV-head-group) segments of visible keys are laid
//    end to end and cut into equal contiguous chunks, one per workgroup.  A
//    segment that one workgroup finishes alone is written straight to the output;
//    otherwise the pieces go to fp32 partial slots (normalised output + base-2
//    log-sum-exp) and dv_merge combines them, as the reference's reduce kernels
//    do (paged_kernel_v21.cuh:307-374).
#include <stdlib.h>

#include "dv_common.h"
#include "dv_device.h"
#include "dv_schedule.h"
#include "dv_stream.h"

namespace dv {

constexpr int kVtStride16 = 288;                 // V tile row (bytes), 16-bit types: 256 + 32 pad
constexpr int kVtStride32 = 528;                 // fp32: 512 + 16 pad
constexpr int kVtBytes16 = kStep * kVtStride16;  // 9216 B per wave
constexpr int kVtBytes32 = kStep * kVtStride32;  // 16896 B per wave

template <int DT> constexpr int vt_bytes() { return DT == kF32 ? kVtBytes32 : kVtBytes16; }

// ---- per-wave K/V staging -----------------------------------------------------

// Page-table window: lane l holds the physical page of logical page wbase + l.
struct PageWin {
    long long wbase;
    int pg;
};

struct KvCtx {
    const unsigned char* k;  // base of this view's K (contig) or the K cache (paged)
    const unsigned char* v;
    long long off;           // paged: logical position of the view's first token
    long long bstride;       // contig: element offset of this row's batch entry
    int L;                   // contig: tokens in the fragment tensor
    int w;
    int hkv;
};

template <int DT, int KVM>
__device__ inline void window_update(const DecodeParams& p, const KvCtx& c, PageWin& win, int l, int l1) {
    if (KVM != kKvPaged) return;
    const long long pf = c.off + l;
    const long long plast = c.off + (l + kStep - 1 < l1 - 1 ? l + kStep - 1 : l1 - 1);
    long long lpf, lpl;
    if (p.bs_shift >= 0) {
        lpf = pf >> p.bs_shift;
        lpl = plast >> p.bs_shift;
    } else {
        lpf = pf >= 0 ? pf / p.bs : -((-pf + p.bs - 1) / p.bs);
        lpl = plast >= 0 ? plast / p.bs : -((-plast + p.bs - 1) / p.bs);
    }
    if (lpf >= win.wbase && lpl < win.wbase + kWave) return;
    win.wbase = lpf;
    const long long lp = lpf + (threadIdx.x & 63);
    win.pg = (lp >= 0 && lp < p.maxB) ? p.bt[(long long)c.w * p.maxB + lp] : -1;
}

// Element offset (same for K and V since E == Ev) of the row holding key `key`
// of the current view, or -1 if the key is not visible / not addressable.
template <int KVM>
__device__ inline long long kv_row(const DecodeParams& p, const KvCtx& c, const PageWin& win,
                                   int key, int l1) {
    if (KVM == kKvPaged) {
        const long long pos = c.off + key;
        long long lp, r;
        if (p.bs_shift >= 0) {
            lp = pos >> p.bs_shift;
            r = pos - (lp << p.bs_shift);
        } else {
            lp = pos >= 0 ? pos / p.bs : -((-pos + p.bs - 1) / p.bs);
            r = pos - lp * p.bs;
        }
        const long long idx = lp - win.wbase;
        const int page = shfl_i(win.pg, (int)(idx & 63));
        const bool ok = key < l1 && idx >= 0 && idx < kWave && lp < p.maxB && page >= 0 && page < p.nblocks;
        const long long off = (((long long)page * p.bs + r) * p.Hkv + c.hkv) * kHeadDim;
        return ok ? off : -1;
    } else {
        const long long off = c.bstride + ((long long)c.hkv * c.L + key) * kHeadDim;
        return key < l1 ? off : -1;
    }
}

struct SoftState {
    f32x4 o[8];   // O^T: lane (g, n) holds dims c*16 + g*4 + i of head n
    float m;      // running max of base-2 scores (same in the 4 lane groups)
    float l;      // this lane's partial sum of exp2(score - m)
};

// Online softmax update for one step, given the two 16-key S^T blocks.
// Returns the unnormalised probabilities (8 per lane) in pr.
__device__ inline void softmax_step(SoftState& st, const f32x4& s0, const f32x4& s1, uint32_t mask,
                                    float l2scale, float (&pr)[8]) {
    softmax32(st.o, st.m, st.l, s0, s1, mask, l2scale, pr);
}

// fp32: lane (g, m) loads dims [c*16 + g*4, +4), c = 0..7, of keys m and 16+m.
struct Kv32 {
    f32x4 k[2][8];
    f32x4 v[2][8];
    uint32_t mask;
};

template <int KVM>
__device__ inline void issue32(const DecodeParams& p, const KvCtx& c, const PageWin& win, Kv32& b,
                               int l, int l1) {
    const int lane = threadIdx.x & 63;
    const int g = lane >> 4, m = lane & 15;
    bool okb[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
        const long long row = kv_row<KVM>(p, c, win, l + kb * 16 + m, l1);
        okb[kb] = row >= 0;
        const unsigned char* kp = okb[kb] ? c.k + (row + g * 4) * 4 : g_zero_row + g * 16;
        const unsigned char* vp = okb[kb] ? c.v + (row + g * 4) * 4 : g_zero_row + g * 16;
#pragma unroll
        for (int cc = 0; cc < 8; ++cc) b.k[kb][cc] = ld16f_nt(kp + cc * 64);
#pragma unroll
        for (int cc = 0; cc < 8; ++cc) b.v[kb][cc] = ld16f_nt(vp + cc * 64);
    }
    b.mask = (uint32_t)(ballot(okb[0]) & 0xffffu) | ((uint32_t)(ballot(okb[1]) & 0xffffu) << 16);
}

__device__ inline void compute32(SoftState& st, const Kv32& b, const f32x4 (&qB)[8], unsigned char* vt,
                                 float l2scale) {
    const int lane = threadIdx.x & 63;
    const int g = lane >> 4, m = lane & 15, n = lane & 15;
    f32x4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int cc = 0; cc < 8; ++cc)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            s0 = Tr<kF32>::mma1(b.k[0][cc][j], qB[cc][j], s0);
            s1 = Tr<kF32>::mma1(b.k[1][cc][j], qB[cc][j], s1);
        }
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int cc = 0; cc < 8; ++cc)
            *reinterpret_cast<f32x4*>(vt + (kb * 16 + m) * kVtStride32 + (cc * 16 + g * 4) * 4) = b.v[kb][cc];
    compiler_fence();
    float pr[8];
    softmax_step(st, s0, s1, b.mask, l2scale, pr);
    // O^T += V^T P^T, 4 keys per MFMA: k = g <-> key kb*16 + g*4 + i
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float* vrow = reinterpret_cast<const float*>(vt + (kb * 16 + g * 4 + i) * kVtStride32);
            const float pb = pr[kb * 4 + i];
#pragma unroll
            for (int cc = 0; cc < 8; ++cc) st.o[cc] = Tr<kF32>::mma1(vrow[cc * 16 + n], pb, st.o[cc]);
        }
    compiler_fence();
}

// ---- one wave: one KV head over visible keys [v0, v1) of one row ---------------

template <int DT, int QM, int KVM, int RM>
__device__ void process_piece(const DecodeParams& p, unsigned char* vt, int row, int hkv, long long v0,
                              long long v1, bool final_out, int slot, int wv, long long row_keys) {
    const int lane = threadIdx.x & 63;
    const int g = lane >> 4, n = lane & 15;

    int w;
    if (RM == kRowVarlen) w = varlen_seq(p, row);
    else w = row / p.S;

    SoftState st;
#pragma unroll
    for (int c = 0; c < 8; ++c) st.o[c] = f32x4{0.f, 0.f, 0.f, 0.f};
    st.m = -DV_INF;
    st.l = 0.0f;

    PageWin win;
    win.wbase = -(1ll << 60);
    win.pg = -1;

    // P: visible keys of the earlier views; off: logical position of view f
    // (paged): sum of the earlier fragment_lengths
    auto one_view = [&](int f, int vis, long long P, long long off) {
        const long long a = v0 > P ? v0 : P;
        const long long bnd = v1 < P + vis ? v1 : P + vis;
        {
            const int l0 = (int)(a - P), l1 = (int)(bnd - P);
            KvCtx c;
            c.w = w;
            c.hkv = hkv;
            if (KVM == kKvPaged) {
                c.k = reinterpret_cast<const unsigned char*>(p.kc);
                c.v = reinterpret_cast<const unsigned char*>(p.vc);
                c.off = off;
                c.bstride = 0;
                c.L = 0;
            } else {
                const FragDesc& fd = frag<KVM>(p, f);
                c.k = reinterpret_cast<const unsigned char*>(fd.k);
                c.v = reinterpret_cast<const unsigned char*>(fd.v);
                c.off = 0;
                c.bstride = fd.bstride * w;
                c.L = fd.L;
            }
            static_assert(DT == kF32, "16-bit types use dv_stream");
            f32x4 qB[8];
            // the first stage's K/V loads go out before the query's, so the two
            // round trips overlap
            Kv32 b;
            window_update<DT, KVM>(p, c, win, l0, l1);
            issue32<KVM>(p, c, win, b, l0, l1);
            load_q32<QM, RM>(p, row, f, hkv, qB);
            compute32(st, b, qB, vt, p.l2scale);
            for (int l = l0 + kStep; l < l1; l += kStep) {
                window_update<DT, KVM>(p, c, win, l, l1);
                issue32<KVM>(p, c, win, b, l, l1);
                compute32(st, b, qB, vt, p.l2scale);
            }
        }
    };
    if (p.F == 1) {
        // one view: its visible keys are the row's, counted by the schedule
        if (row_keys > 0 && v1 > v0) one_view(0, (int)row_keys, 0ll, 0ll);
    } else {
        for_views<KVM, RM>(p, row, v0, v1, one_view);
    }

    // epilogue: total over the four lane groups, normalise, base-2 LSE
    const float lt = rows4_sum(st.l);
    const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
    const int h = hkv * kGqa + n;
    if (final_out) {
        using raw = typename Tr<DT>::raw;
        raw* o;
        if (RM == kRowVarlen) {
            o = reinterpret_cast<raw*>(p.out) + ((long long)row * p.Hq + h) * kHeadDim;
        } else {
            const int s = row - w * p.S;
            o = reinterpret_cast<raw*>(p.out) + (((long long)w * p.Hq + h) * p.S + s) * kHeadDim;
        }
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            const int d = c * 16 + g * 4;
            if constexpr (DT == kF32) {
                *reinterpret_cast<f32x4*>(o + d) = st.o[c] * inv;
            } else {
                const u32x2 pk = {pack2<DT>(st.o[c][0] * inv, st.o[c][1] * inv),
                                  pack2<DT>(st.o[c][2] * inv, st.o[c][3] * inv)};
                *reinterpret_cast<u32x2*>(o + d) = pk;
            }
        }
    } else {
        store_partial<DT>(p.part + (long long)slot * p.slot_floats, p.hpw * kGqa, wv * kGqa + n, g, st.o, inv,
                          lt > 0.0f ? st.m + log2f(lt) : -DV_INF);
    }
}

// ---- work schedule: run_schedule (dv_schedule.h) ------------------------------------


// ---- the fp32 decode kernel --------------------------------------------------------

template <int DT, int QM, int KVM, int RM>
__global__ __launch_bounds__(256) void dv_decode(const DecodeParams p) {
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ long long s_scan[4];
    const int wv = threadIdx.x >> 6;
    const int HPW = p.hpw;
    long long* s_pref = reinterpret_cast<long long*>(smem + HPW * vt_bytes<DT>());
    unsigned char* vt = smem + wv * vt_bytes<DT>();
    run_schedule(p, p.Hkv / HPW, s_pref, s_scan, [&](int row) { return row_visible<KVM, RM>(p, row); },
                 [&](int row, int hg, long long v0, long long v1, bool fin, int slot, long long rk) {
        if (wv < HPW) process_piece<DT, QM, KVM, RM>(p, vt, row, hg * HPW + wv, v0, v1, fin, slot, wv, rk);
    });
}

// ---- the 16-bit streaming decode kernel --------------------------------------------
//
// Same operator and schedule as dv_decode; K/V reach LDS by direct-to-LDS loads
// (global_load_lds_dwordx4) into a two-stage ring private to each wave, so no
// VGPRs are held by loads in flight and the next stage streams in while the
// current one runs on MFMA.  A stage is 32 keys: an 8 KiB K tile and an 8 KiB V
// tile, each key row 256 B with its 16-byte pieces XOR-swizzled (K: piece ^
// (key & 15) for the row-wise ds_read_b128 of the MFMA A operand; V: piece ^
// ((key & 7) << 1) for the transposing reads) so both reads are free of bank
// conflicts.  Completion is tracked with explicit vmcnt waits (16 loads per
// stage and wave); the physical pages of the current key range sit in a
// per-wave LDS page cache, so the loop issues no other vector-memory operation.

// Output row of query head h of decode row `row` (varlen rows: packed tokens).
template <int DT, int RM>
__device__ inline typename Tr<DT>::raw* out_row_ptr(const DecodeParams& p, int row, int h) {
    using raw = typename Tr<DT>::raw;
    if (RM == kRowVarlen) return reinterpret_cast<raw*>(p.out) + ((long long)row * p.Hq + h) * kHeadDim;
    const int w = row / p.S, s = row - (row / p.S) * p.S;
    return reinterpret_cast<raw*>(p.out) + (((long long)w * p.Hq + h) * p.S + s) * kHeadDim;
}

namespace stream {

// One stage on MFMA: S^T = K Q^T from the K tile, online softmax, O^T += V^T P^T
// with V^T from the transposing reads of the V tile.
template <int DT>
__device__ inline void compute(SoftState& st, const unsigned char* kt, const unsigned char* vt, uint32_t mask,
                               const u32x4 (&qB)[4], float l2scale) {
    const int lane = threadIdx.x & 63;
    const int g = lane >> 4, n = lane & 15;
    u32x4 kA[2][4];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int cc = 0; cc < 4; ++cc) {
            const int key = kb * 16 + n;
            kA[kb][cc] = *reinterpret_cast<const u32x4*>(kt + key * 256 + (((cc * 4 + g) ^ (key & 15)) * 16));
        }
    f32x4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int cc = 0; cc < 4; ++cc) {
        s0 = Tr<DT>::mma(kA[0][cc], qB[cc], s0);
        s1 = Tr<DT>::mma(kA[1][cc], qB[cc], s1);
    }
    // V^T operand for dims [c*16, +16): block lane sl -> key g*4 + sl/4 (and +16),
    // dims c*16 + (sl%4)*4; the transposed read hands lane n V[key][c*16 + n].
    u32x4 vA[8];
    {
        const int sl = lane & 15;
        const int k0 = g * 4 + (sl >> 2);
        const int k1 = k0 + 16;
        const int hb = (sl & 1) * 8;
#pragma unroll
        for (int cc = 0; cc < 8; ++cc) {
            const int piece = cc * 2 + ((sl & 3) >> 1);
            const u32x2 a0 = lds_read_tr16(vt + k0 * 256 + ((piece ^ ((k0 & 7) << 1)) * 16) + hb);
            const u32x2 a1 = lds_read_tr16(vt + k1 * 256 + ((piece ^ ((k1 & 7) << 1)) * 16) + hb);
            vA[cc] = u32x4{a0[0], a0[1], a1[0], a1[1]};
        }
    }
    float pr[8];
    softmax32<false>(st.o, st.m, st.l, s0, s1, mask, l2scale, pr);
    // P^T operand: k = g*8 + jj <-> key (jj/4)*16 + g*4 + jj%4
    const POperand pB = p_operands<DT>(pr, st.l);
#pragma unroll
    for (int cc = 0; cc < 8; ++cc) st.o[cc] = Tr<DT>::mma(vA[cc], pB.hi, st.o[cc]);
    if constexpr (DT == kF16)
#pragma unroll
        for (int cc = 0; cc < 8; ++cc) st.o[cc] = Tr<DT>::mma(vA[cc], pB.lo, st.o[cc]);
    mfma_settle(st.o);
}

constexpr int kStreamViews = 4;  // views of one piece streamed back to back

// The visible keys [v0, v1) of up to four paged views of one row (vm: their
// lanes in the view table t) streamed back to back: the views' page ids (one
// shared page cache) and rotated queries are loaded first, then one stage loop
// runs over the concatenated key ranges, so a view boundary does not drain the
// two-stage ring.  Returns false, having done nothing, when the views' pages
// do not fit the page cache.
template <int DT, int QM, int RM>
__device__ bool views_stream(const DecodeParams& p, unsigned char* wlds, int row, int w, int hkv, long long v0,
                             long long v1, uint64_t vm, const ViewTab& t, SoftState& st) {
    const int lane = threadIdx.x & 63;
    const uint32_t ring = __builtin_amdgcn_readfirstlane(lds_addr(wlds));
    int* pc = reinterpret_cast<int*>(wlds + kRing * kStage);
    int vf[kStreamViews], l0[kStreamViews], l1[kStreamViews], ns[kStreamViews], pcb[kStreamViews + 1];
    int voff[kStreamViews], lpa[kStreamViews];
    int npages = 0, N = 0;
    uint64_t m = vm;
#pragma unroll
    for (int j = 0; j < kStreamViews; ++j) {
        const bool has = m != 0;
        const int f = has ? __builtin_ctzll(m) : 0;
        m &= m - 1;
        const int vis = __shfl(t.vis, f, kWave);
        const long long P = __shfl(t.P, f, kWave);
        const long long off = __shfl(t.off, f, kWave);
        const long long a = v0 > P ? v0 : P;
        const long long b = v1 < P + vis ? v1 : P + vis;
        vf[j] = f;
        l0[j] = has ? (int)(a - P) : 0;
        l1[j] = has ? (int)(b - P) : 0;
        ns[j] = (l1[j] - l0[j] + kStep - 1) / kStep;
        N += ns[j];
        voff[j] = (int)off;
        lpa[j] = 0;
        pcb[j] = npages;
        if (has) {
            uint32_t la, lz, r;
            const int pa = voff[j] + l0[j], pz = voff[j] + l1[j] - 1;
            page_split(p, pa > 0 ? (uint32_t)pa : 0u, la, r);
            page_split(p, pz > 0 ? (uint32_t)pz : 0u, lz, r);
            lpa[j] = (int)la;
            npages += (int)(lz - la) + 1;
        }
    }
    pcb[kStreamViews] = npages;
    if (npages > kPc) return false;
    // query loads issued before the page ids' (their round trips overlap): the
    // row's query runs once and every view's cos/sin run (R of 32 or 64),
    // rotated per view once the first stages are issued, so the first compute
    // waits for stage 0 alone
    const bool qsplit = q_split_narrow<QM>(p);
    u32x4 qrow[4];
    QCs1 vcs[kStreamViews];
    if (qsplit) {
        fetch_qrow16<DT, QM, RM>(p, row, hkv, qrow);
#pragma unroll
        for (int j = 0; j < kStreamViews; ++j)
            if (ns[j] > 0) fetch_cs16_narrow<QM>(p, row, vf[j], vcs[j]);
    }
    // the views' page ids in one fill: entry i belongs to the last view j with
    // pcb[j] <= i (selects with constant indices, no dynamically indexed array)
    fill_pages(p, p.bt + (long long)w * p.maxB, pc, npages, [&](int i) {
        uint32_t lp = (uint32_t)lpa[0] + (uint32_t)i;
#pragma unroll
        for (int j = 1; j < kStreamViews; ++j)
            if (i >= pcb[j]) lp = (uint32_t)lpa[j] + (uint32_t)(i - pcb[j]);
        return lp;
    });

    // issue cursor: view ji, next key li; the view's parameters are copied out of
    // the per-view arrays with constant indices (no dynamically indexed arrays,
    // which would live in scratch memory)
    View vi;
    vi.hkv = hkv;
    vi.k = reinterpret_cast<const unsigned char*>(p.kc);
    vi.v = reinterpret_cast<const unsigned char*>(p.vc);
    vi.off = voff[0];
    vi.lp0 = lpa[0];
    vi.b = l1[0];
    const int* pci = pc;
    int ji = 0, li = l0[0];
    auto advance = [&]() {
        li += kStep;
        if (li >= vi.b) {
            ++ji;
#pragma unroll
            for (int k = 1; k < kStreamViews; ++k)
                if (k == ji) {
                    vi.off = voff[k];
                    vi.lp0 = lpa[k];
                    vi.b = l1[k];
                    pci = pc + pcb[k];
                    li = l0[k];
                }
        }
    };
    uint32_t m0 = issue<kKvPaged>(p, vi, pci, ring, li);
    advance();
    uint32_t m1 = 0;
    if (N > 1) {
        m1 = issue<kKvPaged>(p, vi, pci, ring + kStage, li);
        advance();
    }
    // rotated queries of every view while the first stages are in flight, then
    // settled (a query load pending at the loop would make the compiler wait
    // for all vector memory in every step)
    u32x4 q[kStreamViews][4];
#pragma unroll
    for (int j = 0; j < kStreamViews; ++j) {
        if (ns[j] > 0) {
            if (qsplit) rotate_q16_narrow<DT>(p, qrow, vcs[j], q[j]);
            else load_q16<DT, QM, RM>(p, row, vf[j], hkv, q[j]);
        } else {
#pragma unroll
            for (int cc = 0; cc < 4; ++cc) q[j][cc] = u32x4{0u, 0u, 0u, 0u};
        }
    }
#pragma unroll
    for (int j = 0; j < kStreamViews; ++j)
#pragma unroll
        for (int cc = 0; cc < 4; ++cc) asm volatile("" : "+v"(q[j][cc]));
    u32x4 qc[4];
#pragma unroll
    for (int cc = 0; cc < 4; ++cc) qc[cc] = q[0][cc];
    int jc = 0, left = ns[0];
    for (int s = 0; s < N; ++s) {
        if (s + 1 < N) wait_vmcnt<16>();
        else wait_vmcnt<0>();
        const unsigned char* kt = wlds + (s & 1) * kStage;
        compute<DT>(st, kt, kt + kTile, (s & 1) ? m1 : m0, qc, p.l2scale);
        if (s + 2 < N) {
            lds_wait();  // the slot's reads are complete before it is refilled
            const uint32_t mk = issue<kKvPaged>(p, vi, pci, ring + (uint32_t)((s & 1) * kStage), li);
            advance();
            if (s & 1) m1 = mk;
            else m0 = mk;
        }
        if (--left == 0 && s + 1 < N) {
            ++jc;
#pragma unroll
            for (int k = 1; k < kStreamViews; ++k)
                if (k == jc) {
#pragma unroll
                    for (int cc = 0; cc < 4; ++cc) qc[cc] = q[k][cc];
                    left = ns[k];
                }
        }
    }
    lds_wait();
    return true;
}

// One wave: KV head hkv over visible keys [v0, v1) of one row.  wlds: this
// wave's LDS (ring, then page cache).  MV: paged rows of several views stream
// them back to back (a separate instantiation, so single-view launches keep
// their own register allocation).
template <int DT, int QM, int KVM, int RM, bool MV>
__device__ void piece(const DecodeParams& p, unsigned char* wlds, int row, int hkv, long long v0, long long v1,
                      bool final_out, int slot, int wv, long long row_keys) {
    const int lane = threadIdx.x & 63;
    const int g = lane >> 4, n = lane & 15;
    const uint32_t ring = __builtin_amdgcn_readfirstlane(lds_addr(wlds));
    int* pc = reinterpret_cast<int*>(wlds + kRing * kStage);

    // the row's sequence (varlen: the first 64 sequence bounds) and its view
    // table are loaded in one round trip; one view needs no loads: its visible
    // keys are the row's, counted by the schedule
    int cu = 0x7fffffff;
    if (RM == kRowVarlen) cu = lane < p.W ? p.cu_q[lane + 1] : 0x7fffffff;
    ViewTab t;
    if (p.F == 1) {
        t.vis = lane == 0 ? (int)row_keys : 0;
        t.P = 0;
        t.off = 0;
    } else if (p.F <= kWave) {
        t = view_table<KVM, RM>(p, row);
    }
    int w;
    if (RM == kRowVarlen) {
        const uint64_t b = ballot(lane < p.W && row < cu);
        w = b ? __builtin_ctzll(b) : varlen_seq(p, row);
    } else {
        w = row / p.S;
    }

    SoftState st;
#pragma unroll
    for (int c = 0; c < 8; ++c) st.o[c] = f32x4{0.f, 0.f, 0.f, 0.f};
    st.m = -DV_INF;
    st.l = 0.0f;

    // P: visible keys of the earlier views; off: logical position of view f
    // (paged): sum of the earlier fragment_lengths
    auto one_view = [&](int f, int vis, long long P, long long off) {
        const long long a = v0 > P ? v0 : P;
        const long long bnd = v1 < P + vis ? v1 : P + vis;
        {
            const int l0 = (int)(a - P), l1 = (int)(bnd - P);
            View v;
            v.hkv = hkv;
            if (KVM == kKvPaged) {
                v.k = reinterpret_cast<const unsigned char*>(p.kc);
                v.v = reinterpret_cast<const unsigned char*>(p.vc);
                v.off = (int)off;
            } else {
                const FragDesc& fd = frag<KVM>(p, f);
                const long long base = (fd.bstride * w + (long long)hkv * fd.L * kHeadDim) * 2;
                v.k = reinterpret_cast<const unsigned char*>(fd.k) + base;
                v.v = reinterpret_cast<const unsigned char*>(fd.v) + base;
                v.off = 0;
            }
            v.lp0 = 0;
            u32x4 qB[4];
            bool have_q = false;
            // query loads issued before the page ids' (their round trips overlap)
            const bool qsplit = q_split<QM>(p);
            QRaw qr;
            if (qsplit) fetch_q16<DT, QM, RM>(p, row, f, hkv, qr);
            // sub-ranges whose pages fit the page cache
            const long long span = KVM == kKvPaged ? (long long)(kPc - 1) * p.bs : (1ll << 30);
            for (int sa = l0; sa < l1;) {
                const int sb = (long long)l1 - sa > span ? (int)(sa + span) : l1;
                v.b = sb;
                if (KVM == kKvPaged) {
                    uint32_t lpa, lpz, r;
                    const int pa = v.off + sa, pz = v.off + sb - 1;
                    page_split(p, pa > 0 ? (uint32_t)pa : 0u, lpa, r);
                    page_split(p, pz > 0 ? (uint32_t)pz : 0u, lpz, r);
                    v.lp0 = (int)lpa;
                    const int need = (int)(lpz - lpa) + 1;
                    fill_pages(p, p.bt + (long long)w * p.maxB, pc, need,
                               [&](int i) { return lpa + (uint32_t)i; });
                }
                const int n_st = (sb - sa + kStep - 1) / kStep;
                uint32_t m0 = issue<KVM>(p, v, pc, ring, sa);
                uint32_t m1 = 0;
                if (n_st > 1) m1 = issue<KVM>(p, v, pc, ring + kStage, sa + kStep);
                if (!have_q) {
                    // rotated once per (row, view) while the first stages are in flight
                    if (qsplit) rotate_q16<DT, QM>(qr, qB);
                    else load_q16<DT, QM, RM>(p, row, f, hkv, qB);
                    // settle the query loads here: a load still pending in qB at the loop
                    // would make the compiler wait for all vector memory in every step
#pragma unroll
                    for (int cc = 0; cc < 4; ++cc) asm volatile("" : "+v"(qB[cc]));
                    have_q = true;
                }
                for (int s = 0; s < n_st; ++s) {
                    if (s + 1 < n_st) wait_vmcnt<16>();
                    else wait_vmcnt<0>();
                    const unsigned char* kt = wlds + (s & 1) * kStage;
                    compute<DT>(st, kt, kt + kTile, (s & 1) ? m1 : m0, qB, p.l2scale);
                    if (s + 2 < n_st) {
                        lds_wait();  // the slot's reads are complete before it is refilled
                        const uint32_t mk = issue<KVM>(p, v, pc, ring + (uint32_t)((s & 1) * kStage),
                                                       sa + (s + 2) * kStep);
                        if (s & 1) m1 = mk;
                        else m0 = mk;
                    }
                }
                lds_wait();
                sa = sb;
            }
        }
    };
    if (p.F <= kWave) {
        uint64_t vm = ballot(lane < p.F && t.vis > 0 && t.P < v1 && t.P + t.vis > v0);
        const int nv = __builtin_popcountll(vm);
        bool done = false;
        if constexpr (MV && KVM == kKvPaged) {
            if (nv >= 2 && nv <= kStreamViews) done = views_stream<DT, QM, RM>(p, wlds, row, w, hkv, v0, v1, vm, t, st);
        }
        while (!done && vm) {
            const int f = __builtin_ctzll(vm);
            vm &= vm - 1;
            one_view(f, __shfl(t.vis, f, kWave), __shfl(t.P, f, kWave), __shfl(t.off, f, kWave));
        }
    } else {
        for_views<KVM, RM>(p, row, v0, v1, one_view);
    }

    // epilogue: total over the four lane groups, normalise, base-2 LSE
    const float lt = rows4_sum(st.l);
    const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
    const int h = hkv * kGqa + n;
    if (final_out) {
        using raw = typename Tr<DT>::raw;
        raw* o;
        if (RM == kRowVarlen) {
            o = reinterpret_cast<raw*>(p.out) + ((long long)row * p.Hq + h) * kHeadDim;
        } else {
            const int s = row - w * p.S;
            o = reinterpret_cast<raw*>(p.out) + (((long long)w * p.Hq + h) * p.S + s) * kHeadDim;
        }
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            const u32x2 pk = {pack2<DT>(st.o[c][0] * inv, st.o[c][1] * inv),
                              pack2<DT>(st.o[c][2] * inv, st.o[c][3] * inv)};
            *reinterpret_cast<u32x2*>(o + c * 16 + g * 4) = pk;
        }
    } else {
        store_partial<DT>(p.part + (long long)slot * p.slot_floats, p.hpw * kGqa, wv * kGqa + n, g, st.o, inv,
                          lt > 0.0f ? st.m + log2f(lt) : -DV_INF);
    }
}

}  // namespace stream

template <int DT, int QM, int KVM, int RM, bool MV>
__global__ __launch_bounds__(256) void dv_stream(const DecodeParams p) {
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ long long s_scan[4];
    const int wv = threadIdx.x >> 6;
    const int HPW = p.hpw;
    long long* s_pref = reinterpret_cast<long long*>(smem + HPW * stream::kWaveLds);
    unsigned char* wlds = smem + wv * stream::kWaveLds;
    run_schedule<true>(p, p.Hkv / HPW, s_pref, s_scan, [&](int row) { return row_visible<KVM, RM>(p, row); },
                       [&](int row, int hg, long long v0, long long v1, bool fin, int slot, long long rk) {
        if (wv < HPW) stream::piece<DT, QM, KVM, RM, MV>(p, wlds, row, hg * HPW + wv, v0, v1, fin, slot, wv, rk);
    });
}

// ---- split merge -------------------------------------------------------------------

// Block (segment, KV head, quarter of the head dims) with four waves: thread
// t of a wave handles query head t/4, dims [q*32 + (t%4)*8, +8).  count == 1:
// already final; count == 0: no visible key -> zeros (paged_kernel_v21.cuh:318);
// otherwise the base-2-LSE-weighted sum of the pieces' normalised outputs
// (merge_runs, paged_kernel_v21.cuh:325-364).  The quarters spread a long
// segment's partials (up to ~40 pieces x 8 KiB per KV head) over four CUs: one
// CU reads at only ~50-100 GB/s, which set the merge time of segments with
// many pieces.  Segments of up to kMergeBatchLong pieces are merged by wave 0
// alone (one round of loads); longer ones by all four waves, wave w taking the
// w-th quarter of the pieces in one round, and wave 0 combines the four
// partial sums (their maxima, weight sums and weighted sums) through LDS --
// a merge kernel lasts as long as its segment with the most pieces.
constexpr int kMergeQuarters = 4;
constexpr int kMergeWaves = 4;

template <int DT, int RM>
__global__ __launch_bounds__(kMergeWaves * kWave) void dv_merge(const DecodeParams p) {
    __shared__ float s_part[kMergeWaves - 1][10][kWave];  // waves 1..3: m, wsum, acc[8] per lane
    const int qi = blockIdx.x % kMergeQuarters;
    const int sw = blockIdx.x / kMergeQuarters;
    const int sg = sw / p.hpw;
    const int wi = sw - sg * p.hpw;
    const int base = p.dir[2 * sg], cnt = p.dir[2 * sg + 1];
    if (cnt == 1) return;
    const int NHG = p.Hkv / p.hpw;
    const int wv = threadIdx.x / kWave, t = threadIdx.x % kWave;
    const int n = t >> 2;
    const int r = sg / NHG, hg = sg - (sg / NHG) * NHG;
    const int d[1] = {qi * 32 + (t & 3) * 8};
    typename Tr<DT>::raw* o = out_row_ptr<DT, RM>(p, p.row_begin + r, (hg * p.hpw + wi) * kGqa + n) + d[0];
    if (cnt <= kMergeBatchLong) {  // uniform: the other waves leave before any barrier
        if (wv != 0) return;
        float v[1][8];
        merge_runs<DT, 1>(p.part, p.slot_floats, p.hpw * kGqa, wi * kGqa + n, d, base, cnt, v);
        store_run8<DT>(o, v[0]);
        return;
    }
    // consecutive quarters of the pieces: with cnt > kMergeBatchLong every
    // quarter is non-empty (3 * ceil(cnt / 4) < cnt), and one round long while
    // cnt <= 4 * kMergeBatchLong
    const int per = (cnt + kMergeWaves - 1) / kMergeWaves;
    const int b0 = wv * per;
    const int c0 = cnt - b0 < per ? cnt - b0 : per;
    float m, wsum, acc[1][8];
    merge_acc_b<DT, 1, kMergeBatchLong>(p.part, p.slot_floats, p.hpw * kGqa, wi * kGqa + n, d, base + b0, c0, m, wsum,
                                        acc);
    if (wv > 0) {
        s_part[wv - 1][0][t] = m;
        s_part[wv - 1][1][t] = wsum;
#pragma unroll
        for (int e = 0; e < 8; ++e) s_part[wv - 1][2 + e][t] = acc[0][e];
    }
    __syncthreads();
    if (wv != 0) return;
    float mw[kMergeWaves], ww[kMergeWaves], M = m;
    mw[0] = m;
    ww[0] = wsum;
#pragma unroll
    for (int w = 1; w < kMergeWaves; ++w) {
        mw[w] = s_part[w - 1][0][t];
        ww[w] = s_part[w - 1][1][t];
        M = fmaxf(M, mw[w]);
    }
    float v[8];
    if (M == -DV_INF) {  // no piece has a visible key
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = 0.0f;
    } else {
        float sc[kMergeWaves], tw = 0.0f;
#pragma unroll
        for (int w = 0; w < kMergeWaves; ++w) {
            sc[w] = exp2f(mw[w] - M);  // a quarter without visible keys (-inf) -> 0
            tw += ww[w] * sc[w];
        }
        const float inv = tw > 0.0f ? 1.0f / tw : 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            float a = acc[0][e] * sc[0];
#pragma unroll
            for (int w = 1; w < kMergeWaves; ++w) a += s_part[w - 1][2 + e][t] * sc[w];
            v[e] = a * inv;
        }
    }
    store_run8<DT>(o, v);
}

// ---- host side --------------------------------------------------------------------

namespace {

thread_local const char* g_site = "";

hipError_t note_site(hipError_t e, const char* site) {
    g_site = site;
    return e;
}

int device_cus(int device) { return device_cu_count(device); }

// workgroups per CU such that about eight waves share a CU
int wgs_per_cu(int hpw) { return 8 / hpw; }

// The decode kernel for a dtype: the LDS-streaming kernel for 16-bit types,
// the register-staged one for fp32.
template <int DT, int QM, int KVM, int RM, bool MV>
const void* decode_kernel() {
    if constexpr (DT == kF32) return reinterpret_cast<const void*>(&dv_decode<DT, QM, KVM, RM>);
    else return reinterpret_cast<const void*>(&dv_stream<DT, QM, KVM, RM, MV>);
}

template <int DT>
size_t wave_lds() {
    return DT == kF32 ? (size_t)vt_bytes<DT>() : (size_t)stream::kWaveLds;
}

// Resident workgroups per CU for one kernel instance at a given dynamic LDS
// size, cached per 1 KiB of LDS (hipOccupancy queries cost host time).
template <int DT, int QM, int KVM, int RM, bool MV>
int resident_wgs(int hpw, size_t lds) {
    static std::atomic<int> cache[4][161];  // [hpw-1][lds KiB]; 0 = not queried yet
    const int kib = (int)((lds + 1023) / 1024);
    if (kib > 160 || hpw < 1 || hpw > 4) return 1;
    std::atomic<int>& slot = cache[hpw - 1][kib];
    int nb = slot.load(std::memory_order_relaxed);
    if (nb == 0) {
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, decode_kernel<DT, QM, KVM, RM, MV>(), hpw * kWave,
                                                         (size_t)kib * 1024) != hipSuccess ||
            nb < 1)
            nb = 1;
        slot.store(nb, std::memory_order_relaxed);
    }
    return nb;
}

template <int DT, int QM, int KVM, int RM, bool MV>
hipError_t launch_one(DecodeParams p, int device, long long max_wg, long long cap, int cus, hipStream_t stream) {
    const size_t lds = (size_t)p.hpw * wave_lds<DT>() + (size_t)(p.nrows + 1) * sizeof(long long);
    const void* kern = decode_kernel<DT, QM, KVM, RM, MV>();
    static std::atomic<unsigned long long> attr_done{0};
    const hipError_t ea = once_per_device(attr_done, device, [&] {
        // largest dynamic LDS any launch of this kernel asks for (4 waves, kMaxRows rows)
        const size_t max_lds = (size_t)kMaxWavesPerWg * wave_lds<DT>() + (size_t)(kMaxRows + 1) * sizeof(long long);
        return hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)max_lds);
    });
    if (ea != hipSuccess) return note_site(ea, "hipFuncSetAttribute(decode)");
    // one wave of workgroups that are all resident at once, bounded by the work
    long long nwg = (long long)cus * resident_wgs<DT, QM, KVM, RM, MV>(p.hpw, lds);
    if (nwg > max_wg) nwg = max_wg;
    if (nwg > cap) nwg = cap;
    p.nwg = nwg < 1 ? 1 : (int)nwg;
    if constexpr (DT == kF32)
        hipLaunchKernelGGL((dv_decode<DT, QM, KVM, RM>), dim3(p.nwg), dim3(p.hpw * kWave), lds, stream, p);
    else
        hipLaunchKernelGGL((dv_stream<DT, QM, KVM, RM, MV>), dim3(p.nwg), dim3(p.hpw * kWave), lds, stream, p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return note_site(e, "launch decode");
    const int nseg = p.nrows * (p.Hkv / p.hpw);
    hipLaunchKernelGGL((dv_merge<DT, RM>), dim3(nseg * p.hpw * kMergeQuarters), dim3(kMergeWaves * kWave), 0,
                       stream, p);
    e = hipGetLastError();
    if (e != hipSuccess) return note_site(e, "launch dv_merge");
    return hipSuccess;
}

template <int DT>
hipError_t dispatch_modes(int qmode, int kvmode, int rowmode, const DecodeParams& p, int device, long long max_wg,
                          long long cap, int cus, hipStream_t stream) {
    if (kvmode == kKvPaged && qmode == kQRotFull && rowmode == kRowWS)
        return p.F >= 2 && DT != kF32
                   ? launch_one<DT, kQRotFull, kKvPaged, kRowWS, true>(p, device, max_wg, cap, cus, stream)
                   : launch_one<DT, kQRotFull, kKvPaged, kRowWS, false>(p, device, max_wg, cap, cus, stream);
    if (kvmode == kKvPaged && qmode == kQRotHalf && rowmode == kRowVarlen)
        return p.F >= 2 && DT != kF32
                   ? launch_one<DT, kQRotHalf, kKvPaged, kRowVarlen, true>(p, device, max_wg, cap, cus, stream)
                   : launch_one<DT, kQRotHalf, kKvPaged, kRowVarlen, false>(p, device, max_wg, cap, cus, stream);
    if (kvmode == kKvContig && qmode == kQPre && rowmode == kRowWS)
        return launch_one<DT, kQPre, kKvContig, kRowWS, false>(p, device, max_wg, cap, cus, stream);
    return hipErrorInvalidValue;
}

}  // namespace

const char* last_hip_site() { return g_site; }

// Workspace per segment after the partial slots: merge directory {first slot,
// pieces}.
constexpr int kSegBytes = 8;

size_t decode_workspace_bytes(int nrows_total, int Hkv, int device, int dtype) {
    (void)dtype;
    if (nrows_total <= 0 || Hkv <= 0) return 0;
    const int hpw = pick_hpw(Hkv);
    const int nhg = Hkv / hpw;
    const int rows = nrows_total < kMaxRows ? nrows_total : kMaxRows;
    const long long nwg = (long long)device_cus(device) * wgs_per_cu(hpw);
    const long long nseg = (long long)rows * nhg;
    const long long slot_floats = (long long)hpw * kGqa * (kHeadDim + 1);
    const long long slots = nwg + nseg;
    size_t bytes = (size_t)(slots * slot_floats * 4);
    bytes = (bytes + 255) & ~(size_t)255;
    bytes += (size_t)(nseg * kSegBytes);
    return bytes;
}

hipError_t launch_decode(int dtype, int qmode, int kvmode, int rowmode, const DecodeParams& base,
                         int nrows_total, long long max_keys_per_row, void* workspace, size_t ws_bytes,
                         hipStream_t stream) {
    if (nrows_total <= 0 || base.Hkv <= 0) return hipSuccess;
    int device = 0;
    hipError_t e = hipGetDevice(&device);
    if (e != hipSuccess) return e;
    DecodeParams p = base;
    p.hpw = pick_hpw(p.Hkv);
    const int nhg = p.Hkv / p.hpw;
    p.slot_floats = p.hpw * kGqa * (kHeadDim + 1);
    const int cus = device_cus(device);
    const long long max_wg = (long long)cus * wgs_per_cu(p.hpw);
    const int rows_cap = nrows_total < kMaxRows ? nrows_total : kMaxRows;
    const long long slots_cap = max_wg + (long long)rows_cap * nhg;
    size_t part_bytes = (size_t)(slots_cap * p.slot_floats * 4);
    part_bytes = (part_bytes + 255) & ~(size_t)255;
    const long long nseg_cap = (long long)rows_cap * nhg;
    if (ws_bytes < part_bytes + (size_t)nseg_cap * kSegBytes) return hipErrorInvalidValue;
    unsigned char* ws = reinterpret_cast<unsigned char*>(workspace);
    p.part = reinterpret_cast<float*>(ws);
    p.dir = reinterpret_cast<int*>(ws + part_bytes);
    p.piece_cost = dtype == kF32 ? 0 : kPieceCost;
    // the fp32 kernel waits for each 32-key stage before the next: one stage per
    // workgroup is worth it on small problems
    if (dtype == kF32 && p.min_keys > kStep) p.min_keys = kStep;
    p.skew_pm = xcd_skew_pm();
    for (int r0 = 0; r0 < nrows_total; r0 += kMaxRows) {
        p.row_begin = r0;
        p.nrows = nrows_total - r0 < kMaxRows ? nrows_total - r0 : kMaxRows;
        // enough workgroups to fill the chip, never more than the key count allows
        const long long cap = ((long long)p.nrows * nhg * max_keys_per_row + p.min_keys - 1) / p.min_keys;
        switch (dtype) {
            case kBF16: e = dispatch_modes<kBF16>(qmode, kvmode, rowmode, p, device, max_wg, cap, cus, stream); break;
            case kF16: e = dispatch_modes<kF16>(qmode, kvmode, rowmode, p, device, max_wg, cap, cus, stream); break;
            case kF32: e = dispatch_modes<kF32>(qmode, kvmode, rowmode, p, device, max_wg, cap, cus, stream); break;
            default: e = hipErrorInvalidValue;
        }
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace dv
