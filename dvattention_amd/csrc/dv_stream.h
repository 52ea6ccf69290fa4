// Row / view helpers, the query loaders and the direct-to-LDS K/V staging of
// the decode kernels (dv_decode.hip), shared with the single-launch path for
// short views (dv_small.hip) and the paged-read probe (dv_probe.hip), so that
// all of them see the same rows, views and rotated queries.
#pragma once

#include "dv_common.h"
#include "dv_device.h"

namespace dv {

// ---- row / view helpers -------------------------------------------------------

template <int RM>
__device__ inline int row_loc(const DecodeParams& p, int row, int f) {
    if (RM == kRowVarlen) return p.loc[(long long)f * p.T + row];
    const int w = row / p.S;
    const int s = row - w * p.S;
    return p.loc[((long long)f * p.W + w) * p.S + s];
}

template <int KVM>
__device__ inline const FragDesc& frag(const DecodeParams& p, int f) {
    return f < kMaxFragArgs ? p.frags[f] : p.frag_tab[f];
}

// Visible keys of view f for a query at location locv:
// min(L_f, loc + 1) clamped at 0 (paged_kernel_v21.cuh:83-85); varlen views with
// loc < 0 are skipped (varlen_paged_kernel_v21.cuh:76-80), which is the same count.
template <int KVM>
__device__ inline int view_vis(const DecodeParams& p, int f, int locv) {
    long long L = p.fl[f];
    if (KVM == kKvContig) L = L < frag<KVM>(p, f).L ? L : frag<KVM>(p, f).L;
    long long v = (long long)locv + 1;
    v = v < L ? v : L;
    return v > 0 ? (int)v : 0;
}

template <int KVM, int RM>
__device__ inline long long row_visible(const DecodeParams& p, int row) {
    // views four at a time, their loads issued together (one memory round trip
    // per four views instead of two per view)
    long long v = 0;
    int f = 0;
    for (; f + 4 <= p.F; f += 4) {
        int lc[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) lc[j] = row_loc<RM>(p, row, f + j);
#pragma unroll
        for (int j = 0; j < 4; ++j) v += view_vis<KVM>(p, f + j, lc[j]);
    }
    for (; f < p.F; ++f) v += view_vis<KVM>(p, f, row_loc<RM>(p, row, f));
    return v;
}

// The views of one query row, view f in lane f (F <= 64), from one round of
// loads: visible keys, visible keys of the earlier views, and logical position
// of the view's key 0 (sum of the earlier fragment_lengths).
struct ViewTab {
    int vis;
    long long P, off;
};

template <int KVM, int RM>
__device__ inline ViewTab view_table(const DecodeParams& p, int row) {
    const int lane = threadIdx.x & 63;
    int vis = 0;
    long long fl = 0;
    if (lane < p.F) {
        vis = view_vis<KVM>(p, lane, row_loc<RM>(p, row, lane));
        fl = p.fl[lane];
    }
    long long sv = vis, so = fl;
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
        const long long tv = __shfl_up(sv, d, kWave);
        const long long to = __shfl_up(so, d, kWave);
        if (lane >= d) {
            sv += tv;
            so += to;
        }
    }
    return ViewTab{vis, sv - vis, so - fl};
}

// Calls body(f, vis, P, off) for every view of `row` with visible keys in the
// row's visible-key range [v0, v1), in view order.
template <int KVM, int RM, class Body>
__device__ inline void for_views(const DecodeParams& p, int row, long long v0, long long v1, Body&& body) {
    if (p.F <= kWave) {
        const int lane = threadIdx.x & 63;
        const ViewTab t = view_table<KVM, RM>(p, row);
        uint64_t m = ballot(lane < p.F && t.vis > 0 && t.P < v1 && t.P + t.vis > v0);
        while (m) {
            const int f = __builtin_ctzll(m);
            m &= m - 1;
            body(f, __shfl(t.vis, f, kWave), __shfl(t.P, f, kWave), __shfl(t.off, f, kWave));
        }
        return;
    }
    long long P = 0, off = 0;
    for (int f = 0; f < p.F && P < v1; ++f) {
        const int vis = view_vis<KVM>(p, f, row_loc<RM>(p, row, f));
        if (vis > 0 && P + vis > v0) body(f, vis, P, off);
        P += vis;
        off += p.fl[f];
    }
}

// Sequence of packed token t: first i with t < cu_seqlens_q[i+1], else 0
// (varlen_paged_kernel_v21.cuh:40-47).  Wave-cooperative, 64 entries per ballot.
__device__ inline int varlen_seq(const DecodeParams& p, int t) {
    const int lane = threadIdx.x & 63;
    for (int base = 0; base < p.W; base += kWave) {
        const int i = base + lane;
        const bool hit = i < p.W && t < p.cu_q[i + 1];
        const uint64_t b = ballot(hit);
        if (b) return base + __builtin_ctzll(b);
    }
    return 0;
}

// ---- query operand ------------------------------------------------------------

// 16-bit: lane (g, n) holds Q[n][c*32 + g*8 + 0..7] for c = 0..3 (B operand of S^T).
template <int DT, int QM, int RM>
__device__ inline void load_q16(const DecodeParams& p, int row, int f, int hkv, u32x4 (&qB)[4]) {
    using raw = typename Tr<DT>::raw;
    const int lane = threadIdx.x & 63;
    const int g = lane >> 4, n = lane & 15;
    const int h = hkv * kGqa + n;
    if (QM == kQPre) {
        const int w = row / p.S, s = row - (row / p.S) * p.S;
        const raw* q = reinterpret_cast<const raw*>(p.q) +
                       ((((long long)f * p.W + w) * p.Hq + h) * p.S + s) * kHeadDim;
#pragma unroll
        for (int cc = 0; cc < 4; ++cc) qB[cc] = ld16(q + cc * 32 + g * 8);
        return;
    }
    const raw* q;
    const float* cs;
    const float* sn;
    if (QM == kQRotFull) {
        const int w = row / p.S, s = row - (row / p.S) * p.S;
        q = reinterpret_cast<const raw*>(p.q) + (((long long)w * p.Hq + h) * p.S + s) * kHeadDim;
        const long long co = (((long long)f * p.W + w) * p.S + s) * p.R;
        cs = p.cosv + co;
        sn = p.sinv + co;
    } else {
        q = reinterpret_cast<const raw*>(p.q) + ((long long)row * p.Hq + h) * kHeadDim;
        const long long co = ((long long)f * p.T + row) * (p.R >> 1);
        cs = p.cosv + co;
        sn = p.sinv + co;
    }
#pragma unroll
    for (int cc = 0; cc < 4; ++cc) {
        raw r[8];
        rotate_run<DT, 8>(q, cs, sn, p.R, cc * 32 + g * 8, r);
        qB[cc] = u32x4{(uint32_t)r[0] | ((uint32_t)r[1] << 16), (uint32_t)r[2] | ((uint32_t)r[3] << 16),
                       (uint32_t)r[4] | ((uint32_t)r[5] << 16), (uint32_t)r[6] | ((uint32_t)r[7] << 16)};
    }
}

// The same operand in two steps, so that its loads can be issued before the
// piece's page ids are loaded and their round trips overlap: fetch_q16 loads
// lane (g, n)'s query runs Q[n][c*32 + g*8 + 0..7] (c = 0..3) and, for a
// rotation over all 128 dims, the cos/sin runs [h*32 + g*8, +8) (h = 0, 1);
// rotate_q16 then rotates them with load_q16's arithmetic, bit for bit.  With
// R = 128, dims d and d + 64 pair up, so run c's partner is run c ^ 2 and both
// use cos/sin run c & 1.  Taken when q_split() holds (pre-rotated queries, or
// R = 128 with 16-byte aligned cos/sin tables); otherwise load_q16.
struct QRaw {
    u32x4 q[4];
    f32x4 c[2][2], s[2][2];
};

template <int QM>
__device__ inline bool q_split(const DecodeParams& p) {
    return QM == kQPre ||
           (p.R == kHeadDim && ((reinterpret_cast<uintptr_t>(p.cosv) | reinterpret_cast<uintptr_t>(p.sinv)) & 15) == 0);
}

template <int DT, int QM, int RM>
__device__ inline void fetch_q16(const DecodeParams& p, int row, int f, int hkv, QRaw& r) {
    using raw = typename Tr<DT>::raw;
    const int lane = threadIdx.x & 63;
    const int g = lane >> 4, n = lane & 15;
    const int h = hkv * kGqa + n;
    const raw* q;
    const float* cs = nullptr;
    const float* sn = nullptr;
    if (QM == kQPre) {
        const int w = row / p.S, s = row - (row / p.S) * p.S;
        q = reinterpret_cast<const raw*>(p.q) + ((((long long)f * p.W + w) * p.Hq + h) * p.S + s) * kHeadDim;
    } else if (QM == kQRotFull) {
        const int w = row / p.S, s = row - (row / p.S) * p.S;
        q = reinterpret_cast<const raw*>(p.q) + (((long long)w * p.Hq + h) * p.S + s) * kHeadDim;
        const long long co = (((long long)f * p.W + w) * p.S + s) * p.R;
        cs = p.cosv + co;
        sn = p.sinv + co;
    } else {
        q = reinterpret_cast<const raw*>(p.q) + ((long long)row * p.Hq + h) * kHeadDim;
        const long long co = ((long long)f * p.T + row) * (p.R >> 1);
        cs = p.cosv + co;
        sn = p.sinv + co;
    }
#pragma unroll
    for (int cc = 0; cc < 4; ++cc) r.q[cc] = ld16(q + cc * 32 + g * 8);
    if (QM != kQPre) {
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            r.c[hh][0] = ld16f(cs + hh * 32 + g * 8);
            r.c[hh][1] = ld16f(cs + hh * 32 + g * 8 + 4);
            r.s[hh][0] = ld16f(sn + hh * 32 + g * 8);
            r.s[hh][1] = ld16f(sn + hh * 32 + g * 8 + 4);
        }
    }
}

template <int DT, int QM>
__device__ inline void rotate_q16(const QRaw& rin, u32x4 (&qB)[4]) {
#pragma clang fp contract(off)
    // register tie: the rotation is computed here, after whatever the caller
    // issued since fetch_q16 (left to itself, the compiler computed it right
    // after the loads, waiting for them before the page-id loads)
    QRaw r = rin;
#pragma unroll
    for (int cc = 0; cc < 4; ++cc) asm volatile("" : "+v"(r.q[cc]));
    if (QM != kQPre) {
#pragma unroll
        for (int hh = 0; hh < 2; ++hh)
#pragma unroll
            for (int k = 0; k < 2; ++k) asm volatile("" : "+v"(r.c[hh][k]), "+v"(r.s[hh][k]));
    }
    if (QM == kQPre) {
#pragma unroll
        for (int cc = 0; cc < 4; ++cc) qB[cc] = r.q[cc];
        return;
    }
#pragma unroll
    for (int cc = 0; cc < 4; ++cc) {
        const bool first = cc < 2;  // dims [0, 64): x c - x' s; [64, 128): x c + x' s
        const u32x4 x = r.q[cc], xp = r.q[cc ^ 2];
        uint32_t wd[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            uint32_t hv[2];
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const int k = 2 * t + e;
                // halves by shifts (a vector element bit-cast to a 16-bit pair
                // was compiled as a cast of element 0)
                const float xv = Tr<DT>::tof((uint16_t)(e ? x[t] >> 16 : x[t] & 0xffffu));
                const float xq = Tr<DT>::tof((uint16_t)(e ? xp[t] >> 16 : xp[t] & 0xffffu));
                const float c = r.c[cc & 1][k >> 2][k & 3];
                const float s = r.s[cc & 1][k >> 2][k & 3];
                const float a = xv * c;
                const float b = xq * s;
                const float y = first ? a - b : a + b;
                hv[e] = Tr<DT>::fromf(y);
            }
            wd[t] = hv[0] | (hv[1] << 16);
        }
        qB[cc] = u32x4{wd[0], wd[1], wd[2], wd[3]};
    }
}

// Multi-view pieces with a rotary width R of 32 or 64: the row's query runs
// are loaded once (fetch_qrow16, same lanes and runs as fetch_q16) and each
// view's cos/sin run separately (fetch_cs16_narrow: one 8-dim run per lane, at
// (g·8) mod R/2), all before the page ids; rotate_q16_narrow then gives
// load_q16's operand bit for bit.  Dim d pairs with d ± R/2: for R = 64 run c's
// partner is run c ^ 1 (same lane), for R = 32 run 0 of lane ^ 32 (g ^ 2);
// runs from c·32 >= R pass through.  Taken when q_split_narrow() holds.
struct QCs1 {
    f32x4 c[2], s[2];
};

template <int QM>
__device__ inline bool q_split_narrow(const DecodeParams& p) {
    return QM != kQPre && (p.R == 32 || p.R == 64) &&
           ((reinterpret_cast<uintptr_t>(p.cosv) | reinterpret_cast<uintptr_t>(p.sinv)) & 15) == 0;
}

template <int DT, int QM, int RM>
__device__ inline void fetch_qrow16(const DecodeParams& p, int row, int hkv, u32x4 (&q4)[4]) {
    using raw = typename Tr<DT>::raw;
    const int lane = threadIdx.x & 63;
    const int g = lane >> 4, n = lane & 15;
    const int h = hkv * kGqa + n;
    const raw* q;
    if (QM == kQRotFull) {
        const int w = row / p.S, s = row - (row / p.S) * p.S;
        q = reinterpret_cast<const raw*>(p.q) + (((long long)w * p.Hq + h) * p.S + s) * kHeadDim;
    } else {
        q = reinterpret_cast<const raw*>(p.q) + ((long long)row * p.Hq + h) * kHeadDim;
    }
#pragma unroll
    for (int cc = 0; cc < 4; ++cc) q4[cc] = ld16(q + cc * 32 + g * 8);
}

template <int QM>
__device__ inline void fetch_cs16_narrow(const DecodeParams& p, int row, int f, QCs1& r) {
    const int g = (threadIdx.x & 63) >> 4;
    const int half = p.R >> 1;
    long long co;
    if (QM == kQRotFull) {
        const int w = row / p.S, s = row - (row / p.S) * p.S;
        co = (((long long)f * p.W + w) * p.S + s) * p.R;
    } else {
        co = ((long long)f * p.T + row) * half;
    }
    const int ci = (g * 8) & (half - 1);
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
        r.c[hh] = ld16f(p.cosv + co + ci + 4 * hh);
        r.s[hh] = ld16f(p.sinv + co + ci + 4 * hh);
    }
}

template <int DT>
__device__ inline void rotate_q16_narrow(const DecodeParams& p, const u32x4 (&qin)[4], const QCs1& csin,
                                         u32x4 (&qB)[4]) {
#pragma clang fp contract(off)
    // register tie: rotated here, after whatever the caller issued since the
    // fetch (else the compiler computes it right after the loads, waiting for
    // them before the page-id loads)
    u32x4 q[4];
#pragma unroll
    for (int cc = 0; cc < 4; ++cc) {
        q[cc] = qin[cc];
        asm volatile("" : "+v"(q[cc]));
    }
    QCs1 cs = csin;
#pragma unroll
    for (int k = 0; k < 2; ++k) asm volatile("" : "+v"(cs.c[k]), "+v"(cs.s[k]));
    const int g = (threadIdx.x & 63) >> 4;
    const bool r64 = p.R == 64;
    u32x4 x32 = q[0];
    if (!r64) {
#pragma unroll
        for (int e = 0; e < 4; ++e) x32[e] = (uint32_t)__shfl_xor((int)q[0][e], 32, kWave);
    }
#pragma unroll
    for (int cc = 0; cc < 4; ++cc) {
        if (cc >= 2 || (cc == 1 && !r64)) {  // dims past the rotary width pass through
            qB[cc] = q[cc];
            continue;
        }
        // first half: x c - x' s; second: x c + x' s
        const bool first = r64 ? cc == 0 : g < 2;
        const u32x4 x = q[cc];
        const u32x4 xp = r64 ? q[cc ^ 1] : x32;
        uint32_t wd[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            uint32_t hv[2];
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const int k = 2 * t + e;
                // halves by shifts (a vector element bit-cast to a 16-bit pair
                // was compiled as a cast of element 0)
                const float xv = Tr<DT>::tof((uint16_t)(e ? x[t] >> 16 : x[t] & 0xffffu));
                const float xq = Tr<DT>::tof((uint16_t)(e ? xp[t] >> 16 : xp[t] & 0xffffu));
                const float c = cs.c[k >> 2][k & 3];
                const float s = cs.s[k >> 2][k & 3];
                const float a = xv * c;
                const float b = xq * s;
                const float y = first ? a - b : a + b;
                hv[e] = Tr<DT>::fromf(y);
            }
            wd[t] = hv[0] | (hv[1] << 16);
        }
        qB[cc] = u32x4{wd[0], wd[1], wd[2], wd[3]};
    }
}

// fp32: lane (g, n) holds Q[n][c*16 + g*4 + 0..3] for c = 0..7.
template <int QM, int RM>
__device__ inline void load_q32(const DecodeParams& p, int row, int f, int hkv, f32x4 (&qB)[8]) {
    const int lane = threadIdx.x & 63;
    const int g = lane >> 4, n = lane & 15;
    const int h = hkv * kGqa + n;
    if (QM == kQPre) {
        const int w = row / p.S, s = row - (row / p.S) * p.S;
        const float* q = reinterpret_cast<const float*>(p.q) +
                         ((((long long)f * p.W + w) * p.Hq + h) * p.S + s) * kHeadDim;
#pragma unroll
        for (int cc = 0; cc < 8; ++cc) qB[cc] = ld16f(q + cc * 16 + g * 4);
        return;
    }
    const float* q;
    const float* cs;
    const float* sn;
    if (QM == kQRotFull) {
        const int w = row / p.S, s = row - (row / p.S) * p.S;
        q = reinterpret_cast<const float*>(p.q) + (((long long)w * p.Hq + h) * p.S + s) * kHeadDim;
        const long long co = (((long long)f * p.W + w) * p.S + s) * p.R;
        cs = p.cosv + co;
        sn = p.sinv + co;
    } else {
        q = reinterpret_cast<const float*>(p.q) + ((long long)row * p.Hq + h) * kHeadDim;
        const long long co = ((long long)f * p.T + row) * (p.R >> 1);
        cs = p.cosv + co;
        sn = p.sinv + co;
    }
#pragma unroll
    for (int cc = 0; cc < 8; ++cc) {
        float r[4];
        rotate_run<kF32, 4>(q, cs, sn, p.R, cc * 16 + g * 4, r);
        qB[cc] = f32x4{r[0], r[1], r[2], r[3]};
    }
}

// Rows of zeros that invisible keys load from, so every lane issues the same
// loads (no divergent branches around the memory instructions).
static __device__ __align__(16) unsigned char g_zero_row[512];

// Logical page and in-page offset of a logical key position (32-bit, as the
// reference's absolute_key_pos, paged_kernel_v21.cuh:103-104).
__device__ inline void page_split(const DecodeParams& p, uint32_t pos, uint32_t& lp, uint32_t& r) {
    if (p.bs_shift >= 0) {
        lp = pos >> p.bs_shift;
        r = pos & ((1u << p.bs_shift) - 1u);
    } else {
        lp = pos / (uint32_t)p.bs;
        r = pos - lp * (uint32_t)p.bs;
    }
}

// ---- work-split parameters of the 16-bit decode --------------------------------

// KV heads (waves) per workgroup.
inline int pick_hpw(int Hkv) {
    if (Hkv % 4 == 0) return 4;
    if (Hkv % 2 == 0) return 2;
    return 1;
}

// Start cost of a piece in the 16-bit decode's work split, in keys: about the
// time a workgroup needs to restart its pipeline on a new segment (measured
// against 64, 96, 128 and 160: configurations 2 and 3 ran fastest at 192,
// configuration 4 within its spread).
constexpr int kPieceCost = 192;

// Smallest key range worth a workgroup in the decode split.
constexpr int kDecodeMinKeys = 64;

// Per mille of a chunk the work split moves from each odd workgroup (odd XCD)
// to the even one before it: measured on MI355X, the odd XCD of each pair ends
// 5-8 % later with equal chunks, and 40-60 per mille gave the shortest calls
// on configurations 2-4.  DVATTN_XCD_SKEW_PM overrides it (0: equal chunks).
inline int xcd_skew_pm() {
    static const int v = env_per_mille("DVATTN_XCD_SKEW_PM", 50);
    return v;
}

namespace stream {

constexpr int kTile = kStep * 256;           // one K (or V) stage tile: 32 keys x 256 B
constexpr int kStage = 2 * kTile;            // K tile then V tile
constexpr int kRing = 2;                     // stages per wave
constexpr int kPc = 512;                     // page ids cached per wave
constexpr int kWaveLds = kRing * kStage + kPc * 4;

// Page-cache fill of one wave: pc[i] = block_tables row entry lp_of(i) for i in
// [0, n) (n <= kPc), -1 for an entry past the row or a page id outside
// [0, num_blocks).  All of the wave's loads are issued before the first is
// waited for (a loop that stored each pass's ids before loading the next paid
// one memory round trip per 64 entries): every pass loads from a clamped,
// in-bounds index, and the range checks and LDS stores follow in a second pass.
template <class LpOf>
__device__ inline void fill_pages(const DecodeParams& p, const int* bt, int* pc, int n, LpOf&& lp_of) {
    constexpr int kIt = kPc / kWave;
    const int lane = threadIdx.x & 63;
    const uint32_t maxB = (uint32_t)p.maxB;
    const int nk = (n + kWave - 1) / kWave;  // passes with entries (wave-uniform)
    if (n <= 0) return;
    int pg[kIt];
    uint32_t ok = 0;  // bit k: entry lane + 64k exists and lies in the row
#pragma unroll
    for (int k = 0; k < kIt; ++k) {
        const int i = lane + k * kWave;
        const uint32_t lp = lp_of(i < n ? i : n - 1);
        ok |= (i < n && lp < maxB) ? (1u << k) : 0u;
        pg[k] = -1;
        if (k < nk && maxB > 0) pg[k] = bt[lp < maxB ? lp : maxB - 1];
    }
#pragma unroll
    for (int k = 0; k < kIt; ++k) {
        const int i = lane + k * kWave;
        if (k < nk && i < n) {
            int v = ((ok >> k) & 1u) ? pg[k] : -1;
            if (v < 0 || v >= p.nblocks) v = -1;
            pc[i] = v;
        }
    }
}

struct View {
    const unsigned char* k;  // paged: the cache; contiguous: K row 0 of (batch entry, head)
    const unsigned char* v;
    int off;                 // paged: logical position of the view's key 0
    int lp0;                 // paged: logical page of page-cache entry 0
    int b;                   // end (exclusive) of the current view-local key range
    int hkv;
};

// Issue the 16 direct-to-LDS loads of the stage holding keys [l, l+32) into the
// ring slot at LDS address sbase.  Load i moves key rows 4i .. 4i+3: lane ->
// (row lane/16, swizzled piece).  Returns the visibility mask of the 32 keys.
template <int KVM>
__device__ inline uint32_t issue(const DecodeParams& p, const View& v, const int* pc, uint32_t sbase, int l) {
    const int lane = threadIdx.x & 63;
    const int c16 = lane & 15, sub = lane >> 4;
    // addresses of the 8 key rows first (page-cache reads batched), then the loads
    const unsigned char* ka[8];
    const unsigned char* va[8];
    bool ok[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int kk = i * 4 + sub;
        const int key = l + kk;
        unsigned long long boff;
        if (KVM == kKvPaged) {
            const int pos = v.off + key;
            uint32_t lp, r;
            page_split(p, pos > 0 ? (uint32_t)pos : 0u, lp, r);
            const uint32_t idx = lp - (uint32_t)v.lp0;
            const bool in = key < v.b && pos >= 0 && idx < (uint32_t)kPc;
            const int page = in ? pc[in ? idx : 0u] : -1;
            ok[i] = page >= 0;
            const uint32_t rowidx = ((uint32_t)page * (uint32_t)p.bs + r) * (uint32_t)p.Hkv + (uint32_t)v.hkv;
            boff = (unsigned long long)rowidx << 8;
        } else {
            ok[i] = key < v.b;
            boff = (unsigned long long)(uint32_t)key << 8;
        }
        const int gk = c16 ^ (kk & 15), gv = c16 ^ ((kk & 7) << 1);
        ka[i] = ok[i] ? v.k + boff + gk * 16 : g_zero_row + gk * 16;
        va[i] = ok[i] ? v.v + boff + gv * 16 : g_zero_row + gv * 16;
    }
    uint32_t mask = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        dma16(ka[i], sbase + (uint32_t)(i * 1024));
        dma16(va[i], sbase + (uint32_t)(kTile + i * 1024));
        const uint64_t bl = ballot(ok[i]);
        const uint32_t bits = (uint32_t)(bl & 1u) | (uint32_t)((bl >> 15) & 2u) | (uint32_t)((bl >> 30) & 4u) |
                              (uint32_t)((bl >> 45) & 8u);
        mask |= bits << (i * 4);
    }
    return mask;
}

}  // namespace stream

}  // namespace dv
