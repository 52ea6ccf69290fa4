// Work split shared by the decode and chunk kernels.
#pragma once

#include "dv_common.h"
#include "dv_device.h"

namespace dv {

// Every workgroup computes the same schedule from the per-row visible key
// counts (row_keys(absolute row), rows [p.row_begin, p.row_begin + p.nrows)).
// The (row, head-group) segments are laid end to end, each non-empty one
// preceded by p.piece_cost keys of "start cost" (the pipeline start of a piece:
// page ids, query rotation, first loads), and this cost space is cut into equal
// contiguous chunks, one per workgroup; a workgroup whose chunk crosses into a
// new segment thus gets fewer real keys.  The per-row cost prefix sums stay in
// registers when the kernel asks for it (kRegPrefix) and there are at most 64
// rows (every wave scans them itself), else they live in LDS (s_pref, nrows + 1 entries; s_scan: one entry per
// wave); both give the same chunks.  Workgroup 0 writes
// the merge directory (segment -> first partial slot, piece count).  Then
// piece(row, head_group, v0, v1, final, slot, row_keys) runs for each piece of
// this workgroup's chunk: visible keys [v0, v1) of the segment, `final` when
// the segment has no other piece, `slot` its partial slot, `row_keys` the row's
// visible key count.  Slots are
// sg + workgroup index, increasing along the cost space, so they are unique and
// below nwg + nrows * NHG.
// a / b for non-negative operands, in 32 bits when both fit (a 64-bit division
// is a long instruction sequence on the GPU)
__device__ inline long long udiv(long long a, long long b) {
    if (((unsigned long long)(a | b) >> 32) == 0) return (long long)((uint32_t)a / (uint32_t)b);
    return a / b;
}

// Chunks of the cost space and the pieces of this workgroup's chunk, given the
// per-row cost prefix sums: pref_u(r) for a wave-uniform r, pref_v(r) for a
// per-lane r (called with every lane active), find_row(u) = the last row r
// with NHG * pref[r] <= u, total = pref[nrows].
template <class PrefU, class PrefV, class FindRow, class PieceFn>
__device__ inline void split_chunks(const DecodeParams& p, int NHG, long long total, PrefU&& pref_u, PrefV&& pref_v,
                                    FindRow&& find_row, PieceFn&& piece) {
    const int tid = threadIdx.x;
    const int nthreads = blockDim.x;
    const int nrows = p.nrows;
    const long long c = p.piece_cost;

    // 2. chunks of the cost space; segment (r, hg) spans D_r cost units at
    //    NHG*pref[r] + hg*D_r, its keys the last D_r - c of them.  Workgroups are
    //    dispatched to the XCDs round robin (workgroup i on XCD i % 8) and the odd
    //    XCD of each pair streams a few percent slower, so chunk 2k is `skew` cost
    //    units longer and chunk 2k+1 as much shorter than the mean (p.skew_pm per
    //    mille; 0: equal chunks).  Chunk i spans [bound(i), bound(i + 1)).
    const long long Wc = total * NHG;
    const long long ng = udiv(Wc + p.min_keys - 1, p.min_keys);
    const int geff = Wc == 0 ? 0 : (int)(ng < p.nwg ? ng : p.nwg);
    const long long chunk = geff ? udiv(Wc + geff - 1, geff) : 1;
    const long long skew = udiv(chunk * p.skew_pm, 1000);
    auto bound = [&](long long i) {
        const long long b = i * chunk + ((i & 1) ? skew : 0);
        return b < Wc ? b : Wc;
    };
    // chunk holding cost position x (< Wc)
    auto chunk_of = [&](long long x) {
        const long long k = udiv(x, 2 * chunk);
        return 2 * k + (x - 2 * k * chunk >= chunk + skew ? 1 : 0);
    };

    if (blockIdx.x == 0) {
        const int nseg = nrows * NHG;
        for (int b0 = 0; b0 < nseg; b0 += nthreads) {
            const int sg = b0 + tid;
            const int sgc = sg < nseg ? sg : nseg - 1;
            const int r = sgc / NHG, hg = sgc - (sgc / NHG) * NHG;
            const long long pr = pref_v(r), pn = pref_v(r + 1);
            if (sg < nseg) {
                const long long D = pn - pr;
                int base = 0, cnt = 0;
                if (D > 0) {
                    const long long segc = NHG * pr + hg * D;
                    const long long gf = chunk_of(segc + c), gl = chunk_of(segc + D - 1);
                    cnt = (int)(gl - gf + 1);
                    base = (int)gf + sg;
                }
                p.dir[2 * sg] = base;
                p.dir[2 * sg + 1] = cnt;
            }
        }
    }
    const int gidx = blockIdx.x;
    if (gidx >= geff) return;

    const long long u0 = bound(gidx);
    const long long uend = bound(gidx + 1);
    long long u = u0;
    int r = find_row(u);
    while (u < uend && r < nrows) {
        const long long pr = pref_u(r);
        const long long rs = NHG * pr;
        const long long D = pref_u(r + 1) - pr;
        if (D == 0 || u >= rs + NHG * D) {
            ++r;
            continue;
        }
        const int hg = (int)udiv(u - rs, D);
        const long long segc = rs + hg * D;  // the segment's cost range [segc, segc + D)
        const long long ka = segc + c;       // its keys: cost positions [ka, segc + D)
        const long long a = u > ka ? u : ka;
        const long long b = uend < segc + D ? uend : segc + D;
        if (a < b) {
            const int sg = r * NHG + hg;
            // the segment has no other piece iff its first and last keys both lie
            // in this chunk (chunk_of(ka) == chunk_of(segc + D - 1) == gidx, without
            // the divisions)
            const bool fin = ka >= u0 && segc + D - 1 < uend;
            const int slot = sg + gidx;  // = first slot of the segment (chunk_of(ka) + sg) + piece index
            piece(p.row_begin + r, hg, a - ka, b - ka, fin, slot, D - c);
        }
        u = segc + D;
    }
}

template <bool kRegPrefix = false, class RowKeys, class PieceFn>
__device__ inline void run_schedule(const DecodeParams& p, int NHG, long long* s_pref, long long* s_scan,
                                    RowKeys&& row_keys, PieceFn&& piece) {
    const int tid = threadIdx.x;
    const int wv = tid >> 6;
    const int lane = tid & 63;
    const int nthreads = blockDim.x;
    const long long c = p.piece_cost;
    const int nrows = p.nrows;

    // 1. per-row cost (visible keys + start cost, 0 for an empty row) -> exclusive
    //    prefix sums.  kRegPrefix and at most 64 rows: one row per lane, every
    //    wave on its own, the sums in registers (lane r holds pref[r]; lanes
    //    from nrows on hold the total), with no LDS round trip and no workgroup
    //    barrier before the first piece -- for kernels with registers to spare
    //    (the 16-bit decode: one wave per SIMD); the sums stay live through the
    //    piece loop.  Otherwise rows split over the threads, sums in LDS.
    const bool inreg = kRegPrefix && nrows <= kWave;
    long long excl = 0, total = 0;
    if (inreg) {
        long long d = 0;
        if (lane < nrows) {
            const long long v = row_keys(p.row_begin + lane);
            d = v > 0 ? v + c : 0;
        }
        long long incl = d;
#pragma unroll
        for (int o = 1; o < kWave; o <<= 1) {
            const long long t = __shfl_up(incl, o, kWave);
            if (lane >= o) incl += t;
        }
        excl = incl - d;
        total = __shfl(incl, kWave - 1, kWave);
    } else {
        const int per = (nrows + nthreads - 1) / nthreads;
        const int r0 = tid * per;
        const int r1 = r0 + per < nrows ? r0 + per : nrows;
        long long mine = 0;
        for (int r = r0; r < r1; ++r) {
            const long long v = row_keys(p.row_begin + r);
            const long long d = v > 0 ? v + c : 0;
            s_pref[r] = d;  // the row's cost, replaced by its prefix below
            mine += d;
        }
        long long incl = mine;
#pragma unroll
        for (int d = 1; d < kWave; d <<= 1) {
            const long long o = __shfl_up(incl, d, kWave);
            if (lane >= d) incl += o;
        }
        if (lane == 63) s_scan[wv] = incl;
        __syncthreads();
        long long before = 0;
        for (int i = 0; i < wv; ++i) before += s_scan[i];
        long long run = before + incl - mine;
        for (int r = r0; r < r1; ++r) {
            const long long d = s_pref[r];
            s_pref[r] = run;
            run += d;
        }
        for (int i = 0; i < nthreads / kWave; ++i) total += s_scan[i];
        if (tid == 0) s_pref[nrows] = total;
        __syncthreads();
    }
    // pref[r], r uniform
    auto pref_u = [&](int r) -> long long {
        if (!inreg) return s_pref[r];
        if (r >= kWave) return total;
        const int rr = __builtin_amdgcn_readfirstlane(r);
        const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)excl, rr);
        const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)((unsigned long long)excl >> 32), rr);
        return (long long)(((unsigned long long)hi << 32) | lo);
    };
    // pref[r], r per lane, every lane active
    auto pref_v = [&](int r) -> long long {
        if (!inreg) return s_pref[r];
        const long long x = __shfl(excl, r < kWave ? r : 0, kWave);
        return r < kWave ? x : total;
    };
    // the last row r with NHG * pref[r] <= u
    auto find_row = [&](long long u) -> int {
        if (inreg) {
            const uint64_t b = ballot(lane < nrows && NHG * excl <= u);
            return b ? 63 - __builtin_clzll(b) : 0;
        }
        int lo = 0, hi = nrows - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (NHG * s_pref[mid] <= u) lo = mid;
            else hi = mid - 1;
        }
        return lo;
    };
    split_chunks(p, NHG, total, pref_u, pref_v, find_row, piece);
}

}  // namespace dv
