// Row groups, work split pieces and the split merge shared by the multi-query
// ("chunk") kernels: dv_chunk (16-bit, dv_chunk.hip) and dv_chunk32 (fp32,
// dv_chunk32.hip).  A row group is up to kTokBlk query tokens of one sequence
// that share one K/V stream; segments are (row group, KV head); every piece
// leaves kTokBlk x 16 normalised output rows in a partial slot, which
// dv_merge_chunk combines.
#pragma once

#include <climits>

#include "dv_common.h"
#include "dv_device.h"
#include "dv_schedule.h"
#include "dv_stream.h"

namespace dv {
namespace chunk {

constexpr int kWaves = 8;                     // waves per workgroup (two per SIMD)
constexpr int kThreads = kWaves * kWave;
constexpr int kTiles = 2;                     // 16-head query tiles (tokens) per wave
constexpr int kHalf = kTiles / 2;             // tiles per MFMA/VALU group
constexpr int kTokBlk = kWaves * kTiles;      // tokens per row group
constexpr int kStages = 8;                    // K/V ring depth
constexpr int kKvBytes = kStep * 256;         // one K (or V) stage tile: 32 keys x 256 B
constexpr int kStageBytes = 2 * kKvBytes;     // K tile then V tile
constexpr int kRingBytes = kStages * kStageBytes;
constexpr int kPageCap = 2048;                // page ids cached in LDS per view sub-range
constexpr int kAhead = 7;                     // stages in flight ahead of the one computed
constexpr int kDmaPerStage = 2;               // per wave: 1 x K + 1 x V (1 KiB = 4 key rows each)

// Start cost of a piece in the work split, in keys (query staging and rotation,
// page ids, the ring prologue).
constexpr int kPieceCost = 256;

static __device__ __align__(16) unsigned char zrow[512];

struct Range {
    const unsigned char* k;  // K base (paged cache or this view's fragment)
    const unsigned char* v;
    long long off;           // paged: logical position of the view's key 0
    long long bstride;       // contig: element offset of the sequence's batch entry
    int L;                   // contig: tokens in the fragment tensor
    uint32_t lp0;            // paged: first cached logical page
    bool pages_ok;           // paged: every page of the current sub-range is valid
    int w, hkv;
    int b;                   // end (exclusive) of the view-local key range
};

// Byte offset of key l's K (= V) row, or -1 when not visible / not addressable.
// Paged rows are indexed in 32 bits (the C ABI rejects caches of 2^32 rows or
// more) and positions are 32-bit as in the reference (paged_kernel_v21.cuh:103-104).
template <int KVM, bool P2>
__device__ inline long long row_of(const DecodeParams& p, const Range& r, const int* pages, int l) {
    if (KVM == kKvPaged) {
        const uint32_t pos = (uint32_t)(r.off + l);
        uint32_t lp, rr;
        if (P2) {  // block_size a power of two
            lp = pos >> p.bs_shift;
            rr = pos & ((1u << p.bs_shift) - 1u);
        } else {
            lp = pos / (uint32_t)p.bs;
            rr = pos - lp * (uint32_t)p.bs;
        }
        // the page-cache read is unconditional (clamped index), so no branch
        // forms around it
        const uint32_t idx = lp - r.lp0;
        const int pg = pages[idx < (uint32_t)kPageCap ? idx : (uint32_t)(kPageCap - 1)];
        const bool ok = l < r.b && idx < (uint32_t)kPageCap && pg >= 0;
        const uint32_t rowidx = ((uint32_t)pg * (uint32_t)p.bs + rr) * (uint32_t)p.Hkv + (uint32_t)r.hkv;
        return ok ? (long long)((unsigned long long)rowidx << 8) : -1;
    } else {
        return l < r.b ? (r.bstride + ((long long)r.hkv * r.L + l) * kHeadDim) * 2 : -1;
    }
}

// A row group: up to kTokBlk query tokens of one sequence that share one K/V
// stream.  kRowWS: group rg is block rg % nsb of sequence rg / nsb in the
// [W, S] token grid (tokens s0 .. s0 + ntok - 1); kRowVarlen: entry rg of the
// table dv_varlen_groups writes (packed tokens lin .. lin + ntok - 1 of
// sequence w).  lin: the first token's index on the token axis of locations
// and cos/sin (w * S + s0, or the packed token).
struct Grp {
    int w, s0, lin, ntok;
};

template <int RM>
__device__ inline Grp group_of(const DecodeParams& p, int rg) {
    Grp g;
    if (RM == kRowVarlen) {
        const int4 e = reinterpret_cast<const int4*>(p.vgroups)[rg];
        g.lin = e.x;
        g.ntok = e.y;
        g.w = e.z;
        g.s0 = 0;
    } else {
        const int nsb = (p.S + kTokBlk - 1) / kTokBlk;
        g.w = rg / nsb;
        g.s0 = (rg - g.w * nsb) * kTokBlk;
        g.ntok = p.S - g.s0 < kTokBlk ? p.S - g.s0 : kTokBlk;
        g.lin = g.w * p.S + g.s0;
    }
    return g;
}

// Length of the token axis of locations [F, tokens] and cos/sin.
template <int RM>
__device__ inline long long tok_axis(const DecodeParams& p) {
    return RM == kRowVarlen ? (long long)p.T : (long long)p.W * p.S;
}

// Element offset of the query row (head h) and of the output row of token i
// of group g (view f for pre-rotated queries [F, W, Hq, S, E]).
template <int QM, int RM>
__device__ inline long long q_row(const DecodeParams& p, const Grp& g, int i, int h, int f) {
    if (RM == kRowVarlen) return ((long long)(g.lin + i) * p.Hq + h) * kHeadDim;
    if (QM == kQPre) return ((((long long)f * p.W + g.w) * p.Hq + h) * p.S + g.s0 + i) * kHeadDim;
    return (((long long)g.w * p.Hq + h) * p.S + g.s0 + i) * kHeadDim;
}
template <int RM>
__device__ inline long long out_row(const DecodeParams& p, const Grp& g, int i, int h) {
    if (RM == kRowVarlen) return ((long long)(g.lin + i) * p.Hq + h) * kHeadDim;
    return (((long long)g.w * p.Hq + h) * p.S + g.s0 + i) * kHeadDim;
}

// Location of token i of group g in view f (locations [F, tokens]).
template <int RM>
__device__ inline int loc_of(const DecodeParams& p, int f, const Grp& g, int i) {
    return p.loc[(long long)f * tok_axis<RM>(p) + g.lin + i];
}

// Length of a row group's key space: per view, the union (max) over its tokens
// of the view's visible count, summed over views -- the coordinates chunk_piece
// walks (view f's keys follow the longest range of views 0 .. f-1).  The max
// over tokens of the per-token sum is shorter whenever different tokens see
// most in different views, and would leave the tail of the key space unassigned.
// View f's visible count, the largest over the tokens of group g: the tokens'
// locations are loaded together (one round trip instead of one per token; the
// loads are unconditional, on a clamped token index, so none waits behind a
// branch); a token past the group's end counts as location -1, which sees no
// key.  (A group without tokens -- varlen padding, first token 0 -- reads token
// 0's location and discards it.)
template <int KVM, int RM>
__device__ inline int group_view_vis(const DecodeParams& p, int f, const Grp& g) {
    const int last = g.ntok > 0 ? g.ntok - 1 : 0;
    int lc[kTokBlk];
#pragma unroll
    for (int i = 0; i < kTokBlk; ++i) {
        const int x = loc_of<RM>(p, f, g, i < last ? i : last);
        lc[i] = i < g.ntok ? x : -1;
    }
    int best = 0;
#pragma unroll
    for (int i = 0; i < kTokBlk; ++i) {
        const int v = view_vis<KVM>(p, f, lc[i]);
        best = v > best ? v : best;
    }
    return best;
}

template <int KVM, int RM>
__device__ inline long long group_visible(const DecodeParams& p, int rg) {
    const Grp g = group_of<RM>(p, rg);
    long long total = 0;
    for (int f = 0; f < p.F; ++f) total += group_view_vis<KVM, RM>(p, f, g);
    return total;
}

// Page-cache fill of a chunk workgroup (kThreads threads): pages[i] = entry
// lp0 + i of the sequence's block_tables row bt, for i < kPageCap (-1 past the
// row or outside [0, num_blocks)).  Each thread issues all of its loads (on
// clamped, in-bounds indices) before the first is waited for, where a strided
// loop waited once per pass.  Returns whether this thread's entries up to
// logical page lpl are all valid.
__device__ inline bool fill_page_cache(const DecodeParams& p, const int* bt, int* pages, uint32_t lp0, uint32_t lpl) {
    constexpr int kIt = kPageCap / kThreads;
    static_assert(kIt * kThreads == kPageCap, "page cache entries per thread");
    const int tid = threadIdx.x;
    const uint32_t maxB = (uint32_t)p.maxB;
    int pg[kIt];
#pragma unroll
    for (int k = 0; k < kIt; ++k) {
        const uint32_t lp = lp0 + (uint32_t)(tid + k * kThreads);
        pg[k] = -1;
        if (maxB > 0) pg[k] = bt[lp < maxB ? lp : maxB - 1];
    }
    bool ok = true;
#pragma unroll
    for (int k = 0; k < kIt; ++k) {
        const uint32_t lp = lp0 + (uint32_t)(tid + k * kThreads);
        int v = lp < maxB ? pg[k] : -1;
        if (v < 0 || v >= p.nblocks) v = -1;
        pages[tid + k * kThreads] = v;
        if (lp <= lpl && v < 0) ok = false;
    }
    return ok;
}

__device__ inline uint32_t token_mask(int vis, int kb0) {
    const int lim = vis - kb0;
    return lim >= 32 ? 0xffffffffu : (lim <= 0 ? 0u : ((1u << lim) - 1u));
}

// Block (segment, token of the block): thread t -> head t/16, dims [(t%16)*8, +8).
// A segment without pieces (no visible key) writes zeros, as the decode merge does.
template <int DT, int RM>
__global__ __launch_bounds__(256) void dv_merge_chunk(const DecodeParams p) {
    using raw = typename Tr<DT>::raw;
    const int sg = blockIdx.x / kTokBlk;
    const int tb = blockIdx.x - sg * kTokBlk;
    const int base = p.dir[2 * sg], cnt = p.dir[2 * sg + 1];
    if (cnt == 1) return;
    const int NHG = p.Hkv;
    const int r = sg / NHG, hkv = sg - (sg / NHG) * NHG;
    const Grp gr = group_of<RM>(p, p.row_begin + r);
    if (tb >= gr.ntok) return;
    const int tid = threadIdx.x;
    const int n = tid >> 4;
    const int d[1] = {(tid & 15) * 8};
    const int h = hkv * kGqa + n;
    raw* o = reinterpret_cast<raw*>(p.out) + out_row<RM>(p, gr, tb, h) + d[0];
    float v[1][8];
    // rounds of 8 pieces: a chunk segment rarely has more (configuration 5: two),
    // and the 16-piece round's registers would cost this 256-thread kernel a
    // wave per SIMD of occupancy
    merge_runs_b<DT, 1, kMergeBatch>(p.part, p.slot_floats, kTokBlk * kGqa, tb * kGqa + n, d, base, cnt, v);
    store_run8<DT>(o, v[0]);
}

}  // namespace chunk

// fp32 launches of the chunk path (dv_chunk32.hip): the decode kernel and the
// split merge for rows [p.row_begin, p.row_begin + p.nrows) of row groups.
hipError_t launch_chunk32(int qmode, int kvmode, int rowmode, DecodeParams p, int device, int cus, long long cap,
                          hipStream_t stream);

}  // namespace dv
