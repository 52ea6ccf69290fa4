// gfx950 fp32 multi-query attention with fused query RoPE: fp32 calls with
// S >= 2 query tokens per sequence (paged, contiguous) or packed varlen tokens
// of several per sequence.  Same operator semantics as the decode kernels
// (src/kernels/paged_kernel_v21.cuh:17-374, varlen_paged_kernel_v21.cuh:17-371,
// kernel_v21.cuh:17-367 in the reference repository, which re-read K/V once per
// query token: grid.y = W*S, paged_kernel_v21.cuh:391).  Built without the
// VGPR-form MFMA flag of dv_chunk.hip.
#include "dv_chunk.h"

namespace dv {
namespace chunk {

// ---- fp32 multi-query kernel ------------------------------------------------------
//
// fp32 calls with several query tokens per sequence: the row groups (up to 16
// tokens of one sequence), work split, partial slots and merge
// (dv_merge_chunk<kF32>) of dv_chunk, with the fp32 decode's arithmetic
// (16x16x4 fp32 MFMA, softmax32).  Workgroup = four waves, one per SIMD (each
// holds 4 tiles of O^T accumulators and query operands: 256 registers), on one
// (row group, KV head) and a key range of it; wave w owns the group's tokens
// w, w + 4, w + 8 and w + 12 (query tiles of 16 heads).  K/V rows stream
// through a three-stage LDS ring (32 keys of K and of V per stage, 32 KiB)
// filled by direct-to-LDS loads, each wave issuing a quarter of every stage,
// with one workgroup barrier per stage; every wave then reads each stage's K
// and V^T operands from LDS once for all of its tiles.  A row group's K/V rows are
// thus read from HBM once per 16 tokens, where the fp32 decode kernel reads
// them once per token, as the reference does (paged_kernel_v21.cuh:391).
// Rows are 512 bytes with their 16-byte chunks XOR-swizzled by the row's low
// four bits, so the sixteen rows one operand read touches hit different banks.
constexpr int kWaves32 = 8;
constexpr int kT32 = kTokBlk / kWaves32;     // query tiles per wave
constexpr int kRow32 = 512;                  // bytes of one fp32 K or V row
constexpr int kKv32Bytes = kStep * kRow32;   // one stage of K (or of V): 16 KiB
constexpr int kSt32Bytes = 2 * kKv32Bytes;   // K then V
constexpr int kRing32 = 3;                   // stages in the ring: two in flight ahead of the one computed
constexpr int kDma32 = 4;                    // direct-to-LDS loads per wave and stage (2 K + 2 V)

struct Tile32 {
    f32x4 o[8];
    float m, l;
};

// LDS position of 16-byte chunk c of key row r of a stage.
__device__ inline int swz32(int r, int c) { return c ^ (r & 15); }

__device__ inline f32x4 lds_read16f_at(uint32_t addr) {
    typedef __attribute__((address_space(3))) const f32x4 lds_f32x4;
    return *(lds_f32x4*)(uintptr_t)addr;
}
__device__ inline float lds_read4f_at(uint32_t addr) {
    typedef __attribute__((address_space(3))) const float lds_f32;
    return *(lds_f32*)(uintptr_t)addr;
}

// Element offset of key l's fp32 row (KV head r.hkv), or -1 when it has none.
template <int KVM, bool P2>
__device__ inline long long row32(const DecodeParams& p, const Range& r, const int* pages, int l) {
    if (KVM == kKvPaged) {
        const uint32_t pos = (uint32_t)(r.off + l);
        uint32_t lp, rr;
        if (P2) {
            lp = pos >> p.bs_shift;
            rr = pos & ((1u << p.bs_shift) - 1u);
        } else {
            lp = pos / (uint32_t)p.bs;
            rr = pos - lp * (uint32_t)p.bs;
        }
        const uint32_t idx = lp - r.lp0;
        const int pg = pages[idx < (uint32_t)kPageCap ? idx : (uint32_t)(kPageCap - 1)];
        const bool ok = l < r.b && idx < (uint32_t)kPageCap && pg >= 0;
        const long long rowidx = ((long long)pg * p.bs + rr) * p.Hkv + r.hkv;
        return ok ? rowidx * kHeadDim : -1;
    } else {
        return l < r.b ? r.bstride + ((long long)r.hkv * r.L + l) * kHeadDim : -1;
    }
}

// This wave's quarter of stage st (keys kb0 .. kb0 + 31): K and V rows 8w .. 8w + 7,
// two rows per instruction; lane l writes chunk position l % 32 of row
// 8w + 2j + l / 32, fetching the chunk the swizzle puts there.  Rows without
// K/V (past the range, invalid page) load a row of zeros.
template <int KVM, bool P2>
__device__ inline void issue32(const DecodeParams& p, const Range& r, const int* pages, uint32_t ring, int st,
                               int kb0) {
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const uint32_t sbase = ring + (uint32_t)(st % kRing32) * kSt32Bytes;
    const float* zero = reinterpret_cast<const float*>(zrow);
#pragma unroll
    for (int j = 0; j < kDma32 / 2; ++j) {
        const int row = wv * (kStep / kWaves32) + j * 2 + (lane >> 5);
        const int c = swz32(row, lane & 31);
        const long long e = row32<KVM, P2>(p, r, pages, kb0 + row);
        const float* kp = e >= 0 ? reinterpret_cast<const float*>(r.k) + e + c * 4 : zero + c * 4;
        const float* vp = e >= 0 ? reinterpret_cast<const float*>(r.v) + e + c * 4 : zero + c * 4;
        const uint32_t off = (uint32_t)(wv * (kStep / kWaves32) + j * 2) * kRow32;
        dma16(kp, __builtin_amdgcn_readfirstlane(sbase + off));
        dma16(vp, __builtin_amdgcn_readfirstlane(sbase + kKv32Bytes + off));
    }
}

// Bit k: key kb0 + k has a K/V row.
template <int KVM, bool P2>
__device__ inline uint32_t mask32(const DecodeParams& p, const Range& r, const int* pages, int kb0) {
    const int lane = threadIdx.x & 63;
    const bool ok = row32<KVM, P2>(p, r, pages, kb0 + (lane & 31)) >= 0;
    return (uint32_t)ballot(ok && lane < 32);
}

// One stage (slot) for this wave's nt tiles: S^T = K Q^T (lane (g, m): K row
// kb*16 + m, dims cc*16 + g*4 .. +3, one LDS read for both tiles), the online
// softmax, O^T += V^T P^T (4 keys per MFMA: k = g <-> key kb*16 + g*4 + i; lane
// (g, n) reads dim cc*16 + n of that key's V row, once for both tiles).  The
// swizzle only changes address bits 4-8, so each read is a per-lane base XOR
// (cc << 6) plus a constant; the bases come from opaque_tid() so the compiler
// recomputes them per stage instead of holding 80 precomputed offsets.
__device__ inline void compute32(const unsigned char* slot, int nt, uint32_t okm, int kb0, const int (&vis_t)[kT32],
                                 const f32x4 (&qB)[kT32][8], Tile32 (&tl)[kT32], float l2) {
    const int lane = opaque_tid() & 63;
    const int g = lane >> 4, m = lane & 15, n = lane & 15;
    const uint32_t sb = lds_addr(slot);
    // K row m: chunk (cc*4 + g) ^ m sits at m*512 + 16 * (((cc ^ (m >> 2)) << 2) | (g ^ (m & 3)))
    const uint32_t kbase = sb + (uint32_t)(m * kRow32 + (((m >> 2) << 2) | (g ^ (m & 3))) * 16);
    f32x4 s[kT32][2];
#pragma unroll
    for (int t = 0; t < kT32; ++t) s[t][0] = s[t][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int cc = 0; cc < 8; ++cc)
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            // an opaque base per read: the reads are not all hoisted ahead of the
            // MFMAs (16 x 4 registers held at once)
            uint32_t ka = (kbase ^ (uint32_t)(cc << 6)) + (uint32_t)(kb * 16 * kRow32);
            asm volatile("" : "+v"(ka));
            const f32x4 kv = lds_read16f_at(ka);
#pragma unroll
            for (int t = 0; t < kT32; ++t) {
                if (t >= nt) continue;
#pragma unroll
                for (int jj = 0; jj < 4; ++jj) s[t][kb] = Tr<kF32>::mma1(kv[jj], qB[t][cc][jj], s[t][kb]);
            }
        }
    float pr[kT32][8];
#pragma unroll
    for (int t = 0; t < kT32; ++t) {
        if (t >= nt) continue;
        softmax32(tl[t].o, tl[t].m, tl[t].l, s[t][0], s[t][1], okm & token_mask(vis_t[t], kb0), l2, pr[t]);
    }
    // V row kb*16 + g*4 + i: dim cc*16 + n is word n % 4 of chunk (cc*4 + n/4) ^ (g*4 + i),
    // at row*512 + 16 * ((((cc ^ g) << 2) | ((n >> 2) ^ i))) + 4 * (n % 4)
    const uint32_t vb = sb + (uint32_t)kKv32Bytes + (uint32_t)(g * 4 * kRow32 + (g << 6) + (n & 3) * 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t vbi = vb + (uint32_t)((((n >> 2) ^ i) << 4));
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            float v[8];
#pragma unroll
            for (int cc = 0; cc < 8; ++cc)
                v[cc] = lds_read4f_at((vbi ^ (uint32_t)(cc << 6)) + (uint32_t)((kb * 16 + i) * kRow32));
#pragma unroll
            for (int t = 0; t < kT32; ++t) {
                if (t >= nt) continue;
                const float pb = pr[t][kb * 4 + i];
#pragma unroll
                for (int cc = 0; cc < 8; ++cc) tl[t].o[cc] = Tr<kF32>::mma1(v[cc], pb, tl[t].o[cc]);
            }
        }
    }
}

// Keys [sa, sbnd) of the current view: the stage loop.  Ring slot i % 3 holds
// stage i; per stage every wave waits for its own share, the workgroup barrier
// then guarantees the whole stage has landed and that every wave is done with
// stage i - 1, whose slot the loads of stage i + 2 then refill.  Loads past the
// range end fetch rows of zeros, so the loop needs no tail branch.
template <int KVM, bool P2>
__device__ inline void stream32(const DecodeParams& p, const Range& r, const int* pages, unsigned char* smem, int sa,
                                int sbnd, int nt, const int (&vis_t)[kT32], const f32x4 (&qB)[kT32][8],
                                Tile32 (&tl)[kT32]) {
    const uint32_t ring = lds_addr(smem);
    const int nsteps = (sbnd - sa + kStep - 1) / kStep;
    issue32<KVM, P2>(p, r, pages, ring, 0, sa);
    issue32<KVM, P2>(p, r, pages, ring, 1, sa + kStep);
    for (int i = 0; i < nsteps; ++i) {
        wait_vmcnt<kDma32>();  // own share of stage i landed (stage i + 1 may still be in flight)
        __syncthreads();
        issue32<KVM, P2>(p, r, pages, ring, i + 2, sa + (i + 2) * kStep);
        const int kb0 = sa + i * kStep;
        const uint32_t okm = mask32<KVM, P2>(p, r, pages, kb0);
        if (nt > 0) compute32(smem + (i % kRing32) * kSt32Bytes, nt, okm, kb0, vis_t, qB, tl, p.l2scale);
    }
    wait_vmcnt<0>();  // the trailing stages land before the ring is reused
    __syncthreads();
}

// One workgroup: keys [v0, v1) of row group rg for KV head hkv (fp32).
template <int QM, int KVM, bool P2, int RM>
__device__ void chunk32_piece(const DecodeParams& p, unsigned char* smem, int* pages, int rg, int hkv, long long v0,
                              long long v1, bool final_out, int slot) {
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int g = lane >> 4, n = lane & 15;
    const Grp gr = group_of<RM>(p, rg);
    const int w = gr.w;
    // this wave's tiles: tokens wv + kWaves32 * t of the group
    const int nt = gr.ntok > wv ? (gr.ntok - wv + kWaves32 - 1) / kWaves32 : 0;

    Tile32 tl[kT32];
#pragma unroll
    for (int t = 0; t < kT32; ++t) {
#pragma unroll
        for (int c = 0; c < 8; ++c) tl[t].o[c] = f32x4{0.f, 0.f, 0.f, 0.f};
        tl[t].m = -DV_INF;
        tl[t].l = 0.0f;
    }

    long long P = 0, off = 0;
    for (int f = 0; f < p.F && P < v1; ++f) {
        const int vis_blk = group_view_vis<KVM, RM>(p, f, gr);
        int vis_t[kT32];
#pragma unroll
        for (int t = 0; t < kT32; ++t)
            vis_t[t] = __builtin_amdgcn_readfirstlane(
                t < nt ? view_vis<KVM>(p, f, loc_of<RM>(p, f, gr, wv + kWaves32 * t)) : 0);
        const long long a = v0 > P ? v0 : P;
        const long long bnd = v1 < P + vis_blk ? v1 : P + vis_blk;
        if (a < bnd) {
            f32x4 qB[kT32][8];
#pragma unroll
            for (int t = 0; t < kT32; ++t) {
                if (t < nt) {
                    load_q32<QM, RM>(p, gr.lin + wv + kWaves32 * t, f, hkv, qB[t]);
                } else {
#pragma unroll
                    for (int c = 0; c < 8; ++c) qB[t][c] = f32x4{0.f, 0.f, 0.f, 0.f};
                }
            }
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
            const int span = KVM == kKvPaged ? (p.bs_shift >= 0 ? (kPageCap - 2) << p.bs_shift : (kPageCap - 2) * p.bs)
                                             : (1 << 30);
            for (int sa = la; sa < lb; sa += span) {
                const int sbnd = sa + span < lb ? sa + span : lb;
                r.b = sbnd;
                r.pages_ok = true;
                if (KVM == kKvPaged) {
                    const uint32_t p0 = (uint32_t)(off + sa);
                    r.lp0 = p.bs_shift >= 0 ? (p0 >> p.bs_shift) : p0 / (uint32_t)p.bs;
                    __syncthreads();  // every wave is done with the previous sub-range's page ids
                    static_assert(kWaves32 * kWave == kThreads, "one page-cache fill per workgroup");
                    fill_page_cache(p, p.bt + (long long)w * p.maxB, pages, r.lp0, 0u);
                    __syncthreads();
                }
                stream32<KVM, P2>(p, r, pages, smem, sa, sbnd, nt, vis_t, qB, tl);
            }
        }
        P += vis_blk;
        off += p.fl[f];
    }

    // epilogue: per tile, normalise and write the output or a partial slot
#pragma unroll
    for (int t = 0; t < kT32; ++t) {
        if (t >= nt) continue;
        const int tb = wv + kWaves32 * t;  // token within the group
        const float lt = rows4_sum(tl[t].l);
        const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
        const int h = hkv * kGqa + n;
        if (final_out) {
            float* o = reinterpret_cast<float*>(p.out) + out_row<RM>(p, gr, tb, h);
#pragma unroll
            for (int c = 0; c < 8; ++c) *reinterpret_cast<f32x4*>(o + c * 16 + g * 4) = tl[t].o[c] * inv;
        } else {
            store_partial<kF32>(p.part + (long long)slot * p.slot_floats, kTokBlk * kGqa, tb * kGqa + n, g, tl[t].o,
                                inv, lt > 0.0f ? tl[t].m + log2f(lt) : -DV_INF);
        }
    }
}

template <int QM, int KVM, bool P2, int RM>
__global__ __launch_bounds__(kWaves32 * kWave) void dv_chunk32(const DecodeParams p) {
    extern __shared__ __align__(16) unsigned char smem_raw[];
    // the ring starts at a 512-byte aligned LDS address (compute32's operand
    // addresses XOR address bits 6-8 of the row bases)
    unsigned char* smem = smem_raw + ((512u - (lds_addr(smem_raw) & 511u)) & 511u);
    int* pages = reinterpret_cast<int*>(smem + kRing32 * kSt32Bytes);
    long long* s_scan = reinterpret_cast<long long*>(smem + kRing32 * kSt32Bytes + kPageCap * 4);
    long long* s_pref = s_scan + kWaves32;
    run_schedule(p, p.Hkv, s_pref, s_scan, [&](int rg) { return group_visible<KVM, RM>(p, rg); },
                 [&](int rg, int hg, long long v0, long long v1, bool fin, int slot, long long) {
                     chunk32_piece<QM, KVM, P2, RM>(p, smem, pages, rg, hg, v0, v1, fin, slot);
                 });
}

size_t lds_bytes32(int nrows) {
    return 512 + (size_t)kRing32 * kSt32Bytes + (size_t)kPageCap * 4 + (size_t)(kWaves32 + nrows + 1) * sizeof(long long);
}


template <int QM, int KVM, bool P2, int RM>
hipError_t launch1_f32(DecodeParams p, int device, int cus, long long cap, hipStream_t stream) {
    const void* kern = reinterpret_cast<const void*>(&dv_chunk32<QM, KVM, P2, RM>);
    static std::atomic<unsigned long long> attr_done{0};
    hipError_t ea = once_per_device(attr_done, device, [kern] {
        return hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds_bytes32(kMaxRows));
    });
    if (ea != hipSuccess) return ea;
    const size_t lds = lds_bytes32(p.nrows);
    long long nwg = cus;  // one four-wave workgroup per CU (registers: one wave per SIMD)
    if (nwg > cap) nwg = cap;
    p.nwg = nwg < 1 ? 1 : (int)nwg;
    hipLaunchKernelGGL((dv_chunk32<QM, KVM, P2, RM>), dim3(p.nwg), dim3(kWaves32 * kWave), lds, stream, p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((dv_merge_chunk<kF32, RM>), dim3(p.nrows * p.Hkv * kTokBlk), dim3(256), 0, stream, p);
    return hipGetLastError();
}

}  // namespace chunk

hipError_t launch_chunk32(int qmode, int kvmode, int rowmode, DecodeParams p, int device, int cus, long long cap,
                          hipStream_t stream) {
    using namespace chunk;
    const bool p2 = kvmode == kKvPaged && p.bs_shift >= 0;
    if (rowmode == kRowVarlen) {
        if (qmode == kQRotHalf && kvmode == kKvPaged)
            return p2 ? launch1_f32<kQRotHalf, kKvPaged, true, kRowVarlen>(p, device, cus, cap, stream)
                      : launch1_f32<kQRotHalf, kKvPaged, false, kRowVarlen>(p, device, cus, cap, stream);
        return hipErrorInvalidValue;
    }
    if (qmode == kQRotFull && kvmode == kKvPaged)
        return p2 ? launch1_f32<kQRotFull, kKvPaged, true, kRowWS>(p, device, cus, cap, stream)
                  : launch1_f32<kQRotFull, kKvPaged, false, kRowWS>(p, device, cus, cap, stream);
    if (qmode == kQPre && kvmode == kKvContig)
        return launch1_f32<kQPre, kKvContig, false, kRowWS>(p, device, cus, cap, stream);
    return hipErrorInvalidValue;
}

}  // namespace dv
