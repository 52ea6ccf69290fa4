// Measurement probes (libdvattn_probe.so, used by `bench.py --read-ceiling`
// and `bench.py --mfma-ceiling`).
//
// Paged-read probe:
// the 16-bit decode kernel's K/V stream with the attention taken out.  It runs
// the decode's work split (run_schedule with the same start cost, XCD skew and
// minimum range), fills the same per-wave page-id cache and streams every
// visible K/V row of every piece through the same two-stage direct-to-LDS ring
// (stream::issue) with the same completion waits -- but computes nothing: each
// stage is consumed by one LDS word per lane.  Its rate is the HBM read rate
// the decode's access pattern (256-byte rows of randomly placed pages) can
// reach on the part, the ceiling the decode kernel is measured against.
//
// Single-view paged rows only (the configurations whose ceiling is reported).
#include <string.h>

#include <atomic>

#include "../../include/dvattn_amd.h"
#include "dv_common.h"
#include "dv_device.h"
#include "dv_schedule.h"
#include "dv_stream.h"

namespace dv {
namespace {

// One wave: KV head hkv over visible keys [v0, v1) of a one-view row (the
// decode's stream::piece minus the query, the MFMAs and the epilogue).
__device__ unsigned read_piece(const DecodeParams& p, unsigned char* wlds, int row, int hkv, long long v0,
                               long long v1, long long row_keys) {
    const int lane = threadIdx.x & 63;
    const uint32_t ring = __builtin_amdgcn_readfirstlane(lds_addr(wlds));
    int* pc = reinterpret_cast<int*>(wlds + stream::kRing * stream::kStage);
    const int w = row / p.S;
    unsigned acc = 0;
    if (row_keys <= 0 || v1 <= v0) return acc;
    stream::View v;
    v.hkv = hkv;
    v.k = reinterpret_cast<const unsigned char*>(p.kc);
    v.v = reinterpret_cast<const unsigned char*>(p.vc);
    v.off = 0;
    v.lp0 = 0;
    const int l0 = (int)v0, l1 = (int)(v1 < row_keys ? v1 : row_keys);
    const long long span = (long long)(stream::kPc - 1) * p.bs;
    for (int sa = l0; sa < l1;) {
        const int sb = (long long)l1 - sa > span ? (int)(sa + span) : l1;
        v.b = sb;
        uint32_t lpa, lpz, r;
        page_split(p, (uint32_t)sa, lpa, r);
        page_split(p, (uint32_t)(sb - 1), lpz, r);
        v.lp0 = (int)lpa;
        const int need = (int)(lpz - lpa) + 1;
        const int* bt = p.bt + (long long)w * p.maxB;
        for (int i = lane; i < need; i += kWave) {
            const uint32_t lp = lpa + (uint32_t)i;
            int pg = lp < (uint32_t)p.maxB ? bt[lp] : -1;
            if (pg < 0 || pg >= p.nblocks) pg = -1;
            pc[i] = pg;
        }
        const int n_st = (sb - sa + kStep - 1) / kStep;
        uint32_t m = stream::issue<kKvPaged>(p, v, pc, ring, sa);
        if (n_st > 1) m ^= stream::issue<kKvPaged>(p, v, pc, ring + stream::kStage, sa + kStep);
        for (int s = 0; s < n_st; ++s) {
            if (s + 1 < n_st) wait_vmcnt<16>();
            else wait_vmcnt<0>();
            acc += *reinterpret_cast<const unsigned*>(wlds + (s & 1) * stream::kStage + lane * 4) ^ m;
            if (s + 2 < n_st) {
                lds_wait();  // the slot's read is complete before it is refilled
                m = stream::issue<kKvPaged>(p, v, pc, ring + (uint32_t)((s & 1) * stream::kStage),
                                            sa + (s + 2) * kStep);
            }
        }
        lds_wait();
        sa = sb;
    }
    return acc;
}

__global__ __launch_bounds__(256) void dv_read_probe(const DecodeParams p, unsigned* sink) {
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ long long s_scan[4];
    const int wv = threadIdx.x >> 6;
    const int HPW = p.hpw;
    long long* s_pref = reinterpret_cast<long long*>(smem + HPW * stream::kWaveLds);
    unsigned char* wlds = smem + wv * stream::kWaveLds;
    unsigned acc = 0;
    run_schedule<true>(p, p.Hkv / HPW, s_pref, s_scan, [&](int row) { return row_visible<kKvPaged, kRowWS>(p, row); },
                 [&](int row, int hg, long long v0, long long v1, bool, int, long long rk) {
        if (wv < HPW) acc += read_piece(p, wlds, row, hg * HPW + wv, v0, v1, rk);
    });
    if ((threadIdx.x & 63) == 0) sink[blockIdx.x * kMaxWavesPerWg + wv] = acc;
}

// Plain streaming read of a contiguous buffer (16-byte loads, 8 per lane in
// flight per iteration, grid-stride), with the non-temporal or the default
// cache policy: the part's read rate for an access pattern with no paging, to
// set the paged probe's rate against.
template <bool NT>
__global__ __launch_bounds__(256) void dv_plain_read(const u32x4* __restrict__ buf, long long n16, unsigned* sink) {
    constexpr int U = 8;
    long long i = (long long)blockIdx.x * 256 * U + threadIdx.x;
    const long long stride = (long long)gridDim.x * 256 * U;
    unsigned acc = 0;
    for (; i + (U - 1) * 256 < n16; i += stride) {
        u32x4 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const gu32x4* q = (const gu32x4*)(buf + i + u * 256);
            v[u] = NT ? __builtin_nontemporal_load(q) : *q;
        }
#pragma unroll
        for (int u = 0; u < U; ++u) acc ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
    }
    if ((threadIdx.x & 63) == 0) sink[blockIdx.x * 4 + (threadIdx.x >> 6)] = acc;
}

// MFMA rate probe: back-to-back v_mfma_f32_16x16x32_bf16 on every SIMD (eight
// waves per CU, two per SIMD, as the chunk kernel runs; eight independent
// accumulator chains per wave) with N other instructions per MFMA, each on an
// independent register: fp32 FMAs (EXP false) or v_exp_f32 (EXP true).  Every
// wave records its shader-clock cycles (s_memtime) and 100 MHz reference ticks
// (s_memrealtime) over the loop, so the host can report the clock it ran at.
template <int N, bool EXP>
__global__ __launch_bounds__(512) void dv_mfma_rate(float* sink, unsigned long long* clocks, int iters) {
    constexpr int kChains = 8;
    constexpr int kX = N > 0 ? N : 1;
    const int lane = threadIdx.x & 63;
    const u32x4 a = {0x3f803f80u ^ (unsigned)lane, 0x3f003f00u, 0x3e803e80u + (unsigned)lane, 0x3f803f00u};
    const u32x4 b = {0x3f003f80u, 0x3e803f80u ^ (unsigned)(lane << 3), 0x3f803f80u, 0x3f003f00u};
    f32x4 c[kChains];
#pragma unroll
    for (int i = 0; i < kChains; ++i) c[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    float x[kX];
#pragma unroll
    for (int v = 0; v < kX; ++v) x[v] = (float)(lane + v) * 0.01f;
    const unsigned long long t0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int i = 0; i < kChains; ++i) {
            c[i] = Tr<kBF16>::mma(a, b, c[i]);
#pragma unroll
            for (int v = 0; v < N; ++v)
                x[v] = EXP ? __builtin_amdgcn_exp2f(x[v]) : __builtin_fmaf(x[v], 0.999f, 0.5f);
        }
    }
    const unsigned long long t1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
    float s = 0.f;
#pragma unroll
    for (int v = 0; v < kX; ++v) s += x[v];
#pragma unroll
    for (int i = 0; i < kChains; ++i) s += c[i][0] + c[i][1] + c[i][2] + c[i][3];
    sink[(size_t)blockIdx.x * blockDim.x + threadIdx.x] = s;
    const int w = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (lane == 0) {
        clocks[2 * w] = t1 - t0;
        clocks[2 * w + 1] = r1 - r0;
    }
}

// The same with v_mfma_f32_32x32x16_bf16 (twice the work per instruction,
// sixteen accumulators per lane): N other instructions per MFMA here equal N/2
// per 16x16x32-equivalent of matrix work.
typedef __attribute__((ext_vector_type(16))) float f32x16;

template <int N>
__global__ __launch_bounds__(512) void dv_mfma_rate32(float* sink, unsigned long long* clocks, int iters) {
    constexpr int kChains = 8;
    constexpr int kX = N > 0 ? N : 1;
    const int lane = threadIdx.x & 63;
    const u32x4 a = {0x3f803f80u ^ (unsigned)lane, 0x3f003f00u, 0x3e803e80u + (unsigned)lane, 0x3f803f00u};
    const u32x4 b = {0x3f003f80u, 0x3e803f80u ^ (unsigned)(lane << 3), 0x3f803f80u, 0x3f003f00u};
    f32x16 c[kChains];
#pragma unroll
    for (int i = 0; i < kChains; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) c[i][e] = 0.f;
    float x[kX];
#pragma unroll
    for (int v = 0; v < kX; ++v) x[v] = (float)(lane + v) * 0.01f;
    const unsigned long long t0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int i = 0; i < kChains; ++i) {
            c[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                           c[i], 0, 0, 0);
#pragma unroll
            for (int v = 0; v < N; ++v) x[v] = __builtin_fmaf(x[v], 0.999f, 0.5f);
        }
    }
    const unsigned long long t1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
    float s = 0.f;
#pragma unroll
    for (int v = 0; v < kX; ++v) s += x[v];
#pragma unroll
    for (int i = 0; i < kChains; ++i) s += c[i][0] + c[i][5] + c[i][10] + c[i][15];
    sink[(size_t)blockIdx.x * blockDim.x + threadIdx.x] = s;
    const int w = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (lane == 0) {
        clocks[2 * w] = t1 - t0;
        clocks[2 * w + 1] = r1 - r0;
    }
}

thread_local const char* g_msg = "";

}  // namespace
}  // namespace dv

extern "C" {

__attribute__((visibility("default"))) const char* dvprobe_last_error(void) { return dv::g_msg; }

// Streams the visible K/V rows of a single-view 16-bit paged call exactly as
// dvattn_paged_sdpa's decode kernel does (same split and launch shape) without
// computing attention.  Arguments as dvattn_paged_sdpa (locations [1,W,1],
// fragment_lengths [1], caches, block_tables, shape); `workspace` holds the
// split's merge directory (dvattn_paged_sdpa_workspace_size bytes suffice);
// `sink` receives one word per wave (4 per workgroup, sink_words >= 4 x CUs).
// Returns 0, or -1 with a message for dvprobe_last_error().
__attribute__((visibility("default"))) int dvprobe_paged_read(int dtype, const int* locations,
                                                               const int* fragment_lengths, const void* k_cache,
                                                               const void* v_cache, const int* block_tables,
                                                               const dvattn_shape* s, void* workspace,
                                                               size_t workspace_bytes, unsigned* sink,
                                                               long long sink_words, void* stream) {
    using namespace dv;
    if (!s || (dtype != DVATTN_BF16 && dtype != DVATTN_F16) || s->F != 1 || s->S != 1 || s->E != 128 ||
        s->Hq != 16 * s->Hkv || s->Hkv <= 0 || s->W <= 0 || s->W > kMaxRows || s->block_size <= 0) {
        g_msg = "probe: one-view 16-bit paged decode rows only (F = 1, S = 1, W <= 2048, GQA 16, E = 128)";
        return -1;
    }
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess) {
        g_msg = "probe: hipGetDevice failed";
        return -1;
    }
    DecodeParams p;
    memset(&p, 0, sizeof(p));
    p.loc = locations;
    p.fl = fragment_lengths;
    p.kc = k_cache;
    p.vc = v_cache;
    p.bt = block_tables;
    p.F = 1;
    p.W = s->W;
    p.S = 1;
    p.Hq = s->Hq;
    p.Hkv = s->Hkv;
    p.bs = s->block_size;
    p.bs_shift = -1;
    for (int sh = 0; sh < 31; ++sh)
        if ((1 << sh) == s->block_size) p.bs_shift = sh;
    p.maxB = s->max_blocks_per_seq;
    p.nblocks = s->num_blocks;
    p.hpw = pick_hpw(p.Hkv);
    p.piece_cost = kPieceCost;
    p.min_keys = kDecodeMinKeys;
    p.skew_pm = xcd_skew_pm();
    p.row_begin = 0;
    p.nrows = p.W;
    const int nhg = p.Hkv / p.hpw;
    if (workspace_bytes < (size_t)p.nrows * nhg * 2 * sizeof(int) || !workspace) {
        g_msg = "probe: workspace too small for the merge directory";
        return -1;
    }
    p.dir = reinterpret_cast<int*>(workspace);
    const size_t lds = (size_t)p.hpw * stream::kWaveLds + (size_t)(p.nrows + 1) * sizeof(long long);
    static std::atomic<unsigned long long> attr_done{0};
    hipError_t e = once_per_device(attr_done, device, [&] {
        const size_t max_lds = (size_t)kMaxWavesPerWg * stream::kWaveLds + (size_t)(kMaxRows + 1) * sizeof(long long);
        return hipFuncSetAttribute(reinterpret_cast<const void*>(&dv_read_probe),
                                   hipFuncAttributeMaxDynamicSharedMemorySize, (int)max_lds);
    });
    if (e != hipSuccess) {
        g_msg = "probe: hipFuncSetAttribute failed";
        return -1;
    }
    int per_cu = 1;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void*>(&dv_read_probe),
                                                     p.hpw * kWave, lds) != hipSuccess || per_cu < 1)
        per_cu = 1;
    // the decode's launch shape: one wave of resident workgroups, bounded by the work
    const int cus = device_cu_count(device);
    long long nwg = (long long)cus * per_cu;
    const long long max_wg = (long long)cus * (8 / p.hpw);
    if (nwg > max_wg) nwg = max_wg;
    const long long cap = ((long long)p.nrows * nhg * s->max_blocks_per_seq * s->block_size + p.min_keys - 1) /
                          p.min_keys;
    if (nwg > cap) nwg = cap;
    p.nwg = nwg < 1 ? 1 : (int)nwg;
    if (sink_words < (long long)p.nwg * kMaxWavesPerWg || !sink) {
        g_msg = "probe: sink too small (4 words per workgroup)";
        return -1;
    }
    hipLaunchKernelGGL(dv_read_probe, dim3(p.nwg), dim3(p.hpw * kWave), lds, (hipStream_t)stream, p, sink);
    if (hipGetLastError() != hipSuccess) {
        g_msg = "probe: launch failed";
        return -1;
    }
    g_msg = "";
    return 0;
}

// Reads `bytes` (a multiple of 32 KiB, 16-byte aligned) of `buf` once with
// 16-byte loads, non-temporal when `nontemporal` is set; `sink` receives 4 words
// per workgroup (sink_words >= 4 * 8192).  Returns 0, or -1 with a message.
__attribute__((visibility("default"))) int dvprobe_plain_read(const void* buf, size_t bytes, int nontemporal,
                                                               unsigned* sink, long long sink_words, void* stream) {
    using namespace dv;
    constexpr int kGrid = 8192;
    if (!buf || !sink || (bytes & 32767) || ((uintptr_t)buf & 15) || sink_words < 4ll * kGrid) {
        g_msg = "probe: plain read needs a 16-byte aligned buffer of a multiple of 32 KiB and 4 x 8192 sink words";
        return -1;
    }
    const long long n16 = (long long)(bytes / 16);
    const u32x4* b = reinterpret_cast<const u32x4*>(buf);
    if (nontemporal)
        hipLaunchKernelGGL(dv_plain_read<true>, dim3(kGrid), dim3(256), 0, (hipStream_t)stream, b, n16, sink);
    else
        hipLaunchKernelGGL(dv_plain_read<false>, dim3(kGrid), dim3(256), 0, (hipStream_t)stream, b, n16, sink);
    if (hipGetLastError() != hipSuccess) {
        g_msg = "probe: launch failed";
        return -1;
    }
    g_msg = "";
    return 0;
}

// MFMA 16x16x32 bf16 rate with `n_other` independent fp32 FMAs (exp = 0) or
// v_exp_f32 (exp = 1) per MFMA: one workgroup of eight waves per CU, `iters`
// rounds of eight MFMAs per wave.  n_other is 0, 1, 2, 3, 4 or 6 for FMAs and
// 1 or 2 for exponentials.  `sink` takes 512 floats per CU; `clocks` two words
// per wave (shader cycles, 100 MHz ticks; 16 per CU).  Returns the number of
// workgroups launched, or -1 with a message for dvprobe_last_error().
__attribute__((visibility("default"))) int dvprobe_mfma_rate(int n_other, int exp, int iters, float* sink,
                                                              long long sink_floats, unsigned long long* clocks,
                                                              long long clock_words, void* stream) {
    using namespace dv;
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess) {
        g_msg = "probe: no device";
        return -1;
    }
    const int cus = device_cu_count(device);
    if (!sink || !clocks || iters <= 0 || sink_floats < 512ll * cus || clock_words < 16ll * cus) {
        g_msg = "probe: mfma rate needs iters > 0, 512 sink floats and 16 clock words per CU";
        return -1;
    }
    void (*k)(float*, unsigned long long*, int) = nullptr;
    if (!exp) {
        switch (n_other) {
            case 0: k = dv_mfma_rate<0, false>; break;
            case 1: k = dv_mfma_rate<1, false>; break;
            case 2: k = dv_mfma_rate<2, false>; break;
            case 3: k = dv_mfma_rate<3, false>; break;
            case 4: k = dv_mfma_rate<4, false>; break;
            case 6: k = dv_mfma_rate<6, false>; break;
            default: break;
        }
    } else {
        if (n_other == 1) k = dv_mfma_rate<1, true>;
        if (n_other == 2) k = dv_mfma_rate<2, true>;
    }
    if (!k) {
        g_msg = "probe: unsupported mix (FMAs: 0, 1, 2, 3, 4, 6; exponentials: 1, 2)";
        return -1;
    }
    hipLaunchKernelGGL(k, dim3(cus), dim3(512), 0, (hipStream_t)stream, sink, clocks, iters);
    if (hipGetLastError() != hipSuccess) {
        g_msg = "probe: launch failed";
        return -1;
    }
    g_msg = "";
    return cus;
}

// dvprobe_mfma_rate with v_mfma_f32_32x32x16_bf16 and n_other fp32 FMAs per MFMA
// (0, 2, 4, 6, 8, 12).  Same arguments and return value.
__attribute__((visibility("default"))) int dvprobe_mfma_rate32(int n_other, int iters, float* sink,
                                                                long long sink_floats, unsigned long long* clocks,
                                                                long long clock_words, void* stream) {
    using namespace dv;
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess) {
        g_msg = "probe: no device";
        return -1;
    }
    const int cus = device_cu_count(device);
    if (!sink || !clocks || iters <= 0 || sink_floats < 512ll * cus || clock_words < 16ll * cus) {
        g_msg = "probe: mfma rate needs iters > 0, 512 sink floats and 16 clock words per CU";
        return -1;
    }
    void (*k)(float*, unsigned long long*, int) = nullptr;
    switch (n_other) {
        case 0: k = dv_mfma_rate32<0>; break;
        case 2: k = dv_mfma_rate32<2>; break;
        case 4: k = dv_mfma_rate32<4>; break;
        case 6: k = dv_mfma_rate32<6>; break;
        case 8: k = dv_mfma_rate32<8>; break;
        case 12: k = dv_mfma_rate32<12>; break;
        default: break;
    }
    if (!k) {
        g_msg = "probe: unsupported mix (FMAs: 0, 2, 4, 6, 8, 12)";
        return -1;
    }
    hipLaunchKernelGGL(k, dim3(cus), dim3(512), 0, (hipStream_t)stream, sink, clocks, iters);
    if (hipGetLastError() != hipSuccess) {
        g_msg = "probe: launch failed";
        return -1;
    }
    g_msg = "";
    return cus;
}

}  // extern "C"
