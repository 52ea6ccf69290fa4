// Cache-side kernels around the decode path:
//  * dv_kv_append -- rotate the new tokens' keys and write keys and values into
//    their cache rows (the K side of a decode step: attention.py:304 rotates
//    key_states with the model's (cos, sin), attention.py:141-152 appends them to
//    the sequence's own cache).  The same kernel with one (cos, sin) row
//    broadcast over all tokens is merge_caches' constant-offset re-rotation
//    (attention.py:245-251).
//  * dv_view_meta -- per (view, sequence, new token) locations and rotary
//    cos/sin on the device (attention.py:158-186: suffix sums of the segment
//    lengths in each sequence's segment order, then the model's rotary
//    embedding at those positions).
// Both are elementwise and HBM- or launch-bound; one thread per 16-byte run.
#include "dv_common.h"
#include "dv_device.h"

namespace dv {

namespace {

typedef __attribute__((address_space(1))) u32x4 gw_u32x4;

// N elements of X from / to global memory, 16 bytes at a time when the run is
// a multiple of 16 bytes (the launcher checks the alignment).
template <typename X, int N>
__device__ inline void load_run(const X* src, X (&dst)[N]) {
    if constexpr ((sizeof(X) * N) % 16 == 0) {
        constexpr int V = (int)(sizeof(X) * N / 16);
        u32x4 t[V];
#pragma unroll
        for (int i = 0; i < V; ++i) t[i] = ld16(reinterpret_cast<const unsigned char*>(src) + 16 * i);
        __builtin_memcpy(dst, t, sizeof(dst));
    } else {
#pragma unroll
        for (int i = 0; i < N; ++i) dst[i] = src[i];
    }
}

template <typename X, int N>
__device__ inline void store_run(X* dst, const X (&src)[N]) {
    if constexpr ((sizeof(X) * N) % 16 == 0) {
        constexpr int V = (int)(sizeof(X) * N / 16);
        u32x4 t[V];
        __builtin_memcpy(t, src, sizeof(t));
#pragma unroll
        for (int i = 0; i < V; ++i) *(gw_u32x4*)(reinterpret_cast<unsigned char*>(dst) + 16 * i) = t[i];
    } else {
#pragma unroll
        for (int i = 0; i < N; ++i) dst[i] = src[i];
    }
}

template <int DT>
__device__ inline float round_to(float f) {
    return Tr<DT>::tof(Tr<DT>::fromf(f));
}

// One rotated element as PyTorch evaluates attention.py:82-88,
// x_rot * cos + rotate_half(x_rot) * sin: each product and the sum are rounded
// to the promoted dtype of (x, cos) -- fp32 if either is fp32, else the 16-bit
// storage type -- and the result to the storage type.  `first`: dims [0, R/2),
// where rotate_half contributes -x[e + R/2].
template <int DT, int CDT>
__device__ inline float rope_elem(float x, float xp, float c, float s, bool first) {
#pragma clang fp contract(off)
    constexpr bool kF32Math = DT == kF32 || CDT == kF32;
    float a = x * c;
    float b = xp * s;
    if constexpr (!kF32Math) {
        a = round_to<DT>(a);
        b = round_to<DT>(b);
    }
    float y = first ? a - b : a + b;
    if constexpr (!kF32Math) y = round_to<DT>(y);
    return y;
}

}  // namespace

// Thread = one run of RUN dims of one (token, KV head) row; consecutive threads
// cover one row, so every warp-wide access is contiguous.  Tokens whose
// position is negative, past the block table row or on an invalid page are not
// written.
template <int DT, int CDT, int RUN>
__global__ __launch_bounds__(256) void dv_kv_append(const AppendParams p, uint32_t nruns, uint32_t runs) {
    using raw = typename Tr<DT>::raw;
    using craw = typename Tr<CDT>::raw;
    // 32-bit index arithmetic: the launcher keeps a launch below 2^31 runs
    const uint32_t idx = blockIdx.x * 256u + threadIdx.x;
    if (idx >= nruns) return;
    const uint32_t hr = idx / runs;
    const int d0 = (int)(idx - hr * runs) * RUN;
    const uint32_t n = hr / (uint32_t)p.Hkv;  // token index w*S + s
    const int h = (int)(hr - n * (uint32_t)p.Hkv);
    const int w = (int)(n / (uint32_t)p.S);
    const int s = (int)(n - (uint32_t)w * (uint32_t)p.S);
    // the token's inputs are loaded first, then the page lookup (positions,
    // then block_tables: two dependent loads) runs while they are in flight
    const int ps = p.pos[n];
    const bool has_k = d0 < p.E, has_v = d0 < p.Ev;
    const bool rot = has_k && d0 < p.R;
    const int half = p.R >> 1;
    const bool first = d0 < half;  // a rotated run lies within one half (R/2 % RUN == 0)
    raw xa[RUN], xb[RUN], vo[RUN];
    craw c[RUN], sn[RUN];
    if (has_k) {
        const raw* x = reinterpret_cast<const raw*>(p.k) + w * p.ks[0] + h * p.ks[1] + s * p.ks[2];
        load_run<raw, RUN>(x + d0, xa);
        if (rot) {
            const long long co = w * p.cs[0] + s * p.cs[1] + d0;
            load_run<raw, RUN>(x + (first ? d0 + half : d0 - half), xb);
            load_run<craw, RUN>(reinterpret_cast<const craw*>(p.cosv) + co, c);
            load_run<craw, RUN>(reinterpret_cast<const craw*>(p.sinv) + co, sn);
        }
    }
    if (has_v)
        load_run<raw, RUN>(reinterpret_cast<const raw*>(p.v) + w * p.vs[0] + h * p.vs[1] + s * p.vs[2] + d0, vo);
    if (ps < 0) return;
    const int lp = ps / p.bs;
    if (lp >= p.maxB) return;
    const int page = p.bt[(long long)w * p.maxB + lp];
    if (has_k && rot) {
#pragma unroll
        for (int e = 0; e < RUN; ++e)
            xa[e] = Tr<DT>::fromf(rope_elem<DT, CDT>(Tr<DT>::tof(xa[e]), Tr<DT>::tof(xb[e]), Tr<CDT>::tof(c[e]),
                                                     Tr<CDT>::tof(sn[e]), first));
    }
    if (page < 0 || page >= p.nblocks) return;
    const long long row = ps - (long long)lp * p.bs;
    if (has_k)
        store_run<raw, RUN>(reinterpret_cast<raw*>(p.kc) + page * p.kcs[0] + row * p.kcs[1] + h * p.kcs[2] + d0, xa);
    if (has_v)
        store_run<raw, RUN>(reinterpret_cast<raw*>(p.vc) + page * p.vcs[0] + row * p.vcs[1] + h * p.vcs[2] + d0, vo);
}

template <int DT, int CDT, int RUN>
hipError_t append_go(const AppendParams& p, hipStream_t stream) {
    const int E = p.E > p.Ev ? p.E : p.Ev;
    const int runs = (E + RUN - 1) / RUN;
    const long long nruns = (long long)p.W * p.S * p.Hkv * runs;
    if (nruns == 0) return hipSuccess;
    if (nruns >= (1ll << 31)) return hipErrorInvalidValue;  // the C ABI rejects such calls first
    const long long blocks = (nruns + 255) / 256;
    hipLaunchKernelGGL((dv_kv_append<DT, CDT, RUN>), dim3((unsigned)blocks), dim3(256), 0, stream, p,
                       (uint32_t)nruns, (uint32_t)runs);
    return hipGetLastError();
}

template <int DT, int CDT>
hipError_t append_dispatch(const AppendParams& p, hipStream_t stream) {
    constexpr int kRun = DT == kF32 ? 4 : 8;
    constexpr int kEs = Tr<DT>::kBytes, kCs = Tr<CDT>::kBytes;
    auto al = [](const void* ptr) { return ((uintptr_t)ptr & 15) == 0; };
    auto st = [](long long stride, int bytes) { return (stride * bytes) % 16 == 0; };
    bool vec = p.E % kRun == 0 && p.Ev % kRun == 0 && (p.R / 2) % kRun == 0;
    vec = vec && al(p.kc) && al(p.vc) && al(p.k) && al(p.v) && al(p.cosv) && al(p.sinv);
    for (int i = 0; i < 3; ++i)
        vec = vec && st(p.kcs[i], kEs) && st(p.vcs[i], kEs) && st(p.ks[i], kEs) && st(p.vs[i], kEs);
    vec = vec && st(p.cs[0], kCs) && st(p.cs[1], kCs);
    if (vec) return append_go<DT, CDT, kRun>(p, stream);
    return append_go<DT, CDT, 1>(p, stream);
}

hipError_t launch_kv_append(int dtype, int rope_dtype, const AppendParams& p, hipStream_t stream) {
    const bool f32rope = rope_dtype == kF32;
    switch (dtype) {
        case kBF16: return f32rope ? append_dispatch<kBF16, kF32>(p, stream) : append_dispatch<kBF16, kBF16>(p, stream);
        case kF16: return f32rope ? append_dispatch<kF16, kF32>(p, stream) : append_dispatch<kF16, kF16>(p, stream);
        case kF32: return append_dispatch<kF32, kF32>(p, stream);
        default: return hipErrorInvalidValue;
    }
}

// Thread = (view f, sequence w, new token s, rotary pair i).  The location of
// view f for sequence w is the total length of w's segments from f's place in
// its segment order to the last one, minus the new tokens, plus s
// (attention.py:167-176 walks the order backwards accumulating lengths that
// already include the new tokens).  cos/sin follow the rotary embedding of
// transformers: angle = fp32(position) * inv_freq[i] (one fp32 product),
// cos/sin of it times the attention scaling, the same value in both halves.
// A view missing from w's order gets location -1 and the identity rotation.
__global__ __launch_bounds__(256) void dv_view_meta(const MetaParams p, long long n, int rh) {
    const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= n) return;
    const int i = (int)(idx % rh);
    const long long t = idx / rh;  // (f*W + w)*S + s
    const int s = (int)(t % p.S);
    const long long fw = t / p.S;
    const int w = (int)(fw % p.W);
    const int f = (int)(fw / p.W);
    // the whole row is walked: if f appears more than once, its first place
    // wins, as in the reference, whose backward walk assigns it last
    long long suffix = 0, at = 0;
    bool found = false;
    const int* ord = p.order + (long long)w * p.F;
    for (int j = p.F - 1; j >= 0; --j) {
        const int g = ord[j];
        if (g >= 0 && g < p.F) suffix += p.fl[g];
        if (g == f) {
            found = true;
            at = suffix;
        }
    }
    const int loc = found ? (int)(at - p.S + s) : -1;
    if (i == 0) p.loc[t] = loc;
    if (p.R > 0) {
        float c = 1.0f, sn = 0.0f;
        if (found) {
            const float ang = (float)loc * p.inv_freq[i];
            c = cosf(ang) * p.scaling;
            sn = sinf(ang) * p.scaling;
        }
        if (p.round_dt == kBF16) {
            c = round_to<kBF16>(c);
            sn = round_to<kBF16>(sn);
        } else if (p.round_dt == kF16) {
            c = round_to<kF16>(c);
            sn = round_to<kF16>(sn);
        }
        const long long o = t * p.R;
        p.cosv[o + i] = c;
        p.cosv[o + i + rh] = c;
        p.sinv[o + i] = sn;
        p.sinv[o + i + rh] = sn;
    }
}

hipError_t launch_view_meta(const MetaParams& p, hipStream_t stream) {
    const int rh = p.R > 0 ? p.R / 2 : 1;
    const long long n = (long long)p.F * p.W * p.S * rh;
    if (n == 0) return hipSuccess;
    const long long blocks = (n + 255) / 256;
    hipLaunchKernelGGL(dv_view_meta, dim3((unsigned)blocks), dim3(256), 0, stream, p, n, rh);
    return hipGetLastError();
}

}  // namespace dv
