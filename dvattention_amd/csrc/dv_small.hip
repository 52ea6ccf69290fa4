// Single-launch attention for short contiguous views (ops dvattn_sdpa and
// dvattn_fused, fp32 / fp16 / bf16): the query rotation, the attention and the
// merge of the key chunks in one kernel, where the general path (dv_decode.hip) takes a
// rotation launch, a decode launch whose every workgroup first computes the
// whole work split, and a merge launch.  Same operator semantics as
// src/kernels/kernel_v21.cuh:17-414 and src/binding.cu:356-372 (reference
// repository): rotated query per view, softmax over the visible keys of all
// views, zeros for a query with no visible key.
//
//  * Work: the tensor keys of every view are cut into chunks of kSmallChunk; a
//    workgroup takes one chunk of one (query row, KV head) item, its four waves
//    16 keys each.  The chunk boundaries depend only on the fragment tensor
//    lengths (host-known), so every K/V address is known at launch: a
//    workgroup issues its K/V, query, cos/sin and location loads together and
//    masks the keys past the view's visible count afterwards.
//  * A wave computes S^T = K Q^T for its 16 keys x 16 query heads on the fp32
//    MFMA (16x16x4, dims as the reduction index), the softmax of each head over
//    its keys, and O = P V with V read straight from global memory (a lane
//    loads 4 consecutive dims, so output column n of the t-th MFMA is dim
//    64 b + 4 n + t).  The four waves are combined in LDS.  16-bit inputs are
//    widened to fp32 in registers (exactly) and take the same fp32 arithmetic;
//    the rotated query is rounded to the storage type first, as the
//    reference's rq tensor is, and the output is rounded once at the end.
//  * Merge: a workgroup stores its chunk's normalised output and base-2
//    log-sum-exp, then raises its arrival flag and reads the flags of all the
//    item's chunks; a workgroup that finds them all raised merges every chunk
//    of the item and writes the output.  A flag is raised by writing the
//    call's tag, a per-call 48-bit value, so flags need no clearing before a
//    call (a word left by an earlier call, or arbitrary workspace bytes, hold
//    another value); a merging workgroup lowers the item's flags to zero, so
//    the same tag replayed (a captured graph) starts from lowered flags too.
//  * Cost of the merge protocol: the agent-scope fences write back and
//    invalidate the L2 of the workgroup's XCD, work that grows with the
//    number of workgroups in flight (measured: +2-3 us at 64 workgroups of
//    several chunks, +18 us at 256).  The host therefore sends a call here
//    only when it has a single chunk per item (one view of at most
//    kSmallChunk keys: no merge, no fence) or when items x chunks is small
//    (dv_capi.hip: small_path_chunks); larger calls take the general path.
#include <string.h>

#include <atomic>
#include <type_traits>

#include "dv_common.h"
#include "dv_device.h"
#include "dv_stream.h"

namespace dv {
namespace small {

constexpr int kWaves = 4;
constexpr int kKeysPerWave = kSmallChunk / kWaves;  // 16: one MFMA key block
constexpr int kSlot = kGqa * (kHeadDim + 1);         // floats per partial: 16 x 128 outputs, 16 LSE
constexpr int kMergeBatch = 8;                       // partials loaded together by the merge
static_assert(kKeysPerWave == 16, "one 16-key MFMA block per wave");

struct Smem {
    float q[kGqa][kHeadDim];          // the item's query rows (unrotated in rotating mode; 16-bit
                                      // types: [kGqa][kHeadDim] raw elements in the first half)
    float cs[kHeadDim], sn[kHeadDim]; // cos / sin row (rotating mode)
    float spare[4];                   // written by threads without a cos/sin part (store_query)
    float o[kWaves][kGqa][kHeadDim];  // each wave's unnormalised output
    float m[kWaves][kGqa];            // its per-head max (base-2 scores)
    float l[kWaves][kGqa];            // its per-head sum of exp2(score - max)
    int last;
};

// Four 16-bit values (8 bytes) widened to fp32 (exact).
template <int DT>
__device__ inline f32x4 widen4(u32x2 v) {
    if constexpr (DT == kBF16) {
        return f32x4{__uint_as_float(v[0] << 16), __uint_as_float(v[0] & 0xffff0000u), __uint_as_float(v[1] << 16),
                     __uint_as_float(v[1] & 0xffff0000u)};
    } else {
        // the words are copied to scalars first: a bit cast of a vector
        // element (v[1], v.y) is compiled into a cast of element 0
        const uint32_t lo = v[0], hi = v[1];
        const f16x2 a = __builtin_bit_cast(f16x2, lo);
        const f16x2 b = __builtin_bit_cast(f16x2, hi);
        return f32x4{(float)a[0], (float)a[1], (float)b[0], (float)b[1]};
    }
}

typedef __attribute__((address_space(1))) const u32x2 gu32x2;

// Four consecutive elements of a K/V row as loaded (fp32: f32x4; 16-bit: two
// words), widened where they are used: a conversion next to the loads is
// scheduled between them, and the loads after it then wait for the earlier ones.
template <int DT>
using Run4 = typename std::conditional<DT == kF32, f32x4, u32x2>::type;

// The run at element offset `e` of `row` (non-temporal: read once per call).
template <int DT>
__device__ inline Run4<DT> ld4_nt(const void* row, int e) {
    if constexpr (DT == kF32)
        return ld16f_nt(reinterpret_cast<const float*>(row) + e);
    else
        return __builtin_nontemporal_load((gu32x2*)(reinterpret_cast<const uint16_t*>(row) + e));
}

template <int DT>
__device__ inline f32x4 run_f32(Run4<DT> r) {
    if constexpr (DT == kF32)
        return r;
    else
        return widen4<DT>(r);
}

// Query rows of the item, staged in LDS: thread t loads dims (t%16)*8 .. +7
// of head t/16 (rotated queries [F,W,Hq,S,E] in kQPre mode, queries
// [W,Hq,S,E] otherwise), and in rotating mode threads 0..R/4-1 the cos row,
// threads 64..64+R/4-1 the sin row of (view, sequence, token).  Loaded into
// registers first (load_query), stored to LDS after the K/V loads have been
// issued (store_query), so every global load of the workgroup is in flight
// at once.
struct QStage {
    f32x4 a, b, c;  // fp32 query run (a, b) or 16-bit run (u), cos/sin run (c)
    u32x4 u;
    bool trig;
};

template <int DT, int QM>
__device__ inline QStage load_query(const DecodeParams& p, int w, int s, int f, int hkv) {
    const int tid = threadIdx.x;
    const int hh = tid >> 4, dd = (tid & 15) * 8;
    const long long qrow = QM == kQPre ? ((((long long)f * p.W + w) * p.Hq + hkv * kGqa + hh) * p.S + s) * kHeadDim
                                       : (((long long)w * p.Hq + hkv * kGqa + hh) * p.S + s) * kHeadDim;
    QStage r;
    if constexpr (DT == kF32) {
        const float* q = reinterpret_cast<const float*>(p.q) + qrow + dd;
        r.a = ld16f(q);
        r.b = ld16f(q + 4);
    } else {
        r.u = ld16(reinterpret_cast<const uint16_t*>(p.q) + qrow + dd);
    }
    const int j = tid & 63;
    r.trig = QM != kQPre && tid < 128 && j * 4 < p.R;
    // a select of the address rather than a branch around the load, so the
    // waits of the loads after it stay partial
    const long long co = (((long long)f * p.W + w) * p.S + s) * p.R + j * 4;
    // both row pointers read as scalars first (a lane-dependent choice between
    // two kernel arguments is otherwise read with a vector load, one more round trip)
    const float* cp = p.cosv;
    const float* sp = p.sinv;
    asm volatile("" : "+s"(cp), "+s"(sp));
    r.c = ld16f(r.trig ? (tid < 64 ? cp : sp) + co : reinterpret_cast<const float*>(g_zero_row));
    return r;
}

template <int DT>
__device__ inline void store_query(const QStage& r, float (*qs)[kHeadDim], float* cs, float* sn, float* spare) {
    const int tid = threadIdx.x;
    const int hh = tid >> 4, dd = (tid & 15) * 8;
    if constexpr (DT == kF32) {
        *reinterpret_cast<f32x4*>(&qs[hh][dd]) = r.a;
        *reinterpret_cast<f32x4*>(&qs[hh][dd + 4]) = r.b;
    } else {
        // stored as loaded: a conversion here is scheduled between the K/V
        // loads, whose last ones then wait for the query
        *reinterpret_cast<u32x4*>(reinterpret_cast<uint16_t*>(qs) + hh * kHeadDim + dd) = r.u;
    }
    // unconditional store (threads without a cos/sin part write the spare
    // slot): a conditional one lets the compiler sink the load into the branch
    float* dst = r.trig ? (tid < 64 ? cs : sn) + (tid & 63) * 4 : spare;
    *reinterpret_cast<f32x4*>(dst) = r.c;
}

// Dims d .. d+3 of staged query row n, as fp32.
template <int DT>
__device__ inline f32x4 staged_run(const float (*qs)[kHeadDim], int n, int d) {
    if constexpr (DT == kF32)
        return *reinterpret_cast<const f32x4*>(&qs[n][d]);
    else
        return widen4<DT>(*reinterpret_cast<const u32x2*>(reinterpret_cast<const uint16_t*>(qs) + n * kHeadDim + d));
}

// Query operand from the staged rows: lane (g, n) holds Q[n][c*16 + g*4 + 0..3],
// c = 0..7 (the B operand of S^T).  Rotating mode applies the reference's rope
// (src/rope.cuh:18-51) with the same roundings as rotate_run: separate fp32
// products, then their difference or sum, rounded to the storage type; dims
// >= R are copied.  Needs rotary_dim % 8 == 0, so a run of 4 dims never
// straddles the two halves.
template <int DT, int QM>
__device__ inline void query_operand(const DecodeParams& p, const float (*qs)[kHeadDim], const float* cs,
                                     const float* sn, f32x4 (&qB)[8]) {
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63;
    const int g = lane >> 4, n = lane & 15;
    const int half = p.R >> 1;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
        const int d = c * 16 + g * 4;
        const f32x4 x = staged_run<DT>(qs, n, d);
        if constexpr (QM == kQPre) {
            qB[c] = x;
        } else {
            const bool rot = d < p.R;
            const bool first = d < half;
            const int pd = rot ? (first ? d + half : d - half) : d;
            const int ci = rot ? (first ? d : pd) : 0;
            const f32x4 xp = staged_run<DT>(qs, n, pd);
            const f32x4 cv = *reinterpret_cast<const f32x4*>(cs + ci);
            const f32x4 sv = *reinterpret_cast<const f32x4*>(sn + ci);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float a = x[e] * cv[e];
                const float b = xp[e] * sv[e];
                const float y = first ? a - b : a + b;
                qB[c][e] = rot ? Tr<DT>::tof(Tr<DT>::fromf(y)) : x[e];
            }
        }
    }
}

template <int DT>
__device__ inline void store8(void* dst, const float (&o)[8], float inv) {
    if constexpr (DT == kF32) {
        float* d = reinterpret_cast<float*>(dst);
        *reinterpret_cast<f32x4*>(d) = f32x4{o[0] * inv, o[1] * inv, o[2] * inv, o[3] * inv};
        *reinterpret_cast<f32x4*>(d + 4) = f32x4{o[4] * inv, o[5] * inv, o[6] * inv, o[7] * inv};
    } else {
        *reinterpret_cast<u32x4*>(dst) = u32x4{pack2<DT>(o[0] * inv, o[1] * inv), pack2<DT>(o[2] * inv, o[3] * inv),
                                               pack2<DT>(o[4] * inv, o[5] * inv), pack2<DT>(o[6] * inv, o[7] * inv)};
    }
}

template <int DT, int QM>
__global__ __launch_bounds__(256) void dv_small(const SmallParams sp) {
    using raw = typename Tr<DT>::raw;
    __shared__ __align__(16) Smem sm;
    const DecodeParams& p = sp.d;
    const int item = blockIdx.x / sp.chunks;  // (query row, KV head)
    const int ci = blockIdx.x - item * sp.chunks;
    const int row = item / p.Hkv;
    const int hkv = item - row * p.Hkv;
    const int w = row / p.S;
    const int s = row - w * p.S;
    int f = 0;
    while (f + 1 < p.F && sp.first_chunk[f + 1] <= ci) ++f;
    const FragDesc& fd = p.frags[f];
    const int tid = threadIdx.x;
    const int wv = tid >> 6, lane = tid & 63, g = lane >> 4, n = lane & 15;
    const int k0 = (ci - sp.first_chunk[f]) * kSmallChunk + wv * kKeysPerWave;  // wave's first tensor key
    const raw* kbase = reinterpret_cast<const raw*>(fd.k) + fd.bstride * w + (long long)hkv * fd.L * kHeadDim;
    const raw* vbase = reinterpret_cast<const raw*>(fd.v) + fd.bstride * w + (long long)hkv * fd.L * kHeadDim;
    const raw* zrow = reinterpret_cast<const raw*>(g_zero_row);
    const int vis = view_vis<kKvContig>(p, f, row_loc<kRowWS>(p, row, f));

    // ---- loads, all issued together: the query rows and cos/sin (staged in
    // LDS), K (key k0 + n, dims c*16 + g*4 + 0..3) and V (key k0 + g*4 + i,
    // dims 64 b + 4 n + 0..3) to registers; keys past the tensor read the zero row
    const QStage qst = load_query<DT, QM>(p, w, s, f, hkv);
    Run4<DT> kr[8], vr[4][2];
    {
        const int key = k0 + n;
        const raw* kp = key < fd.L ? kbase + (long long)key * kHeadDim : zrow;
#pragma unroll
        for (int c = 0; c < 8; ++c) kr[c] = ld4_nt<DT>(kp, c * 16 + g * 4);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int key = k0 + g * 4 + i;
        const raw* vp = key < fd.L ? vbase + (long long)key * kHeadDim : zrow;
        vr[i][0] = ld4_nt<DT>(vp, n * 4);
        vr[i][1] = ld4_nt<DT>(vp, 64 + n * 4);
    }
    // nothing that uses a loaded value is scheduled above the last load
    __builtin_amdgcn_sched_barrier(0);
    store_query<DT>(qst, sm.q, sm.cs, sm.sn, sm.spare);
    __syncthreads();
    f32x4 qB[8];
    query_operand<DT, QM>(p, sm.q, sm.cs, sm.sn, qB);
    if (QM == kQRotFull && wv == 0 && ci == sp.first_chunk[f]) {
        // the view's rotated query, as dvattn_rope writes it
        raw* rq = reinterpret_cast<raw*>(sp.rq) +
                  ((((long long)f * p.W + w) * p.Hq + hkv * kGqa + n) * p.S + s) * kHeadDim + g * 4;
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            if constexpr (DT == kF32)
                *reinterpret_cast<f32x4*>(rq + c * 16) = qB[c];
            else  // exact: the values are rounded to the storage type already
                *reinterpret_cast<u32x2*>(rq + c * 16) =
                    u32x2{pack2<DT>(qB[c][0], qB[c][1]), pack2<DT>(qB[c][2], qB[c][3])};
        }
    }

    // ---- S^T: lane (g, n) holds keys k0 + g*4 + i of head n
    f32x4 sc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < 8; ++c) {
        const f32x4 kc = run_f32<DT>(kr[c]);
#pragma unroll
        for (int j = 0; j < 4; ++j) sc = Tr<kF32>::mma1(kc[j], qB[c][j], sc);
    }
    float pr[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) pr[i] = k0 + g * 4 + i < vis ? sc[i] * p.l2scale : -DV_INF;
    const float mx = rows4_max(fmaxf(fmaxf(pr[0], pr[1]), fmaxf(pr[2], pr[3])));
    const float mm = mx == -DV_INF ? 0.0f : mx;  // p = 0 for a head with no visible key here
#pragma unroll
    for (int i = 0; i < 4; ++i) pr[i] = __builtin_amdgcn_exp2f(pr[i] - mm);
    const float l = rows4_sum((pr[0] + pr[1]) + (pr[2] + pr[3]));

    // ---- O = P V: A = P (head n, key g*4 + i), B = V (key g*4 + i, dim 64 b + 4 n + t);
    // lane (g, n) receives O[head g*4 + j][dim 64 b + 4 n + t]
    f32x4 acc[2][4];
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int t = 0; t < 4; ++t) acc[b][t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            const f32x4 vv = run_f32<DT>(vr[i][b]);
#pragma unroll
            for (int t = 0; t < 4; ++t) acc[b][t] = Tr<kF32>::mma1(pr[i], vv[t], acc[b][t]);
        }
    mfma_settle(reinterpret_cast<f32x4(&)[8]>(acc));
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int j = 0; j < 4; ++j)
            *reinterpret_cast<f32x4*>(&sm.o[wv][g * 4 + j][b * 64 + n * 4]) =
                f32x4{acc[b][0][j], acc[b][1][j], acc[b][2][j], acc[b][3][j]};
    if (g == 0) {
        sm.m[wv][n] = mx;
        sm.l[wv][n] = l;
    }
    __syncthreads();

    // ---- the chunk: thread (h, d0) combines the four waves for head h, dims d0..d0+7
    const int h = tid >> 4;
    const int d0 = (tid & 15) * 8;
    float M = -DV_INF;
#pragma unroll
    for (int k = 0; k < kWaves; ++k) M = fmaxf(M, sm.m[k][h]);
    float L = 0.0f, o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = 0.0f;
    if (M != -DV_INF) {
#pragma unroll
        for (int k = 0; k < kWaves; ++k) {
            const float e = __builtin_amdgcn_exp2f(sm.m[k][h] - M);  // wave without visible keys: 0
            L += e * sm.l[k][h];
            const f32x4 a = *reinterpret_cast<const f32x4*>(&sm.o[k][h][d0]);
            const f32x4 c = *reinterpret_cast<const f32x4*>(&sm.o[k][h][d0 + 4]);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                o[q] += e * a[q];
                o[4 + q] += e * c[q];
            }
        }
    }
    const float inv = L > 0.0f ? 1.0f / L : 0.0f;
    raw* outp = reinterpret_cast<raw*>(p.out) + (((long long)w * p.Hq + hkv * kGqa + h) * p.S + s) * kHeadDim + d0;
    if (sp.chunks == 1) {
        store8<DT>(outp, o, inv);
        return;
    }
    float* slot = sp.part + ((long long)item * sp.chunks + ci) * kSlot;
    store8<kF32>(slot + h * kHeadDim + d0, o, inv);
    if ((tid & 15) == 0) slot[kGqa * kHeadDim + h] = L > 0.0f ? M + log2f(L) : -DV_INF;
    // every thread's partial stores complete before the barrier; the agent-scope
    // release of wave 0 then writes the workgroup's partial back from this XCD's
    // L2, and the flag is raised after it.  The sequentially consistent fence
    // between raising the own flag and reading all flags (all in wave 0's
    // program order) makes the workgroup whose fence comes last see every flag
    // raised, so at least one workgroup merges; several may, writing the same
    // output.
    unsigned long long* flags = sp.flags + (long long)item * sp.chunks;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __syncthreads();
    if (wv == 0) {
        if (lane == 0) {
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
            __hip_atomic_store(flags + ci, sp.tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "agent");
        const unsigned long long v =
            lane < sp.chunks ? __hip_atomic_load(flags + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : sp.tag;
        const bool all = ballot(v != sp.tag) == 0;
        if (lane == 0) sm.last = all;
    }
    __syncthreads();
    if (!sm.last) return;
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    // lower the flags (all were raised: no workgroup of this call raises one later)
    if (tid < sp.chunks) __hip_atomic_store(flags + tid, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

    // ---- last arrival: merge the item's chunks (head h, dims d0..d0+7)
    const float* pbase = sp.part + (long long)item * sp.chunks * kSlot;
    float m = -DV_INF, wsum = 0.0f, acc8[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) acc8[e] = 0.0f;
    for (int c0 = 0; c0 < sp.chunks; c0 += kMergeBatch) {
        float lse[kMergeBatch];
        f32x4 v0[kMergeBatch], v1[kMergeBatch];
#pragma unroll
        for (int i = 0; i < kMergeBatch; ++i) {
            const bool in = c0 + i < sp.chunks;
            const float* sl = pbase + (long long)(in ? c0 + i : c0) * kSlot;
            lse[i] = in ? sl[kGqa * kHeadDim + h] : -DV_INF;
            v0[i] = ld16f(sl + h * kHeadDim + d0);
            v1[i] = ld16f(sl + h * kHeadDim + d0 + 4);
        }
        float bm = m;
#pragma unroll
        for (int i = 0; i < kMergeBatch; ++i) bm = fmaxf(bm, lse[i]);
        if (bm == -DV_INF) continue;
        const float scl = __builtin_amdgcn_exp2f(m - bm);  // m == -inf -> 0
        wsum *= scl;
#pragma unroll
        for (int e = 0; e < 8; ++e) acc8[e] *= scl;
#pragma unroll
        for (int i = 0; i < kMergeBatch; ++i) {
            const float wgt = __builtin_amdgcn_exp2f(lse[i] - bm);  // empty chunk (-inf) -> 0
            wsum += wgt;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                acc8[q] += wgt * v0[i][q];
                acc8[4 + q] += wgt * v1[i][q];
            }
        }
        m = bm;
    }
    store8<DT>(outp, acc8, wsum > 0.0f ? 1.0f / wsum : 0.0f);
}

size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

}  // namespace small

int small_chunks(int F, const int* toks) {
    if (F < 1 || F > kMaxFragArgs) return -1;
    long long c = 0;
    for (int f = 0; f < F; ++f) c += toks[f] > 0 ? (toks[f] + kSmallChunk - 1) / kSmallChunk : 1;
    return c <= kSmallMaxChunks ? (int)c : -1;
}

size_t small_workspace_bytes(long long items, int chunks) {
    if (items <= 0 || chunks <= 1) return 0;
    return small::align256((size_t)items * chunks * sizeof(unsigned long long)) +
           (size_t)items * chunks * small::kSlot * sizeof(float);
}

template <int DT>
void launch_small_dt(int qmode, const SmallParams& p, long long grid, hipStream_t stream) {
    if (qmode == kQRotFull)
        hipLaunchKernelGGL((small::dv_small<DT, kQRotFull>), dim3((unsigned)grid), dim3(256), 0, stream, p);
    else
        hipLaunchKernelGGL((small::dv_small<DT, kQPre>), dim3((unsigned)grid), dim3(256), 0, stream, p);
}

hipError_t launch_small(int dtype, int qmode, SmallParams& p, void* workspace, hipStream_t stream) {
    if ((dtype != kF32 && dtype != kF16 && dtype != kBF16) || (qmode != kQPre && qmode != kQRotFull))
        return hipErrorInvalidValue;
    const long long items = (long long)p.d.W * p.d.S * p.d.Hkv;
    if (items <= 0) return hipSuccess;
    const long long grid = items * p.chunks;
    if (p.chunks < 1 || p.chunks > kSmallMaxChunks || grid > 0x7fffffffll) return hipErrorInvalidValue;
    p.flags = reinterpret_cast<unsigned long long*>(workspace);
    p.part = reinterpret_cast<float*>(reinterpret_cast<unsigned char*>(workspace) +
                                      small::align256((size_t)items * p.chunks * sizeof(unsigned long long)));
    p.tag = next_call_tag();
    if (dtype == kF32) launch_small_dt<kF32>(qmode, p, grid, stream);
    else if (dtype == kF16) launch_small_dt<kF16>(qmode, p, grid, stream);
    else launch_small_dt<kBF16>(qmode, p, grid, stream);
    return hipGetLastError();
}

}  // namespace dv
