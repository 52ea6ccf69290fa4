// Standalone query rotation (ops dvattn_rope / dvattn_varlen_rope and the first
// half of dvattn_fused).  Restates src/rope.cuh:2-114 (reference repository):
// one thread per run of 8 (16-bit types) or 4 (fp32) consecutive head dims,
// 16-byte loads/stores, fp32 math without FMA contraction, rounded to the
// storage type -- bit-identical to a separately-rounded fp32 evaluation.
#include "dv_common.h"
#include "dv_device.h"

namespace dv {

template <int DT, int RUN>
__global__ __launch_bounds__(256) void dv_rope_kernel(const RopeParams p, long long nruns) {
    using raw = typename Tr<DT>::raw;
    const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= nruns) return;
    const int runs_per_row = p.E / RUN;
    const long long vr = idx / runs_per_row;  // output vector row
    const int d0 = (int)(idx - vr * runs_per_row) * RUN;
    const raw* qrow;
    const float* crow;
    const float* srow;
    if (!p.half_width) {
        // out [F,W,Hq,S,E]: vr = ((f*W + w)*Hq + h)*S + s
        const long long s = vr % p.S;
        const long long t1 = vr / p.S;
        const long long h = t1 % p.Hq;
        const long long t2 = t1 / p.Hq;
        const long long w = t2 % p.W;
        const long long f = t2 / p.W;
        qrow = reinterpret_cast<const raw*>(p.q) + ((w * p.Hq + h) * p.S + s) * p.E;
        const long long co = ((f * p.W + w) * p.S + s) * p.R;
        crow = p.cosv + co;
        srow = p.sinv + co;
    } else {
        // out [F,T,H,E]: vr = (f*T + t)*H + h
        const long long h = vr % p.Hq;
        const long long t1 = vr / p.Hq;
        const long long t = t1 % p.T;
        const long long f = t1 / p.T;
        qrow = reinterpret_cast<const raw*>(p.q) + (t * p.Hq + h) * p.E;
        const long long co = (f * p.T + t) * (p.R >> 1);
        crow = p.cosv + co;
        srow = p.sinv + co;
    }
    raw r[RUN];
    rotate_run<DT, RUN>(qrow, crow, srow, p.R, d0, r);
    raw* o = reinterpret_cast<raw*>(p.out) + vr * p.E + d0;
#pragma unroll
    for (int e = 0; e < RUN; ++e) o[e] = r[e];
}

template <int DT, int RUN>
hipError_t rope_go(const RopeParams& p, long long rows, hipStream_t stream) {
    const long long nruns = rows * (p.E / RUN);
    if (nruns == 0) return hipSuccess;
    const long long blocks = (nruns + 255) / 256;
    hipLaunchKernelGGL((dv_rope_kernel<DT, RUN>), dim3((unsigned)blocks), dim3(256), 0, stream, p, nruns);
    return hipGetLastError();
}

template <int DT>
hipError_t rope_dispatch(const RopeParams& p, hipStream_t stream) {
    const long long rows = p.half_width ? (long long)p.F * p.T * p.Hq : (long long)p.F * p.W * p.Hq * p.S;
    constexpr int kRun = DT == kF32 ? 4 : 8;
    if (p.E % kRun == 0) return rope_go<DT, kRun>(p, rows, stream);
    return rope_go<DT, 1>(p, rows, stream);
}

hipError_t launch_rope(int dtype, const RopeParams& p, hipStream_t stream) {
    switch (dtype) {
        case kBF16: return rope_dispatch<kBF16>(p, stream);
        case kF16: return rope_dispatch<kF16>(p, stream);
        case kF32: return rope_dispatch<kF32>(p, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace dv
