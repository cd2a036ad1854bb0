// One decode step of the selective scan (L = 1 with a carried state), for inference.
//
// Semantics: the reference's forward_with_state (mamba_cuda.py:271-359) at seqlen 1, i.e.
//   h' = exp(clamp(delta*A, -88, 88)) * h + delta*u*B;  y = sum_n C*h' + D*u
// with the optional transforms of the fused scan (delta' = softplus(delta + delta_bias),
// y_z = y * silu(z)). The state is read and written in the input dtype, (batch, dim, N), and the
// output state may alias the input one (in-place update).
//
// Mapping: a lane holds 16 bytes of a channel's states (4 fp32 or 8 fp16/bf16 states), so the state,
// A, B and C move as coalesced rows of 16-byte accesses, and the C-contraction is an in-lane FMA
// chain plus a DPP sum over the channel's N*s/16 lanes. The step is bound by the state's round trip
// through HBM (2 * batch * dim * N * s bytes) and, at small batch, by launch latency.
#include "common.h"
#include "launch.h"

namespace mwc {

// states per lane: one 16-byte vector of the storage type (all N states when they are fewer)
template <typename T, int NS> constexpr int step_spl() {
    return (int)(16 / sizeof(T)) < NS ? (int)(16 / sizeof(T)) : NS;
}

template <typename T, int NS>
__global__ void __launch_bounds__(256) ssm_step_kernel(const T* __restrict__ u, const T* __restrict__ delta,
                                                       const T* __restrict__ A, const T* __restrict__ Bm,
                                                       const T* __restrict__ Cm, const T* __restrict__ Dv,
                                                       const T* h_in, ScanXf xf, T* __restrict__ y,
                                                       T* __restrict__ y_z, T* h_out, int64_t channels, int D) {
    constexpr int kStepSpl = step_spl<T, NS>();
    constexpr int kStepLpc = NS / kStepSpl;
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;  // over batch * dim * kStepLpc
    const int n0 = (int)(i % kStepLpc) * kStepSpl;
    const int64_t bd = i / kStepLpc;  // b * D + d
    const bool valid = bd < channels;
    const int64_t bdc = valid ? bd : channels - 1;  // keep the group's lanes in bounds
    const int64_t b = bdc / D;
    const int d = (int)(bdc - b * D);
    float dt = ld(delta + bdc);
    if (xf.delta_bias != nullptr) dt += ld(static_cast<const T*>(xf.delta_bias) + d);
    if (xf.softplus) dt = softplus_f(dt);
    const float uu = ld(u + bdc);
    const float dtu = dt * uu;
    // kStepSpl consecutive states per lane: one 16-byte access per tensor
    typedef T vec4 __attribute__((ext_vector_type(kStepSpl)));
    const vec4 a4 = *reinterpret_cast<const vec4*>(A + (int64_t)d * NS + n0);
    const vec4 h4 = *reinterpret_cast<const vec4*>(h_in + bdc * NS + n0);
    const vec4 b4 = *reinterpret_cast<const vec4*>(Bm + b * NS + n0);
    const vec4 c4 = *reinterpret_cast<const vec4*>(Cm + b * NS + n0);
    vec4 o4;
    float yp = 0.f;
#pragma unroll
    for (int j = 0; j < kStepSpl; ++j) {
        const float x = dt * static_cast<float>(a4[j]) * kLog2e;
        const float h = __builtin_fmaf(exp2_clamped(x), static_cast<float>(h4[j]), dtu * static_cast<float>(b4[j]));
        yp = __builtin_fmaf(static_cast<float>(c4[j]), h, yp);
        o4[j] = static_cast<T>(h);
    }
    const float yv = __builtin_fmaf(ld(Dv + d), uu, group_sum<kStepLpc>(yp));
    if (valid) {
        *reinterpret_cast<vec4*>(h_out + bdc * NS + n0) = o4;  // each lane rewrites only what it read
        if (n0 == 0) {
            if (y != nullptr) st(y + bdc, yv);
            if (xf.z != nullptr) {
                const float zv = ld(static_cast<const T*>(xf.z) + bdc);
                st(y_z + bdc, yv * zv * sigmoid_f(zv));
            }
        }
    }
}

hipError_t launch_ssm_step(int dt, int ns, const void* u, const void* delta, const void* A, const void* B,
                           const void* C, const void* Dv, const void* h_in, const ScanXf& xf, void* y, void* y_z,
                           void* h_out, int64_t batch, int64_t dim, hipStream_t st) {
    const int64_t channels = batch * dim;
#define MWC_STEP(N)                                                                                            \
    if (ns == N) {                                                                                             \
        MWC_DISPATCH_DTYPE(dt, TT,                                                                             \
                           const int64_t lanes = channels * (N / step_spl<TT, N>());                          \
                           const int grid = (int)((lanes + 255) / 256);                                        \
                           hipLaunchKernelGGL((ssm_step_kernel<TT, N>), dim3(grid), dim3(256), 0, st,          \
                                              (const TT*)u, (const TT*)delta, (const TT*)A, (const TT*)B,      \
                                              (const TT*)C, (const TT*)Dv, (const TT*)h_in, xf, (TT*)y,        \
                                              (TT*)y_z, (TT*)h_out, channels, (int)dim));                      \
        return hipGetLastError();                                                                              \
    }
    MWC_STEP(8)
    MWC_STEP(16)
    MWC_STEP(32)
    MWC_STEP(64)
#undef MWC_STEP
    return hipErrorInvalidValue;
}

}  // namespace mwc
