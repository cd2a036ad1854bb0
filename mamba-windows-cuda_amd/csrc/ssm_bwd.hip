// Fused selective-scan backward for gfx950.
//
// Semantics: the adjoint of the forward (the gradients torch autograd takes
// through selective_scan_ref, mamba_cuda.py:875-946), i.e. the reference's
// backward kernels (mamba_cuda.py:366-562 and 669-745) plus h_prev/dh_last/
// dh_prev, which those kernels do not handle (they start from h=0):
//   g_t    = dout_t*C_t + dA_{t+1}*g_{t+1}       (g_{L-1} also receives dh_last)
//   du     = D*dout + delta*sum_n g*B
//   ddelta = sum_n g*(A*dA_t*h_{t-1}) + u*sum_n g*B
//   dA     = sum_{b,t} delta*g*dA_t*h_{t-1}      dD = sum_{b,t} dout*u
//   dB     = sum_d g*delta*u                      dC = sum_d dout*h_t
//   dh_prev = dA_0*g_0
//
// Mapping: the forward's lane groups (LPC lanes x SPL states per channel).
// The sequence is walked in reverse in chunks of kCkptSteps steps; each chunk
// restarts from the fp32 checkpoint the forward stored, recomputes the chunk's
// states and decay factors into VGPRs (one exp per state), then runs the
// reverse sweep. Sums over n (du, ddelta) are DPP reductions inside the lane
// group. Sums over channels (dB, dC) go through LDS: every 4 steps each wave
// folds its channels in its own LDS slab (no barrier -- LDS operations of one
// wave complete in order), and once per chunk the workgroup's waves are
// summed and written as a per-group fp32 partial; a second small kernel adds
// the groups in fixed order, so the result is deterministic (no atomics).
// dA and dD accumulate in registers over (t) and are summed over b by the
// finishing kernel.
#include "common.h"
#include "launch.h"

namespace mwc {

namespace {

constexpr int kWpb = 4;       // waves per workgroup in the backward
constexpr int kRedSlots = 4;  // steps folded per in-wave LDS reduction
constexpr int kRowPad = 36;   // floats per channel row in the LDS slab (32 values + pad)

template <int K>
__device__ __forceinline__ void ldv(const float* __restrict__ p, float (&v)[K]) {
    if constexpr (K % 4 == 0) {
#pragma unroll
        for (int k = 0; k < K; k += 4) {
            const float4 q = *reinterpret_cast<const float4*>(p + k);
            v[k] = q.x;
            v[k + 1] = q.y;
            v[k + 2] = q.z;
            v[k + 3] = q.w;
        }
    } else if constexpr (K == 2) {
        const float2 q = *reinterpret_cast<const float2*>(p);
        v[0] = q.x;
        v[1] = q.y;
    } else {
        v[0] = *p;
    }
}

template <int K>
__device__ __forceinline__ void stv(float* p, const float (&v)[K]) {
    if constexpr (K % 4 == 0) {
#pragma unroll
        for (int k = 0; k < K; k += 4) *reinterpret_cast<float4*>(p + k) = make_float4(v[k], v[k + 1], v[k + 2], v[k + 3]);
    } else if constexpr (K == 2) {
        *reinterpret_cast<float2*>(p) = make_float2(v[0], v[1]);
    } else {
        *p = v[0];
    }
}

}  // namespace

template <typename T, int SPL>
__global__ void __launch_bounds__(64 * kWpb) ssm_bwd_kernel(
    const T* __restrict__ u, const T* __restrict__ delta, const T* __restrict__ A, const float* __restrict__ bc,
    const T* __restrict__ Dv, const T* __restrict__ dout, const T* __restrict__ dh_last,
    const float* __restrict__ ckpt, T* __restrict__ du, T* __restrict__ ddelta, T* __restrict__ dh_prev,
    float* __restrict__ dA_part, float* __restrict__ dD_part, float* __restrict__ dbc_part, int Bsz, int L, int D,
    int nck, int ngrp) {
    constexpr int LPC = kNState / SPL;
    constexpr int CPW = 64 / LPC;
    constexpr int TC = kCkptSteps;
    constexpr int HALF = CPW / 2;  // channels each reducing lane folds
    static_assert(CPW >= 2, "reduction needs two channel halves");

    __shared__ float red[kWpb][kRedSlots][CPW][kRowPad];
    __shared__ float wsum[2][kWpb][TC][32];

    const int lid = xcd_remap(blockIdx.x, gridDim.x);
    const int b = lid / ngrp;
    const int grp = lid % ngrp;
    const int wave = threadIdx.x / 64;
    const int lane = threadIdx.x % 64;
    const int c = lane / LPC, g = lane % LPC;
    const int d_raw = (grp * kWpb + wave) * CPW + c;
    const bool valid = d_raw < D;
    const int d = valid ? d_raw : D - 1;
    const int n0 = g * SPL;
    const float vmask = valid ? 1.f : 0.f;  // padded lanes contribute nothing to dB/dC

    float A2[SPL], An[SPL], gc[SPL], dAacc[SPL];
#pragma unroll
    for (int j = 0; j < SPL; ++j) {
        An[j] = ld(A + (int64_t)d * kNState + n0 + j);
        A2[j] = An[j] * kLog2e;
        gc[j] = (dh_last != nullptr && valid) ? ld(dh_last + ((int64_t)b * D + d) * kNState + n0 + j) : 0.f;
        dAacc[j] = 0.f;
    }
    float dDacc = 0.f;
    const float Dd = ld(Dv + d);
    const int64_t base = (int64_t)b * L * D + d;
    const float* __restrict__ bcb = bc + (int64_t)b * L * 32 + n0;
    const float* __restrict__ ckb = ckpt + ((int64_t)b * nck * D + d) * kNState + n0;

    // reduction lane roles: pair p = lane/2 -> (slot, value quad), half = lane&1
    const int rp = lane >> 1, rhalf = lane & 1;
    const int rslot = rp >> 3, rq = rp & 7;
    float(*myred)[CPW][kRowPad] = red[wave];

    for (int k = nck - 1; k >= 0; --k) {
        const int t0 = k * TC;
        const int tn = min(TC, L - t0);
        float hin[SPL];
        ldv<SPL>(ckb + (int64_t)k * D * kNState, hin);

        float H[TC][SPL], E[TC][SPL], DT[TC], UT[TC], YO[TC];
        // ---- recompute the chunk's states (one exp per state) ----
        {
            float hh[SPL];
#pragma unroll
            for (int j = 0; j < SPL; ++j) hh[j] = hin[j];
#pragma unroll
            for (int i = 0; i < TC; ++i) {
                if (i < tn) {
                    const int64_t t = t0 + i;
                    DT[i] = ld(delta + base + t * D);
                    UT[i] = ld(u + base + t * D);
                    YO[i] = ld(dout + base + t * D) * vmask;
                    float Bv[SPL];
                    ldv<SPL>(bcb + t * 32, Bv);
                    const float dtu = DT[i] * UT[i];
#pragma unroll
                    for (int j = 0; j < SPL; ++j) {
                        E[i][j] = exp2_clamped(DT[i] * A2[j]);
                        hh[j] = __builtin_fmaf(E[i][j], hh[j], dtu * Bv[j]);
                        H[i][j] = hh[j];
                    }
                }
            }
        }
        // ---- reverse sweep ----
#pragma unroll
        for (int i = TC - 1; i >= 0; --i) {
            const int slot = i % kRedSlots;
            float dBv[SPL], dCv[SPL];
            if (i < tn) {
                const int64_t t = t0 + i;
                float Bv[SPL], Cv[SPL];
                ldv<SPL>(bcb + t * 32, Bv);
                ldv<SPL>(bcb + t * 32 + kNState, Cv);
                const float yo = YO[i];
                const float dtu = DT[i] * UT[i] * vmask;
                float r1 = 0.f, r2 = 0.f;
#pragma unroll
                for (int j = 0; j < SPL; ++j) {
                    const float prev = (i > 0) ? H[i > 0 ? i - 1 : 0][j] : hin[j];
                    const float gt = __builtin_fmaf(yo, Cv[j], gc[j]);
                    dCv[j] = yo * H[i][j];
                    dBv[j] = gt * dtu;
                    r1 = __builtin_fmaf(gt, Bv[j], r1);
                    const float s = gt * E[i][j] * prev;
                    r2 = __builtin_fmaf(An[j], s, r2);
                    dAacc[j] = __builtin_fmaf(DT[i], s, dAacc[j]);
                    gc[j] = E[i][j] * gt;
                }
                r1 = group_sum<LPC>(r1);
                r2 = group_sum<LPC>(r2);
                if (g == 0 && valid) {
                    st(du + base + t * D, __builtin_fmaf(Dd, yo, DT[i] * r1));
                    st(ddelta + base + t * D, __builtin_fmaf(UT[i], r1, r2));
                }
                dDacc = __builtin_fmaf(yo, UT[i], dDacc);
            } else {
#pragma unroll
                for (int j = 0; j < SPL; ++j) dBv[j] = dCv[j] = 0.f;
            }
            stv<SPL>(&myred[slot][c][n0], dBv);
            stv<SPL>(&myred[slot][c][kNState + n0], dCv);
            if (slot == 0) {
                // fold this wave's channels for steps i..i+3 (values 4*rq..4*rq+3 of slot rslot)
                float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int m = 0; m < HALF; ++m) {
                    float v4[4];
                    ldv<4>(&myred[rslot][rhalf * HALF + m][rq * 4], v4);
#pragma unroll
                    for (int q = 0; q < 4; ++q) acc[q] += v4[q];
                }
#pragma unroll
                for (int q = 0; q < 4; ++q) acc[q] += dpp<kDppXor1>(acc[q]);
                if (rhalf == 0) stv<4>(&wsum[k & 1][wave][i + rslot][rq * 4], acc);
            }
        }
        __syncthreads();
        // sum the workgroup's waves and emit this group's partial for the chunk
        for (int o = threadIdx.x; o < TC * 32; o += 64 * kWpb) {
            const int tt = o / 32;
            float s = 0.f;
#pragma unroll
            for (int w = 0; w < kWpb; ++w) s += wsum[k & 1][w][tt][o % 32];
            if (tt < tn) dbc_part[(((int64_t)grp * Bsz + b) * L + t0 + tt) * 32 + (o % 32)] = s;
        }
    }

    if (valid) {
        if (dh_prev != nullptr) {
#pragma unroll
            for (int j = 0; j < SPL; ++j) st(dh_prev + ((int64_t)b * D + d) * kNState + n0 + j, gc[j]);
        }
        stv<SPL>(dA_part + ((int64_t)b * D + d) * kNState + n0, dAacc);
        if (g == 0) dD_part[(int64_t)b * D + d] = dDacc;
    }
}

// dB/dC: sum the channel-group partials in group order and cast.
template <typename T>
__global__ void __launch_bounds__(256) bwd_finish_bc_kernel(const float* __restrict__ part, T* __restrict__ dB,
                                                            T* __restrict__ dC, int ngrp, int64_t rows) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;  // over rows*32
    if (i >= rows * 32) return;
    float s = 0.f;
    for (int q = 0; q < ngrp; ++q) s += part[(int64_t)q * rows * 32 + i];
    const int64_t r = i >> 5;
    const int v = (int)(i & 31);
    if (v < kNState)
        st(dB + r * kNState + v, s);
    else
        st(dC + r * kNState + v - kNState, s);
}

// dA (D,N) and dD (D,): sum the per-batch partials in batch order and cast.
template <typename T>
__global__ void __launch_bounds__(256) bwd_finish_ad_kernel(const float* __restrict__ dA_part,
                                                            const float* __restrict__ dD_part, T* __restrict__ dA,
                                                            T* __restrict__ dD, int Bsz, int D) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t nA = (int64_t)D * kNState;
    if (i < nA) {
        float s = 0.f;
        for (int b = 0; b < Bsz; ++b) s += dA_part[(int64_t)b * nA + i];
        st(dA + i, s);
    } else if (i < nA + D) {
        const int64_t dd = i - nA;
        float s = 0.f;
        for (int b = 0; b < Bsz; ++b) s += dD_part[(int64_t)b * D + dd];
        st(dD + dd, s);
    }
}

int bwd_groups(const SsmShape& s, int spl) {
    const int cpw = 64 / (kNState / spl);
    const int per_wg = cpw * kWpb;
    return (int)((s.dim + per_wg - 1) / per_wg);
}

template <typename T, int SPL>
static hipError_t bwd_inst(const void* u, const void* delta, const void* A, const float* bc, const void* Dv,
                           const void* dout, const void* dh_last, const float* ckpt, void* du, void* ddelta,
                           void* dh_prev, float* dA_part, float* dD_part, float* dbc_part, const SsmShape& s,
                           hipStream_t st) {
    const int ngrp = bwd_groups(s, SPL);
    const int nck = (int)((s.seqlen + kCkptSteps - 1) / kCkptSteps);
    const int grid = ngrp * (int)s.batch;
    hipLaunchKernelGGL((ssm_bwd_kernel<T, SPL>), dim3(grid), dim3(64 * kWpb), 0, st, (const T*)u, (const T*)delta,
                       (const T*)A, bc, (const T*)Dv, (const T*)dout, (const T*)dh_last, ckpt, (T*)du, (T*)ddelta,
                       (T*)dh_prev, dA_part, dD_part, dbc_part, (int)s.batch, (int)s.seqlen, (int)s.dim, nck, ngrp);
    return hipGetLastError();
}

hipError_t launch_ssm_bwd(bool is_half, int spl, const void* u, const void* delta, const void* A, const float* bc,
                          const void* Dv, const void* dout, const void* dh_last, const float* ckpt, void* du,
                          void* ddelta, void* dh_prev, float* dA_part, float* dD_part, float* dbc_part,
                          const SsmShape& s, hipStream_t st) {
#define MWC_BWD_SPL(S)                                                                                        \
    if (spl == S)                                                                                             \
        return is_half ? bwd_inst<half_t, S>(u, delta, A, bc, Dv, dout, dh_last, ckpt, du, ddelta, dh_prev,  \
                                             dA_part, dD_part, dbc_part, s, st)                               \
                       : bwd_inst<float, S>(u, delta, A, bc, Dv, dout, dh_last, ckpt, du, ddelta, dh_prev,   \
                                            dA_part, dD_part, dbc_part, s, st);
    MWC_BWD_SPL(1)
    MWC_BWD_SPL(2)
    MWC_BWD_SPL(4)
#undef MWC_BWD_SPL
    return hipErrorInvalidValue;
}

template <typename T>
static hipError_t finish_t(const float* dbc_part, const float* dA_part, const float* dD_part, void* dB, void* dC,
                           void* dA, void* dD, int ngrp, const SsmShape& s, hipStream_t st) {
    const int64_t rows = s.batch * s.seqlen;
    const int g1 = (int)((rows * 32 + 255) / 256);
    if (g1 > 0)
        hipLaunchKernelGGL(bwd_finish_bc_kernel<T>, dim3(g1), dim3(256), 0, st, dbc_part, (T*)dB, (T*)dC, ngrp, rows);
    const int64_t n2 = s.dim * kNState + s.dim;
    const int g2 = (int)((n2 + 255) / 256);
    hipLaunchKernelGGL(bwd_finish_ad_kernel<T>, dim3(g2), dim3(256), 0, st, dA_part, dD_part, (T*)dA, (T*)dD,
                       (int)s.batch, (int)s.dim);
    return hipGetLastError();
}

hipError_t launch_bwd_finish(bool is_half, const float* dbc_part, const float* dA_part, const float* dD_part,
                             void* dB, void* dC, void* dA, void* dD, int ngroups, const SsmShape& s,
                             hipStream_t st) {
    return is_half ? finish_t<half_t>(dbc_part, dA_part, dD_part, dB, dC, dA, dD, ngroups, s, st)
                   : finish_t<float>(dbc_part, dA_part, dD_part, dB, dC, dA, dD, ngroups, s, st);
}

}  // namespace mwc
