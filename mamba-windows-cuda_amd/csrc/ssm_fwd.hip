// Fused selective-scan forward for gfx950.
//
// Semantics: the reference's fused forward kernel (mamba_cuda.py:93-174) and
// selective_scan_ref (mamba_cuda.py:875-946): per channel (b,d) and state n,
//   dA = exp(clamp(delta*A, -88, 88)); h = dA*h + delta*u*B; y = sum_n C*h + D*u.
//
// Mapping (not the reference's one-warp-per-channel serial loop): a channel's
// 16 states are spread over a group of LPC = 16/SPL consecutive lanes, each
// lane holding SPL states in VGPRs; a 64-lane wave scans 64/LPC channels and a
// 4-wave workgroup CPB = 4*64/LPC channels of one batch row, walking L in
// chunks of 16 steps. The C-contraction is an in-register FMA chain plus a DPP
// all-reduce inside the lane group.
//
// Data movement: the workgroup stages each chunk's inputs through LDS --
// delta, delta*u and u as fp32 rows per channel (converted once, read back by
// the lanes as 128-bit vectors) and the chunk's B/C rows -- double-buffered,
// with the next chunk's global loads issued before the current chunk is
// computed, so one barrier per chunk is the only synchronisation. Outputs go
// through an LDS tile and leave as coalesced row stores. Steps past L are
// padded with delta = u = 0, which leaves the state unchanged, so the inner
// loop carries no bounds checks. With at most one wave per SIMD at the target
// shapes every issued instruction costs the wave 4 cycles, so the design
// minimises instructions per state, not just VALU work.
#include <type_traits>

#include "common.h"
#include "launch.h"

namespace mwc {

template <int K>
__device__ __forceinline__ void lds_ld(const float* p, float (&v)[K]) {
    static_assert(K % 4 == 0 || K < 4, "vector width");
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
__device__ __forceinline__ void vst(float* p, const float (&v)[K]) {
    if constexpr (K % 4 == 0) {
#pragma unroll
        for (int k = 0; k < K; k += 4) *reinterpret_cast<float4*>(p + k) = make_float4(v[k], v[k + 1], v[k + 2], v[k + 3]);
    } else if constexpr (K == 2) {
        *reinterpret_cast<float2*>(p) = make_float2(v[0], v[1]);
    } else {
        *p = v[0];
    }
}

template <typename T, int SPL, bool HAS_OUT>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 2))) ssm_fwd_kernel(const T* __restrict__ u, const T* __restrict__ delta,
                                                      const T* __restrict__ A, const T* __restrict__ Bm,
                                                      const T* __restrict__ Cm, const T* __restrict__ Dv,
                                                      const T* __restrict__ h_prev, T* __restrict__ out,
                                                      T* __restrict__ h_last, float* __restrict__ ckpt, int L, int D,
                                                      int nck, int nblk_d) {
    constexpr int LPC = kNState / SPL;  // lanes per channel
    constexpr int CPW = 64 / LPC;       // channels per wave
    constexpr int CPB = CPW * 4;        // channels per workgroup
    constexpr int TC = kCkptSteps;      // steps per chunk
    constexpr int RS = TC + 4;          // LDS row stride (floats) of a channel's steps
    constexpr int NSG = 256 / CPB;      // loader step groups
    constexpr int SPG = TC / NSG;       // steps per loader thread
    constexpr int YS = CPB + 4;         // LDS row stride of the output tile
    static_assert(NSG * SPG == TC, "loader tiling");

    __shared__ float s_in[2][3][CPB][RS];  // [buf][delta, delta*u, u][channel][step]
    __shared__ float s_bc[2][TC][2 * kNState];
    __shared__ float s_y[HAS_OUT ? 2 : 1][HAS_OUT ? TC : 1][HAS_OUT ? YS : 1];

    const int tid = threadIdx.x;
    const int lid = xcd_remap(blockIdx.x, gridDim.x);
    const int b = lid / nblk_d;
    const int d0 = (lid % nblk_d) * CPB;

    // consumer role
    const int wave = tid >> 6, lane = tid & 63;
    const int c = wave * CPW + lane / LPC;
    const int g = lane % LPC;
    const int n0 = g * SPL;
    const bool valid = d0 + c < D;
    const int d = valid ? d0 + c : D - 1;

    // loader roles: (channel lc, steps sg*SPG..) for u/delta; (step, n) for B/C
    const int lc = tid % CPB, sg = tid / CPB;
    const bool lvalid = d0 + lc < D;
    const int ld_d = lvalid ? d0 + lc : D - 1;
    const int bc_t = tid >> 4, bc_n = tid & 15;
    const int64_t row0 = (int64_t)b * L;

    float A2[SPL], h[SPL];
#pragma unroll
    for (int j = 0; j < SPL; ++j) {
        A2[j] = ld(A + (int64_t)d * kNState + n0 + j) * kLog2e;
        h[j] = h_prev ? ld(h_prev + ((int64_t)b * D + d) * kNState + n0 + j) : 0.f;
    }
    const float Dd = ld(Dv + d);
    float amax2 = 0.f;  // max_j |A_j| * log2(e) over this lane's states
#pragma unroll
    for (int j = 0; j < SPL; ++j) amax2 = __builtin_fmaxf(amax2, __builtin_fabsf(A2[j]));

    T pu[SPG], pd[SPG], pb, pc;
    auto issue = [&](int k) {
#pragma unroll
        for (int s = 0; s < SPG; ++s) {
            const int t = min(k * TC + sg * SPG + s, L - 1);
            const int64_t off = (row0 + t) * D + ld_d;
            pu[s] = u[off];
            pd[s] = delta[off];
        }
        const int t = min(k * TC + bc_t, L - 1);
        pb = Bm[(row0 + t) * kNState + bc_n];
        if constexpr (HAS_OUT) pc = Cm[(row0 + t) * kNState + bc_n];
    };
    auto commit = [&](int k, int buf) {
        float vd[SPG], vdu[SPG], vu[SPG];
#pragma unroll
        for (int s = 0; s < SPG; ++s) {
            const bool ok = lvalid && (k * TC + sg * SPG + s < L);
            vd[s] = ok ? static_cast<float>(pd[s]) : 0.f;
            vu[s] = ok ? static_cast<float>(pu[s]) : 0.f;
            vdu[s] = vd[s] * vu[s];
        }
        vst<SPG>(&s_in[buf][0][lc][sg * SPG], vd);
        vst<SPG>(&s_in[buf][1][lc][sg * SPG], vdu);
        vst<SPG>(&s_in[buf][2][lc][sg * SPG], vu);
        s_bc[buf][bc_t][bc_n] = static_cast<float>(pb);
        if constexpr (HAS_OUT) s_bc[buf][bc_t][kNState + bc_n] = static_cast<float>(pc);
    };

    if (nck > 0) {  // L == 0: no chunk, h_last = h_prev
        issue(0);
        commit(0, 0);
    }
    __syncthreads();
    float* ckb = ckpt ? ckpt + ((int64_t)b * nck * D + d) * kNState + n0 : nullptr;

    for (int k = 0; k < nck; ++k) {
        const int buf = k & 1;
        const bool more = k + 1 < nck;
        if (more) issue(k + 1);
        if (ckb != nullptr && valid) vst<SPL>(ckb + (int64_t)k * D * kNState, h);

        // the whole chunk's operands, read up front so LDS latency is paid once per chunk
        float dt[TC], dtu[TC], uu[TC], Bv[TC][SPL], Cv[TC][SPL];
        lds_ld<TC>(&s_in[buf][0][c][0], dt);
        lds_ld<TC>(&s_in[buf][1][c][0], dtu);
        if constexpr (HAS_OUT) lds_ld<TC>(&s_in[buf][2][c][0], uu);
#pragma unroll
        for (int i = 0; i < TC; ++i) {
            lds_ld<SPL>(&s_bc[buf][i][n0], Bv[i]);
            if constexpr (HAS_OUT) lds_ld<SPL>(&s_bc[buf][i][kNState + n0], Cv[i]);
        }
        // |delta*A| <= 88 for the whole chunk (the usual case) -> no clamp needed
        float dmax = 0.f;
#pragma unroll
        for (int i = 0; i < TC; ++i) dmax = __builtin_fmaxf(dmax, __builtin_fabsf(dt[i]));
        const bool need_clamp = __builtin_amdgcn_ballot_w64(dmax * amax2 > kExp2Clamp) != 0;
        auto run = [&](auto clamp_tag) {
            constexpr bool CLAMP = decltype(clamp_tag)::value;
#pragma unroll
            for (int i = 0; i < TC; ++i) {
                float y = 0.f;
#pragma unroll
                for (int j = 0; j < SPL; ++j) {
                    const float x = dt[i] * A2[j];
                    const float e = CLAMP ? exp2_clamped(x) : __builtin_amdgcn_exp2f(x);
                    h[j] = __builtin_fmaf(e, h[j], dtu[i] * Bv[i][j]);
                    if constexpr (HAS_OUT) y = __builtin_fmaf(Cv[i][j], h[j], y);
                }
                if constexpr (HAS_OUT) {
                    y = group_sum<LPC>(y);
                    // every lane of the group holds the sum; the duplicate LDS writes are identical
                    s_y[buf][i][c] = __builtin_fmaf(Dd, uu[i], y);
                }
            }
        };
        if (need_clamp)
            run(std::true_type{});
        else
            run(std::false_type{});
        if (more) commit(k + 1, buf ^ 1);
        __syncthreads();
        if constexpr (HAS_OUT) {
            // coalesced store of the chunk's output tile: thread -> (step, SPG channels)
            constexpr int VPT = CPB / (256 / TC);  // channels per thread
            const int st = tid / (CPB / VPT), cq = (tid % (CPB / VPT)) * VPT;
            const int t = k * TC + st;
            if (t < L) {
                float v[VPT];
                lds_ld<VPT>(&s_y[buf][st][cq], v);
                T* op = out + (row0 + t) * D + d0 + cq;
#pragma unroll
                for (int q = 0; q < VPT; ++q)
                    if (d0 + cq + q < D) op[q] = static_cast<T>(v[q]);
            }
        }
    }
    if (h_last != nullptr && valid) {
#pragma unroll
        for (int j = 0; j < SPL; ++j) st(h_last + ((int64_t)b * D + d) * kNState + n0 + j, h[j]);
    }
}

template <typename T, int SPL>
static hipError_t fwd_inst(const void* u, const void* delta, const void* A, const void* B, const void* C,
                           const void* Dv, const void* h_prev, void* out, void* h_last, float* ckpt,
                           const SsmShape& s, hipStream_t st) {
    constexpr int CPB = 4 * 64 / (kNState / SPL);
    const int nblk_d = (int)((s.dim + CPB - 1) / CPB);
    const int grid = nblk_d * (int)s.batch;
    const int nck = (int)((s.seqlen + kCkptSteps - 1) / kCkptSteps);
    if (out != nullptr)
        hipLaunchKernelGGL((ssm_fwd_kernel<T, SPL, true>), dim3(grid), dim3(256), 0, st, (const T*)u,
                           (const T*)delta, (const T*)A, (const T*)B, (const T*)C, (const T*)Dv, (const T*)h_prev,
                           (T*)out, (T*)h_last, ckpt, (int)s.seqlen, (int)s.dim, nck, nblk_d);
    else
        hipLaunchKernelGGL((ssm_fwd_kernel<T, SPL, false>), dim3(grid), dim3(256), 0, st, (const T*)u,
                           (const T*)delta, (const T*)A, (const T*)B, (const T*)C, (const T*)Dv, (const T*)h_prev,
                           (T*)out, (T*)h_last, ckpt, (int)s.seqlen, (int)s.dim, nck, nblk_d);
    return hipGetLastError();
}

hipError_t launch_ssm_fwd(bool is_half, int spl, const void* u, const void* delta, const void* A, const void* B,
                          const void* C, const void* Dv, const void* h_prev, void* out, void* h_last, float* ckpt,
                          const SsmShape& s, hipStream_t st) {
#define MWC_FWD_SPL(S)                                                                                     \
    if (spl == S)                                                                                          \
        return is_half ? fwd_inst<half_t, S>(u, delta, A, B, C, Dv, h_prev, out, h_last, ckpt, s, st)     \
                       : fwd_inst<float, S>(u, delta, A, B, C, Dv, h_prev, out, h_last, ckpt, s, st);
    MWC_FWD_SPL(1)
    MWC_FWD_SPL(2)
    MWC_FWD_SPL(4)
#undef MWC_FWD_SPL
    return hipErrorInvalidValue;
}

}  // namespace mwc
