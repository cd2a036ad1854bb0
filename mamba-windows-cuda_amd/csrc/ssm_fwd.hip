// Fused selective-scan forward for gfx950.
//
// Semantics: the reference's fused forward kernel (mamba_cuda.py:93-174) and
// selective_scan_ref (mamba_cuda.py:875-946): per channel (b,d) and state n,
//   dA = exp(clamp(delta*A, -88, 88)); h = dA*h + delta*u*B; y = sum_n C*h + D*u.
//
// Mapping (not the reference's one-warp-per-channel serial loop): a channel's
// 16 states are spread over a group of LPC = 16/SPL consecutive lanes, each
// lane holding SPL states in VGPRs; a 64-lane wave therefore scans 64/LPC
// channels at once and walks L sequentially. The C-contraction is an
// in-register FMA chain followed by a DPP all-reduce inside the lane group --
// no LDS, no barriers. u/delta loads are contiguous along D; B/C come from a
// packed fp32 [B][L][32] copy so a lane fetches its SPL values with one vector
// load. Loads for the next block of steps are issued before the current block
// is computed (register double buffering) to hide HBM/L2 latency with one
// wave per SIMD.
#include "common.h"
#include "launch.h"

namespace mwc {

template <typename T>
__global__ void __launch_bounds__(256) pack_bc_kernel(const T* __restrict__ B, const T* __restrict__ C,
                                                      float* __restrict__ bc, int64_t rows) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;  // one float4 of bc
    if (i >= rows * 8) return;
    const int64_t r = i >> 3;
    const int q = (int)(i & 7);
    const T* src = (q < 4 ? B : C) + r * kNState + (q & 3) * 4;
    float4 v;
    v.x = ld(src);
    v.y = ld(src + 1);
    v.z = ld(src + 2);
    v.w = ld(src + 3);
    reinterpret_cast<float4*>(bc)[i] = v;
}

template <int K>
__device__ __forceinline__ void load_f32(const float* __restrict__ p, float (&v)[K]) {
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
__device__ __forceinline__ void store_f32(float* __restrict__ p, const float (&v)[K]) {
    if constexpr (K % 4 == 0) {
#pragma unroll
        for (int k = 0; k < K; k += 4) *reinterpret_cast<float4*>(p + k) = make_float4(v[k], v[k + 1], v[k + 2], v[k + 3]);
    } else if constexpr (K == 2) {
        *reinterpret_cast<float2*>(p) = make_float2(v[0], v[1]);
    } else {
        *p = v[0];
    }
}

template <typename T, int SPL, int U>
struct FwdBlock {
    float dt[U], ut[U], Bv[U][SPL], Cv[U][SPL];

    template <bool NEED_C>
    __device__ __forceinline__ void load(const T* __restrict__ up, const T* __restrict__ dp,
                                         const float* __restrict__ bcb, int t0, int D) {
#pragma unroll
        for (int i = 0; i < U; ++i) {
            const int64_t t = t0 + i;
            dt[i] = ld(dp + t * D);
            ut[i] = ld(up + t * D);
            load_f32<SPL>(bcb + t * 32, Bv[i]);
            if constexpr (NEED_C) load_f32<SPL>(bcb + t * 32 + kNState, Cv[i]);
        }
    }
};

template <typename T, int SPL, bool HAS_OUT>
__global__ void __launch_bounds__(64) ssm_fwd_kernel(const T* __restrict__ u, const T* __restrict__ delta,
                                                     const T* __restrict__ A, const float* __restrict__ bc,
                                                     const T* __restrict__ Dv, const T* __restrict__ h_prev,
                                                     T* __restrict__ out, T* __restrict__ h_last,
                                                     float* __restrict__ ckpt, int L, int D, int nck,
                                                     int nblk_d) {
    constexpr int LPC = kNState / SPL;  // lanes per channel
    constexpr int CPW = 64 / LPC;       // channels per wave
    constexpr int U = 8;                // steps per register block
    static_assert(kCkptSteps % U == 0, "checkpoint interval must be a multiple of the block");

    const int lid = xcd_remap(blockIdx.x, gridDim.x);
    const int b = lid / nblk_d;
    const int lane = threadIdx.x;
    const int c = lane / LPC, g = lane % LPC;
    const int d_raw = (lid % nblk_d) * CPW + c;
    const bool valid = d_raw < D;
    const int d = valid ? d_raw : D - 1;
    const int n0 = g * SPL;

    float A2[SPL], h[SPL];
#pragma unroll
    for (int j = 0; j < SPL; ++j) {
        A2[j] = ld(A + (int64_t)d * kNState + n0 + j) * kLog2e;
        h[j] = h_prev ? ld(h_prev + ((int64_t)b * D + d) * kNState + n0 + j) : 0.f;
    }
    const float Dd = ld(Dv + d);
    const int64_t base = (int64_t)b * L * D + d;
    const T* __restrict__ up = u + base;
    const T* __restrict__ dp = delta + base;
    T* __restrict__ op = HAS_OUT ? out + base : nullptr;
    const float* __restrict__ bcb = bc + (int64_t)b * L * 32 + n0;
    float* __restrict__ ckb = ckpt ? ckpt + ((int64_t)b * nck * D + d) * kNState + n0 : nullptr;
    const int64_t ck_stride = (int64_t)D * kNState;

    // Checkpoint k = state before step k*kCkptSteps (checkpoint 0 = h_prev).
    auto checkpoint = [&](int t) {
        if (ckb != nullptr && t % kCkptSteps == 0 && valid) store_f32<SPL>(ckb + (t / kCkptSteps) * ck_stride, h);
    };
    auto step = [&](int t, float dt, float ut, const float (&Bv)[SPL], const float (&Cv)[SPL]) {
        const float dtu = dt * ut;
        float y = 0.f;
#pragma unroll
        for (int j = 0; j < SPL; ++j) {
            const float e = exp2_clamped(dt * A2[j]);
            h[j] = __builtin_fmaf(e, h[j], dtu * Bv[j]);
            if constexpr (HAS_OUT) y = __builtin_fmaf(Cv[j], h[j], y);
        }
        if constexpr (HAS_OUT) {
            y = group_sum<LPC>(y);
            if (g == 0 && valid) st(op + (int64_t)t * D, __builtin_fmaf(Dd, ut, y));
        }
    };

    const int Lmain = L - L % U;
    FwdBlock<T, SPL, U> X, Y;
    int t0 = 0;
    if (Lmain > 0) X.template load<HAS_OUT>(up, dp, bcb, 0, D);
    while (t0 < Lmain) {
        bool more = t0 + U < Lmain;
        if (more) Y.template load<HAS_OUT>(up, dp, bcb, t0 + U, D);
        checkpoint(t0);
#pragma unroll
        for (int i = 0; i < U; ++i) step(t0 + i, X.dt[i], X.ut[i], X.Bv[i], X.Cv[i]);
        t0 += U;
        if (!more) break;
        more = t0 + U < Lmain;
        if (more) X.template load<HAS_OUT>(up, dp, bcb, t0 + U, D);
        checkpoint(t0);
#pragma unroll
        for (int i = 0; i < U; ++i) step(t0 + i, Y.dt[i], Y.ut[i], Y.Bv[i], Y.Cv[i]);
        t0 += U;
        if (!more) break;
    }
    for (int t = Lmain; t < L; ++t) {
        float Bv[SPL], Cv[SPL];
        load_f32<SPL>(bcb + (int64_t)t * 32, Bv);
        if constexpr (HAS_OUT) load_f32<SPL>(bcb + (int64_t)t * 32 + kNState, Cv);
        checkpoint(t);
        step(t, ld(dp + (int64_t)t * D), ld(up + (int64_t)t * D), Bv, Cv);
    }
    if (h_last != nullptr) {
        if (valid) {
#pragma unroll
            for (int j = 0; j < SPL; ++j) st(h_last + ((int64_t)b * D + d) * kNState + n0 + j, h[j]);
        }
    }
}

template <typename T>
static hipError_t pack_bc_t(const void* B, const void* C, float* bc, int64_t rows, hipStream_t st) {
    const int64_t n = rows * 8;
    const int grid = (int)((n + 255) / 256);
    if (grid > 0)
        hipLaunchKernelGGL(pack_bc_kernel<T>, dim3(grid), dim3(256), 0, st, (const T*)B, (const T*)C, bc, rows);
    return hipGetLastError();
}

hipError_t launch_pack_bc(bool is_half, const void* B, const void* C, float* bc, int64_t rows, hipStream_t st) {
    return is_half ? pack_bc_t<half_t>(B, C, bc, rows, st) : pack_bc_t<float>(B, C, bc, rows, st);
}

template <typename T, int SPL>
static hipError_t fwd_inst(const void* u, const void* delta, const void* A, const float* bc, const void* Dv,
                           const void* h_prev, void* out, void* h_last, float* ckpt, const SsmShape& s,
                           hipStream_t st) {
    constexpr int CPW = 64 / (kNState / SPL);
    const int nblk_d = (int)((s.dim + CPW - 1) / CPW);
    const int grid = nblk_d * (int)s.batch;
    const int nck = (int)((s.seqlen + kCkptSteps - 1) / kCkptSteps);
    if (out != nullptr)
        hipLaunchKernelGGL((ssm_fwd_kernel<T, SPL, true>), dim3(grid), dim3(64), 0, st, (const T*)u,
                           (const T*)delta, (const T*)A, bc, (const T*)Dv, (const T*)h_prev, (T*)out, (T*)h_last,
                           ckpt, (int)s.seqlen, (int)s.dim, nck, nblk_d);
    else
        hipLaunchKernelGGL((ssm_fwd_kernel<T, SPL, false>), dim3(grid), dim3(64), 0, st, (const T*)u,
                           (const T*)delta, (const T*)A, bc, (const T*)Dv, (const T*)h_prev, (T*)out, (T*)h_last,
                           ckpt, (int)s.seqlen, (int)s.dim, nck, nblk_d);
    return hipGetLastError();
}

hipError_t launch_ssm_fwd(bool is_half, int spl, const void* u, const void* delta, const void* A, const float* bc,
                          const void* Dv, const void* h_prev, void* out, void* h_last, float* ckpt,
                          const SsmShape& s, hipStream_t st) {
#define MWC_FWD_SPL(S)                                                                                   \
    if (spl == S)                                                                                        \
        return is_half ? fwd_inst<half_t, S>(u, delta, A, bc, Dv, h_prev, out, h_last, ckpt, s, st) \
                       : fwd_inst<float, S>(u, delta, A, bc, Dv, h_prev, out, h_last, ckpt, s, st);
    MWC_FWD_SPL(1)
    MWC_FWD_SPL(2)
    MWC_FWD_SPL(4)
#undef MWC_FWD_SPL
    return hipErrorInvalidValue;
}

}  // namespace mwc
