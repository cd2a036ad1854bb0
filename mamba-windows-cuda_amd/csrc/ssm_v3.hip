// Selective-scan forward/backward for gfx950, "state groups across waves" mapping.
//
// Semantics are those of ssm_fwd.hip / ssm_bwd.hip (the reference's fused
// forward, mamba_cuda.py:93-174, and the adjoint of selective_scan_ref,
// mamba_cuda.py:875-946, with h_prev / dh_last / dh_prev).
//
// Mapping: lane = channel. A 64-lane wave covers 64 consecutive channels for
// SPW of the 16 states; the NW = 16/SPW waves of a workgroup cover all states
// of the same 64 channels. Because every lane of a wave works on the same
// states, the per-step B/C values are wave-uniform: they come from a packed
// fp32 copy through scalar loads into SGPRs and feed the VALU as SGPR
// operands -- no LDS traffic and no VGPRs for B/C. The contractions over n
// (y in the forward, sum_n g*B and sum_n A*s in the backward) become one
// per-wave partial per (channel, step), written to LDS and combined once per
// 16-step chunk by the whole workgroup, which also applies D*u and writes the
// outputs as coalesced rows. Inputs (delta, delta*u, u, dout) are staged per
// chunk through LDS exactly as in the lane-group kernels; the backward's sums
// over channels (dB, dC) use a wave-private LDS slab folded every 4 steps
// against the staged per-channel weights, then summed over the workgroup's
// waves and written as deterministic per-group partials.
#include <type_traits>

#include "common.h"
#include "launch.h"

namespace mwc {

namespace {

template <int K>
__device__ __forceinline__ void ld4(const float* p, float (&v)[K]) {
    static_assert(K % 4 == 0, "vector width");
#pragma unroll
    for (int k = 0; k < K; k += 4) {
        const float4 q = *reinterpret_cast<const float4*>(p + k);
        v[k] = q.x;
        v[k + 1] = q.y;
        v[k + 2] = q.z;
        v[k + 3] = q.w;
    }
}

template <int K>
__device__ __forceinline__ void st4(float* p, const float (&v)[K]) {
    static_assert(K % 4 == 0, "vector width");
#pragma unroll
    for (int k = 0; k < K; k += 4) *reinterpret_cast<float4*>(p + k) = make_float4(v[k], v[k + 1], v[k + 2], v[k + 3]);
}

__device__ __forceinline__ void wave_lds_fence() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

constexpr int kCPB = 64;  // channels per workgroup (one per lane)
constexpr int kPF = 4;    // B/C prefetch distance (steps)

// A lane-varying zero: indexing with it keeps a wave-uniform row load on the vector
// memory path (tracked by vmcnt, so several steps can be in flight) instead of a
// scalar load that the compiler would issue just before its use.
__device__ __forceinline__ int opaque_zero() { return (int)__builtin_amdgcn_mbcnt_lo(0u, 0u); }
constexpr int kTC = kCkptSteps;
constexpr int kRS = kTC + 4;  // LDS row stride of a channel's steps

}  // namespace

// Packed per-step B/C rows for the wave-uniform scalar loads:
// bcp[(b*L + t)*32 + w*2*SPW + j] = B[b,t,w*SPW + j], and + SPW for C.
template <typename T, int SPW>
__global__ void __launch_bounds__(256) pack_bcw_kernel(const T* __restrict__ B, const T* __restrict__ C,
                                                       float* __restrict__ bcp, int64_t rows) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;  // one output float
    if (i >= rows * 32) return;
    const int64_t r = i >> 5;
    const int v = (int)(i & 31);
    const int w = v / (2 * SPW), o = v % (2 * SPW);
    const int n = w * SPW + (o % SPW);
    bcp[i] = static_cast<float>((o < SPW ? B : C)[r * kNState + n]);
}

// ------------------------------------------------------------------------- forward
template <typename T, int SPW, bool HAS_OUT>
__global__ void __launch_bounds__(64 * (kNState / SPW)) __attribute__((amdgpu_waves_per_eu(1, 2)))
ssm_fwd3_kernel(const T* __restrict__ u, const T* __restrict__ delta, const T* __restrict__ A,
                const float* __restrict__ bcp, const T* __restrict__ Dv, const T* __restrict__ h_prev,
                T* __restrict__ out, T* __restrict__ h_last, float* __restrict__ ckpt, int L, int D, int nck,
                int nblk_d) {
    constexpr int NW = kNState / SPW;
    constexpr int NT = 64 * NW;
    constexpr int SPG = kTC / NW;     // steps per loader thread
    constexpr int VPT = kTC * kCPB / NT;  // outputs per thread in the combine
    constexpr int YS = kCPB + 4;

    __shared__ float s_in[2][3][kCPB][kRS];  // [buf][delta, delta*u, u][channel][step]
    __shared__ float s_y[HAS_OUT ? NW : 1][HAS_OUT ? kTC : 1][HAS_OUT ? YS : 1];

    const int tid = threadIdx.x;
    const int lid = xcd_remap(blockIdx.x, gridDim.x);
    const int b = lid / nblk_d;
    const int d0 = (lid % nblk_d) * kCPB;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int c = tid & 63;
    const bool valid = d0 + c < D;
    const int d = valid ? d0 + c : D - 1;
    const int n0 = w * SPW;
    const int sg = tid >> 6;  // loader step group (= wave)
    const int64_t row0 = (int64_t)b * L;

    float A2[SPW], h[SPW];
    float amax2 = 0.f;
#pragma unroll
    for (int j = 0; j < SPW; ++j) {
        A2[j] = ld(A + (int64_t)d * kNState + n0 + j) * kLog2e;
        amax2 = __builtin_fmaxf(amax2, __builtin_fabsf(A2[j]));
        h[j] = h_prev ? ld(h_prev + ((int64_t)b * D + d) * kNState + n0 + j) : 0.f;
    }
    const float Dd = ld(Dv + d);

    T pu[SPG], pd[SPG];
    auto issue = [&](int k) {
#pragma unroll
        for (int s = 0; s < SPG; ++s) {
            const int t = min(k * kTC + sg * SPG + s, L - 1);
            const int64_t off = (row0 + t) * D + d;
            pu[s] = u[off];
            pd[s] = delta[off];
        }
    };
    auto commit = [&](int k, int buf) {
        float vd[SPG], vdu[SPG], vu[SPG];
#pragma unroll
        for (int s = 0; s < SPG; ++s) {
            const bool ok = valid && (k * kTC + sg * SPG + s < L);
            vd[s] = ok ? static_cast<float>(pd[s]) : 0.f;
            vu[s] = ok ? static_cast<float>(pu[s]) : 0.f;
            vdu[s] = vd[s] * vu[s];
        }
        st4<SPG>(&s_in[buf][0][c][sg * SPG], vd);
        st4<SPG>(&s_in[buf][1][c][sg * SPG], vdu);
        st4<SPG>(&s_in[buf][2][c][sg * SPG], vu);
    };

    if (nck > 0) {
        issue(0);
        commit(0, 0);
    }
    // ring of the next kPF steps' B/C values for this wave's states (wave-uniform rows)
    const float* bcrow = bcp + (row0 * NW + w) * (2 * SPW) + opaque_zero();
    auto fetch = [&](float (&dst)[2 * SPW], int t) {
        ld4<2 * SPW>(bcrow + (int64_t)min(t, L - 1) * (NW * 2 * SPW), dst);
    };
    float ring[kPF][2 * SPW];
#pragma unroll
    for (int p = 0; p < kPF; ++p) fetch(ring[p], p);
    __syncthreads();
    float* ckb = ckpt ? ckpt + ((int64_t)b * nck * D + d) * kNState + n0 : nullptr;

    for (int k = 0; k < nck; ++k) {
        const int buf = k & 1;
        const bool more = k + 1 < nck;
        if (more) issue(k + 1);
        if (ckb != nullptr && valid) st4<SPW>(ckb + (int64_t)k * D * kNState, h);

        float dt[kTC], dtu[kTC], uu[kTC];
        ld4<kTC>(&s_in[buf][0][c][0], dt);
        ld4<kTC>(&s_in[buf][1][c][0], dtu);
        if (HAS_OUT && w == 0) ld4<kTC>(&s_in[buf][2][c][0], uu);
        float dmax = 0.f;
#pragma unroll
        for (int i = 0; i < kTC; ++i) dmax = __builtin_fmaxf(dmax, __builtin_fabsf(dt[i]));
        const bool need_clamp = __builtin_amdgcn_ballot_w64(dmax * amax2 > kExp2Clamp) != 0;
        auto run = [&](auto clamp_tag) {
            constexpr bool CLAMP = decltype(clamp_tag)::value;
#pragma unroll
            for (int i = 0; i < kTC; ++i) {
                float r[2 * SPW];
#pragma unroll
                for (int j = 0; j < 2 * SPW; ++j) r[j] = ring[i % kPF][j];
                fetch(ring[i % kPF], k * kTC + i + kPF);
                float y = 0.f;
#pragma unroll
                for (int j = 0; j < SPW; ++j) {
                    const float x = dt[i] * A2[j];
                    const float e = CLAMP ? exp2_clamped(x) : __builtin_amdgcn_exp2f(x);
                    h[j] = __builtin_fmaf(e, h[j], dtu[i] * r[j]);
                    if constexpr (HAS_OUT) y = __builtin_fmaf(r[SPW + j], h[j], y);
                }
                if constexpr (HAS_OUT) {
                    if (w == 0) y = __builtin_fmaf(Dd, uu[i], y);
                    s_y[w][i][c] = y;
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
            // combine the waves' partials: thread -> (step, VPT consecutive channels)
            const int st_ = tid / (kCPB / VPT), cq = (tid % (kCPB / VPT)) * VPT;
            const int t = k * kTC + st_;
            float acc[VPT];
#pragma unroll
            for (int q = 0; q < VPT; ++q) acc[q] = 0.f;
#pragma unroll
            for (int ww = 0; ww < NW; ++ww) {
                float v[VPT];
                ld4<VPT>(&s_y[ww][st_][cq], v);
#pragma unroll
                for (int q = 0; q < VPT; ++q) acc[q] += v[q];
            }
            if (t < L) {
                T* op = out + (row0 + t) * D + d0 + cq;
#pragma unroll
                for (int q = 0; q < VPT; ++q)
                    if (d0 + cq + q < D) op[q] = static_cast<T>(acc[q]);
            }
            __syncthreads();  // s_y is rewritten by the next chunk
        }
    }
    if (h_last != nullptr && valid) {
#pragma unroll
        for (int j = 0; j < SPW; ++j) st(h_last + ((int64_t)b * D + d) * kNState + n0 + j, h[j]);
    }
}

// ------------------------------------------------------------------------- backward
template <typename T, int SPW>
__global__ void __launch_bounds__(64 * (kNState / SPW)) __attribute__((amdgpu_waves_per_eu(1, 2)))
ssm_bwd3_kernel(const T* __restrict__ u, const T* __restrict__ delta, const T* __restrict__ A,
                const float* __restrict__ bcp, const T* __restrict__ Dv, const T* __restrict__ dout,
                const T* __restrict__ dh_last, const float* __restrict__ ckpt, T* __restrict__ du,
                T* __restrict__ ddelta, T* __restrict__ dh_prev, float* __restrict__ dA_part,
                float* __restrict__ dD_part, float* __restrict__ dbc_part, int Bsz, int L, int D, int nck,
                int nblk_d) {
    constexpr int NW = kNState / SPW;
    constexpr int NT = 64 * NW;
    constexpr int SPG = kTC / NW;
    constexpr int VPT = kTC * kCPB / NT;  // combine outputs per thread
    constexpr int OS = kCPB + 4;
    constexpr int SLOTS = 4;              // steps per channel fold
    constexpr int RW = 2 * SPW;           // slab values per (slot, channel): g (dB) then h (dC)
    constexpr int RWP = RW + 4;           // padded row: 16 lanes' deposits hit distinct banks
    constexpr int NQ = SLOTS * 2;         // output quads per fold: slot x {dB, dC}, SPW states each
    constexpr int LPQ = 64 / NQ;          // lanes per quad
    constexpr int CPL = kCPB / LPQ;       // channels per folding lane
    static_assert(SPW == 4, "the backward uses state groups of 4");

    __shared__ float s_in[2][4][kCPB][kRS];    // [buf][delta, delta*u, u, dout][channel][step]
    __shared__ float s_r[2][NW][kTC][OS];      // [r1 = sum_n g*B, r2 = sum_n A*s][wave][step][channel]
    __shared__ float s_red[NW][SLOTS][kCPB][RWP];
    __shared__ float s_part[NW][kTC][2 * kNState];

    const int tid = threadIdx.x;
    const int lid = xcd_remap(blockIdx.x, gridDim.x);
    const int b = lid / nblk_d;
    const int blk = lid % nblk_d;
    const int d0 = blk * kCPB;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int c = tid & 63;
    const bool valid = d0 + c < D;
    const int d = valid ? d0 + c : D - 1;
    const int n0 = w * SPW;
    const int sg = tid >> 6;
    const int64_t row0 = (int64_t)b * L;

    // folding roles: quad q = lane / LPQ -> slot q>>1, kind q&1 (0 = dB, 1 = dC); sub = lane % LPQ
    const int fq = c / LPQ, fsub = c % LPQ;
    const int fslot = fq >> 1, fkind = fq & 1;

    float A2[SPW], gc[SPW], dAacc[SPW];
    float amax2 = 0.f;
#pragma unroll
    for (int j = 0; j < SPW; ++j) {
        A2[j] = ld(A + (int64_t)d * kNState + n0 + j) * kLog2e;
        amax2 = __builtin_fmaxf(amax2, __builtin_fabsf(A2[j]));
        gc[j] = (dh_last != nullptr && valid) ? ld(dh_last + ((int64_t)b * D + d) * kNState + n0 + j) : 0.f;
        dAacc[j] = 0.f;
    }
    float dDacc = 0.f;
    const float* ckb = ckpt + ((int64_t)b * nck * D + d) * kNState + n0;
    // combine role: thread -> (step st_, VPT consecutive channels cq..)
    const int st_ = tid / (kCPB / VPT), cq = (tid % (kCPB / VPT)) * VPT;
    float Dq[VPT];
#pragma unroll
    for (int q = 0; q < VPT; ++q) Dq[q] = ld(Dv + min(d0 + cq + q, D - 1));

    T pu[SPG], pd[SPG], py[SPG];
    float hnext[SPW];
    auto issue = [&](int k) {
#pragma unroll
        for (int s = 0; s < SPG; ++s) {
            const int t = min(k * kTC + sg * SPG + s, L - 1);
            const int64_t off = (row0 + t) * D + d;
            pu[s] = u[off];
            pd[s] = delta[off];
            py[s] = dout[off];
        }
        ld4<SPW>(ckb + (int64_t)k * D * kNState, hnext);
    };
    auto commit = [&](int k, int buf) {
        float vd[SPG], vdu[SPG], vu[SPG], vy[SPG];
#pragma unroll
        for (int s = 0; s < SPG; ++s) {
            const bool ok = valid && (k * kTC + sg * SPG + s < L);
            vd[s] = ok ? static_cast<float>(pd[s]) : 0.f;
            vu[s] = ok ? static_cast<float>(pu[s]) : 0.f;
            vy[s] = ok ? static_cast<float>(py[s]) : 0.f;
            vdu[s] = vd[s] * vu[s];
        }
        st4<SPG>(&s_in[buf][0][c][sg * SPG], vd);
        st4<SPG>(&s_in[buf][1][c][sg * SPG], vdu);
        st4<SPG>(&s_in[buf][2][c][sg * SPG], vu);
        st4<SPG>(&s_in[buf][3][c][sg * SPG], vy);
    };

    float hin[SPW];
    if (nck > 0) {
        issue(nck - 1);
        commit(nck - 1, (nck - 1) & 1);
#pragma unroll
        for (int j = 0; j < SPW; ++j) hin[j] = hnext[j];
    }
    __syncthreads();
    const float* bcrow = bcp + (row0 * NW + w) * (2 * SPW);

    for (int k = nck - 1; k >= 0; --k) {
        const int buf = k & 1;
        const int t0 = k * kTC;
        if (k > 0) issue(k - 1);

        float H[kTC][SPW], E[kTC][SPW], dt[kTC];
        {
            float dtu[kTC];
            ld4<kTC>(&s_in[buf][0][c][0], dt);
            ld4<kTC>(&s_in[buf][1][c][0], dtu);
            float dmax = 0.f;
#pragma unroll
            for (int i = 0; i < kTC; ++i) dmax = __builtin_fmaxf(dmax, __builtin_fabsf(dt[i]));
            const bool need_clamp = __builtin_amdgcn_ballot_w64(dmax * amax2 > kExp2Clamp) != 0;
            auto recompute = [&](auto clamp_tag) {
                constexpr bool CLAMP = decltype(clamp_tag)::value;
                float hh[SPW];
#pragma unroll
                for (int j = 0; j < SPW; ++j) hh[j] = hin[j];
#pragma unroll
                for (int i = 0; i < kTC; ++i) {
                    const float* r = bcrow + (int64_t)min(t0 + i, L - 1) * (NW * 2 * SPW);
#pragma unroll
                    for (int j = 0; j < SPW; ++j) {
                        const float x = dt[i] * A2[j];
                        E[i][j] = CLAMP ? exp2_clamped(x) : __builtin_amdgcn_exp2f(x);
                        hh[j] = __builtin_fmaf(E[i][j], hh[j], dtu[i] * r[j]);
                        H[i][j] = hh[j];
                    }
                }
            };
            if (need_clamp)
                recompute(std::true_type{});
            else
                recompute(std::false_type{});
        }

        float (*red)[kCPB][RWP] = s_red[w];
        float yq[kTC];
        ld4<kTC>(&s_in[buf][3][c][0], yq);
#pragma unroll
        for (int i = kTC - 1; i >= 0; --i) {
            const int slot = i % SLOTS;
            const float yo = yq[i];
            const float* r = bcrow + (int64_t)min(t0 + i, L - 1) * (NW * 2 * SPW);
            float dep[RWP];
            float r1 = 0.f, r2 = 0.f;
#pragma unroll
            for (int j = 0; j < SPW; ++j) {
                const float prev = (i > 0) ? H[i > 0 ? i - 1 : 0][j] : hin[j];
                const float gt = __builtin_fmaf(yo, r[SPW + j], gc[j]);
                r1 = __builtin_fmaf(gt, r[j], r1);
                const float s = gt * E[i][j] * prev;
                r2 = __builtin_fmaf(A2[j], s, r2);
                dAacc[j] = __builtin_fmaf(dt[i], s, dAacc[j]);
                gc[j] = E[i][j] * gt;
                dep[j] = gt;
                dep[SPW + j] = H[i][j];
            }
#pragma unroll
            for (int j = RW; j < RWP; ++j) dep[j] = 0.f;
            s_r[0][w][i][c] = r1;
            s_r[1][w][i][c] = r2;
            st4<RW>(&red[slot][c][0], *reinterpret_cast<float(*)[RW]>(dep));
            if (slot == 0) {
                wave_lds_fence();
                // fold steps i..i+3 over this wave's 64 channels: quad (slot, kind), CPL channels per lane
                const float* wcol = &s_in[buf][fkind ? 3 : 1][0][i + fslot];
                float acc[SPW];
#pragma unroll
                for (int j = 0; j < SPW; ++j) acc[j] = 0.f;
#pragma unroll
                for (int m = 0; m < CPL; ++m) {
                    const int ch = m * LPQ + fsub;
                    float v[SPW];
                    ld4<SPW>(&red[fslot][ch][fkind * SPW], v);
                    const float wgt = wcol[ch * kRS];
#pragma unroll
                    for (int j = 0; j < SPW; ++j) acc[j] = __builtin_fmaf(v[j], wgt, acc[j]);
                }
#pragma unroll
                for (int j = 0; j < SPW; ++j) acc[j] = group_sum<LPQ>(acc[j]);
                if (fsub == 0) {
#pragma unroll
                    for (int j = 0; j < SPW; ++j) s_part[w][i + fslot][fkind * kNState + n0 + j] = acc[j];
                }
                wave_lds_fence();
            }
        }
        if (k > 0) {
            commit(k - 1, buf ^ 1);
#pragma unroll
            for (int j = 0; j < SPW; ++j) hin[j] = hnext[j];
        }
        __syncthreads();
        // combine: thread -> (step, VPT channels): du, ddelta, dD
        {
            const int t = t0 + st_;
            float r1[VPT], r2[VPT];
#pragma unroll
            for (int q = 0; q < VPT; ++q) r1[q] = r2[q] = 0.f;
#pragma unroll
            for (int ww = 0; ww < NW; ++ww) {
                float a1[VPT], a2[VPT];
                if constexpr (VPT % 4 == 0) {
                    ld4<VPT>(&s_r[0][ww][st_][cq], a1);
                    ld4<VPT>(&s_r[1][ww][st_][cq], a2);
                } else {
#pragma unroll
                    for (int q = 0; q < VPT; ++q) {
                        a1[q] = s_r[0][ww][st_][cq + q];
                        a2[q] = s_r[1][ww][st_][cq + q];
                    }
                }
#pragma unroll
                for (int q = 0; q < VPT; ++q) {
                    r1[q] += a1[q];
                    r2[q] += a2[q];
                }
            }
            if (t < L) {
                T* pdu = du + (row0 + t) * D + d0 + cq;
                T* pdd = ddelta + (row0 + t) * D + d0 + cq;
#pragma unroll
                for (int q = 0; q < VPT; ++q) {
                    const int cc = cq + q;
                    if (d0 + cc < D) {
                        const float dtv = s_in[buf][0][cc][st_], uv = s_in[buf][2][cc][st_];
                        const float yv = s_in[buf][3][cc][st_];
                        pdu[q] = static_cast<T>(__builtin_fmaf(Dq[q], yv, dtv * r1[q]));
                        // sum_n A*s was accumulated with A*log2(e)
                        pdd[q] = static_cast<T>(__builtin_fmaf(uv, r1[q], r2[q] * 0.69314718055994531f));
                    }
                }
            }
        }
        // dD partial: one thread per channel over the chunk's steps
        if (tid < kCPB) {
#pragma unroll
            for (int i = 0; i < kTC; ++i) dDacc = __builtin_fmaf(s_in[buf][3][tid][i], s_in[buf][2][tid][i], dDacc);
        }
        for (int o = tid; o < kTC * 2 * kNState; o += NT) {
            const int tt = o >> 5, v = o & 31;
            const int wv = (v & 15) / SPW;  // the wave that owns state v%16
            const float s = s_part[wv][tt][v];
            if (t0 + tt < L) dbc_part[(((int64_t)blk * Bsz + b) * L + t0 + tt) * 32 + v] = s;
        }
        __syncthreads();  // s_r, s_part and the input buffer are reused by the next chunk
    }

    if (valid) {
        if (dh_prev != nullptr) {
#pragma unroll
            for (int j = 0; j < SPW; ++j) st(dh_prev + ((int64_t)b * D + d) * kNState + n0 + j, gc[j]);
        }
#pragma unroll
        for (int j = 0; j < SPW; ++j) dA_part[((int64_t)b * D + d) * kNState + n0 + j] = dAacc[j];
    }
    if (tid < kCPB && d0 + tid < D) dD_part[(int64_t)b * D + d0 + tid] = dDacc;
}

// ------------------------------------------------------------------------- launchers

size_t v3_bcp_bytes(const SsmShape& s) { return (((size_t)s.batch * s.seqlen * 32 * sizeof(float)) + 255) & ~(size_t)255; }

int v3_groups(const SsmShape& s) { return (int)((s.dim + kCPB - 1) / kCPB); }

template <typename T, int SPW>
static hipError_t v3_pack(const void* B, const void* C, float* bcp, int64_t rows, hipStream_t st) {
    const int64_t n = rows * 32;
    const int grid = (int)((n + 255) / 256);
    if (grid > 0)
        hipLaunchKernelGGL((pack_bcw_kernel<T, SPW>), dim3(grid), dim3(256), 0, st, (const T*)B, (const T*)C, bcp, rows);
    return hipGetLastError();
}

hipError_t launch_v3_pack(bool is_half, const void* B, const void* C, float* bcp, const SsmShape& s, hipStream_t st) {
    return is_half ? v3_pack<half_t, 4>(B, C, bcp, s.batch * s.seqlen, st)
                   : v3_pack<float, 4>(B, C, bcp, s.batch * s.seqlen, st);
}

template <typename T>
static hipError_t fwd3_t(const void* u, const void* delta, const void* A, const float* bcp, const void* Dv,
                         const void* h_prev, void* out, void* h_last, float* ckpt, const SsmShape& s,
                         hipStream_t st) {
    constexpr int SPW = 4;
    const int nblk_d = v3_groups(s);
    const int grid = nblk_d * (int)s.batch;
    const int nck = (int)((s.seqlen + kCkptSteps - 1) / kCkptSteps);
    const dim3 blk(64 * (kNState / SPW));
    if (out != nullptr)
        hipLaunchKernelGGL((ssm_fwd3_kernel<T, SPW, true>), dim3(grid), blk, 0, st, (const T*)u, (const T*)delta,
                           (const T*)A, bcp, (const T*)Dv, (const T*)h_prev, (T*)out, (T*)h_last, ckpt,
                           (int)s.seqlen, (int)s.dim, nck, nblk_d);
    else
        hipLaunchKernelGGL((ssm_fwd3_kernel<T, SPW, false>), dim3(grid), blk, 0, st, (const T*)u, (const T*)delta,
                           (const T*)A, bcp, (const T*)Dv, (const T*)h_prev, (T*)out, (T*)h_last, ckpt,
                           (int)s.seqlen, (int)s.dim, nck, nblk_d);
    return hipGetLastError();
}

hipError_t launch_v3_fwd(bool is_half, const void* u, const void* delta, const void* A, const float* bcp,
                         const void* Dv, const void* h_prev, void* out, void* h_last, float* ckpt, const SsmShape& s,
                         hipStream_t st) {
    return is_half ? fwd3_t<half_t>(u, delta, A, bcp, Dv, h_prev, out, h_last, ckpt, s, st)
                   : fwd3_t<float>(u, delta, A, bcp, Dv, h_prev, out, h_last, ckpt, s, st);
}

template <typename T>
static hipError_t bwd3_t(const void* u, const void* delta, const void* A, const float* bcp, const void* Dv,
                         const void* dout, const void* dh_last, const float* ckpt, void* du, void* ddelta,
                         void* dh_prev, float* dA_part, float* dD_part, float* dbc_part, const SsmShape& s,
                         hipStream_t st) {
    constexpr int SPW = 4;
    const int nblk_d = v3_groups(s);
    const int grid = nblk_d * (int)s.batch;
    const int nck = (int)((s.seqlen + kCkptSteps - 1) / kCkptSteps);
    hipLaunchKernelGGL((ssm_bwd3_kernel<T, SPW>), dim3(grid), dim3(64 * (kNState / SPW)), 0, st, (const T*)u,
                       (const T*)delta, (const T*)A, bcp, (const T*)Dv, (const T*)dout, (const T*)dh_last, ckpt,
                       (T*)du, (T*)ddelta, (T*)dh_prev, dA_part, dD_part, dbc_part, (int)s.batch, (int)s.seqlen,
                       (int)s.dim, nck, nblk_d);
    return hipGetLastError();
}

hipError_t launch_v3_bwd(bool is_half, const void* u, const void* delta, const void* A, const float* bcp,
                         const void* Dv, const void* dout, const void* dh_last, const float* ckpt, void* du,
                         void* ddelta, void* dh_prev, float* dA_part, float* dD_part, float* dbc_part,
                         const SsmShape& s, hipStream_t st) {
    return is_half ? bwd3_t<half_t>(u, delta, A, bcp, Dv, dout, dh_last, ckpt, du, ddelta, dh_prev, dA_part,
                                    dD_part, dbc_part, s, st)
                   : bwd3_t<float>(u, delta, A, bcp, Dv, dout, dh_last, ckpt, du, ddelta, dh_prev, dA_part,
                                   dD_part, dbc_part, s, st);
}

}  // namespace mwc
