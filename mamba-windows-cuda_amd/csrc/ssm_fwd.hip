// Fused selective-scan forward for gfx950.
//
// Semantics: the reference's fused forward kernel (mamba_cuda.py:93-174) and
// selective_scan_ref (mamba_cuda.py:875-946): per channel (b,d) and state n,
//   dA = exp(clamp(delta*A, -88, 88)); h = dA*h + delta*u*B; y = sum_n C*h + D*u.
//
// Mapping (not the reference's one-warp-per-channel serial loop): a channel's
// N states (16 in the reference; 8, 32 and 64 are built too) are spread over a
// group of LPC = N/SPL consecutive lanes, each lane holding SPL states in
// VGPRs; a 64-lane wave scans 64/LPC channels and a
// 4-wave workgroup CPB = 4*64/LPC channels of one batch row, walking its part
// of L in chunks of 16 steps. The C-contraction is an in-register FMA chain
// plus a DPP all-reduce inside the lane group.
//
// Parallelism over L: the sequence is cut into `nseg` segments of whole chunks
// so that the grid fills every SIMD evenly. A carry pass (FwdMode kCarry) cuts
// every segment but the last into `cfold` carry segments, runs each from h = 0
// and records its end state and, per state, the sum of its base-2 decay
// exponents, so that it acts on an incoming state as h -> 2^xsum * h + h_end.
// The main pass (kMain, or kState when only checkpoints are wanted) folds the
// preceding carries into its starting state, in sequence order, and runs its
// segment.
//
// Data movement: the workgroup stages each chunk's inputs through LDS --
// delta and delta*u as fp32 rows per channel (converted once, read back by
// the lanes as 128-bit vectors) and the chunk's B/C rows -- double-buffered,
// with the next chunk's global loads issued before the current chunk is
// computed, so one barrier per chunk is the only synchronisation. Outputs go
// through an LDS tile and leave as coalesced row stores. Steps past L are
// padded with delta = u = 0, which leaves the state unchanged, so the inner
// loop carries no bounds checks. The [-88, 88] clamp of the exponent runs only
// in chunks where |delta|*max|A| can reach it (a wave-uniform test).
#include <atomic>
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


enum FwdMode { kMain = 0, kState = 1, kCarry = 2 };

// XF: the transforms of ScanXf compiled in (kXfDelta, kXfGate bits; the gate only with an output).
template <typename T, int NS, int SPL, int MODE, int XF>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(MODE == 2 ? carry_min_waves(NS, SPL) : fwd_min_waves(SPL), 8)))
ssm_fwd_kernel(const T* __restrict__ u, const T* __restrict__ delta, const T* __restrict__ A,
               const T* __restrict__ Bm, const T* __restrict__ Cm, const T* __restrict__ Dv,
               const T* __restrict__ h_prev, T* __restrict__ out, T* __restrict__ h_last, float* __restrict__ ckpt,
               float* __restrict__ car_h, float* __restrict__ car_x, int Bsz, int L, int D, int nck, int nblk_d,
               int nseg, int cps, int ncar, int cfold, ScanXf xf, T* __restrict__ out_z, int nfull) {
    constexpr bool HAS_OUT = MODE == kMain;
    constexpr bool CARRY = MODE == kCarry;
    constexpr int LPC = NS / SPL;  // lanes per channel
    constexpr int CPW = 64 / LPC;       // channels per wave
    constexpr int CPB = CPW * 4;        // channels per workgroup
    constexpr int TC = kCkptSteps;      // steps per chunk
    constexpr int RS = TC + 4;          // LDS row stride (floats) of a channel's steps
    constexpr int NSG = 256 / CPB;      // loader step groups
    constexpr int SPG = TC / NSG;       // steps per loader thread
    constexpr int YS = CPB + 4;         // LDS row stride of the output tile (16 mod 64 banks apart)
    constexpr int BCN = TC * NS;                       // B (and C) values per chunk
    constexpr int BCPT = BCN >= 256 ? BCN / 256 : 1;   // of them per loader thread
    static_assert(NSG * SPG == TC && (BCN < 256 || BCN % 256 == 0), "loader tiling");

    __shared__ __align__(16) float s_in[2][2][CPB][RS];  // [buf][delta, delta*u][channel][step]
    // B/C rows of the chunk: with C, each lane's SPL states of B then of C sit together
    // ([step][n / SPL][B x SPL, C x SPL]) so a lane reads both with one 2*SPL-float access
    __shared__ __align__(16) float s_bc[2][TC][HAS_OUT ? 2 * NS : NS];
    __shared__ __align__(16) float s_y[HAS_OUT ? 2 : 1][HAS_OUT ? TC : 1][HAS_OUT ? YS : 1];
    // per staging buffer: the index of the last chunk staged there whose exponents can reach the clamp
    __shared__ int s_flag[2];

    const int tid = threadIdx.x;
    const int lid = xcd_remap(blockIdx.x, gridDim.x);
    // (the carry pass: carry segment seg of cps chunks; the main pass: segment seg, or the whole row)
    const WorkItem wi = CARRY ? carry_item(lid, nblk_d * Bsz, nfull) : main_item(lid, nblk_d * Bsz, nfull, gridDim.x);
    const int seg = wi.seg;
    const int b = wi.row / nblk_d;
    const int d0 = (wi.row % nblk_d) * CPB;
    const int k0 = wi.whole ? 0 : seg * cps;
    const int k1 = wi.whole ? nck : min(nck, k0 + cps);

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
    const int64_t row0 = (int64_t)b * L;
    // carries of the ncar carry segments (cfold per main segment): car_[b][carry segment][d][n]
    const int64_t car0 = ((int64_t)b * ncar * D + d) * NS + n0;
    const int64_t car_seg = (int64_t)D * NS;

    float A2[SPL], h[SPL], xs[SPL];
#pragma unroll
    for (int j = 0; j < SPL; ++j) {
        A2[j] = ld(A + (int64_t)d * NS + n0 + j) * kLog2e;
        h[j] = (!CARRY && h_prev) ? ld(h_prev + ((int64_t)b * D + d) * NS + n0 + j) : 0.f;
        xs[j] = 0.f;  // carry: the clamped exponents' departure from A2 * sum(delta)
    }
    // max_n |A[ld_d][n]| * log2(e): the loader flags the chunks whose exponents can reach the clamp
    float lamax2 = 0.f;
#pragma unroll
    for (int n = 0; n < NS; ++n) lamax2 = __builtin_fmaxf(lamax2, __builtin_fabsf(ld(A + (int64_t)ld_d * NS + n)));
    lamax2 *= kLog2e;
    float sdt_l = 0.f;  // carry: the sum of the loader's delta values over the segment
    if constexpr (!CARRY) {
#pragma unroll 4
        for (int j = 0; j < seg * cfold; ++j) {  // h -> 2^xsum * h + h_end of each preceding carry segment
            float ch[SPL], cx[SPL];
            lds_ld<SPL>(car_h + car0 + j * car_seg, ch);
            lds_ld<SPL>(car_x + car0 + j * car_seg, cx);
#pragma unroll
            for (int q = 0; q < SPL; ++q) h[q] = __builtin_fmaf(__builtin_amdgcn_exp2f(cx[q]), h[q], ch[q]);
        }
    }
    // Chunk k's rows are read through buffer resources spanning exactly its min(16, L - 16k) rows:
    // rows past L and channels past D (offset kOob) read as 0, which is the padding the scan needs.
    const T* ub = u + row0 * D;
    const T* db = delta + row0 * D;
    const T* Bb = Bm + row0 * NS;
    const T* Cb = Cm + row0 * NS;
    const uint32_t lofs = lvalid ? ((uint32_t)(sg * SPG) * (uint32_t)D + (uint32_t)ld_d) * sizeof(T) : kOob;
    const uint32_t row_bytes = (uint32_t)D * sizeof(T);
    auto chunk_rows = [&](int k) { return (uint32_t)min(TC, L - k * TC); };
    // z is read only when the gated output is stored (the launcher sets kXfGate only with z and out_z)
    constexpr bool XD = (XF & kXfDelta) != 0, XG = HAS_OUT && (XF & kXfGate) != 0;
    const T* zb = XG ? static_cast<const T*>(xf.z) + row0 * D : nullptr;
    T pu[SPG], pd[SPG], pz[SPG], pb[BCPT], pc[BCPT];
    auto issue = [&](int k) {
        const int64_t ck = (int64_t)k * TC;
        const uint32_t rows = chunk_rows(k);
        const rsrc_t ru = make_rsrc(ub + ck * D, rows * row_bytes);
        const rsrc_t rd = make_rsrc(db + ck * D, rows * row_bytes);
#pragma unroll
        for (int s = 0; s < SPG; ++s) {
            pu[s] = buf_raw<T>(ru, lofs + s * row_bytes);
            pd[s] = buf_raw<T>(rd, lofs + s * row_bytes);
        }
        if constexpr (XG) {
            const rsrc_t rz = make_rsrc(zb + ck * D, rows * row_bytes);
#pragma unroll
            for (int s = 0; s < SPG; ++s) pz[s] = buf_raw<T>(rz, lofs + s * row_bytes);
        }
        const rsrc_t rb = make_rsrc(Bb + ck * NS, rows * NS * sizeof(T));
        const rsrc_t rc = make_rsrc(Cb + ck * NS, rows * NS * sizeof(T));
#pragma unroll
        for (int q = 0; q < BCPT; ++q) {  // value e = tid*BCPT + q of the chunk's (step, n) rows
            pb[q] = buf_raw<T>(rb, (tid * BCPT + q) * sizeof(T));
            if constexpr (HAS_OUT) pc[q] = buf_raw<T>(rc, (tid * BCPT + q) * sizeof(T));
        }
    };
    // D*u of the loader's (channel, steps) for the chunk being computed and the next one; the
    // loader thread also stores those outputs, so the consumer lanes never touch u
    const float Dl = HAS_OUT ? ld(Dv + ld_d) : 0.f;
    // delta' = softplus(delta + bias): applied once per element here; rows past L stay 0
    const float lbias = XD && xf.delta_bias ? ld(static_cast<const T*>(xf.delta_bias) + ld_d) : 0.f;
    float du_cur[SPG], du_nxt[SPG], gz_cur[SPG], gz_nxt[SPG];
    auto commit = [&](int k, int buf) {
        float vd[SPG], vdu[SPG];
        float vmax = 0.f;
#pragma unroll
        for (int s = 0; s < SPG; ++s) vd[s] = static_cast<float>(pd[s]);
        if constexpr (XD) {
#pragma unroll
            for (int s = 0; s < SPG; ++s) vd[s] += lbias;  // 0 without a bias
            if (xf.softplus) {
#pragma unroll
                for (int s = 0; s < SPG; ++s) vd[s] = softplus_f(vd[s]);
            }
            if ((k + 1) * TC > L) {  // the ragged last chunk: padded steps keep delta' = 0
#pragma unroll
                for (int s = 0; s < SPG; ++s)
                    if (k * TC + sg * SPG + s >= L) vd[s] = 0.f;
            }
        }
#pragma unroll
        for (int s = 0; s < SPG; ++s) {
            vmax = __builtin_fmaxf(vmax, __builtin_fabsf(vd[s]));
            if constexpr (CARRY) sdt_l += vd[s];
            const float vu = static_cast<float>(pu[s]);
            vdu[s] = vd[s] * vu;
            du_nxt[s] = Dl * vu;
            if constexpr (XG) {
                const float zv = static_cast<float>(pz[s]);
                gz_nxt[s] = zv * sigmoid_f(zv);  // silu(z)
            }
        }
        if (vmax * lamax2 > kExp2Clamp) s_flag[buf] = k;  // benign race: every writer stores k
        vst<SPG>(&s_in[buf][0][lc][sg * SPG], vd);
        vst<SPG>(&s_in[buf][1][lc][sg * SPG], vdu);
#pragma unroll
        for (int q = 0; q < BCPT; ++q) {
            const int e = tid * BCPT + q;
            if (BCN >= 256 || e < BCN) {
                const int n = e % NS;
                if constexpr (HAS_OUT) {
                    float* row = &s_bc[buf][e / NS][(n / SPL) * 2 * SPL + n % SPL];
                    row[0] = static_cast<float>(pb[q]);
                    row[SPL] = static_cast<float>(pc[q]);
                } else {
                    s_bc[buf][e / NS][n] = static_cast<float>(pb[q]);
                }
            }
        }
    };

    if (tid < 2) s_flag[tid] = -1;
    __syncthreads();
    if (k0 < k1) {  // every segment holds a chunk unless L == 0 (then h_last = h_prev)
        issue(k0);
        commit(k0, k0 & 1);
    }
    __syncthreads();
    float* ckb = (!CARRY && ckpt) ? ckpt + ((int64_t)b * nck * D + d) * NS + n0 : nullptr;
    T* ob = HAS_OUT && out != nullptr ? out + row0 * D : nullptr;

    ProgressPrio prio(k1 - k0);
    for (int k = k0; k < k1; ++k) {
        const int buf = k & 1;
        const bool more = k + 1 < k1;
        prio.update(k - k0);
#pragma unroll
        for (int s = 0; s < SPG; ++s) {
            du_cur[s] = du_nxt[s];
            if constexpr (XG) gz_cur[s] = gz_nxt[s];
        }
        if (more) issue(k + 1);
        if (ckb != nullptr && valid) vst<SPL>(ckb + (int64_t)k * D * NS, h);

        // the main pass at two states per lane reads the whole chunk's operands up front, so LDS
        // latency is paid once per chunk; the state-only passes read them four steps at a time, which
        // keeps them to few enough registers for twice the waves per SIMD (their chunks are short on
        // arithmetic, so more waves in flight are what covers the loads)
        float dt[TC], dtu[TC], Bv[TC][SPL], Cv[TC][SPL];
        auto read_steps = [&](int i0, int n) {
#pragma unroll
            for (int i4 = i0; i4 < i0 + n; i4 += 4) {
                float t4[4], u4[4];
                lds_ld<4>(&s_in[buf][0][c][i4], t4);
                lds_ld<4>(&s_in[buf][1][c][i4], u4);
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    dt[i4 + q] = t4[q];
                    dtu[i4 + q] = u4[q];
                }
            }
#pragma unroll
            for (int i = i0; i < i0 + n; ++i) {
                if constexpr (HAS_OUT) {
                    float bc[2 * SPL];
                    lds_ld<2 * SPL>(&s_bc[buf][i][2 * n0], bc);
#pragma unroll
                    for (int j = 0; j < SPL; ++j) {
                        Bv[i][j] = bc[j];
                        Cv[i][j] = bc[SPL + j];
                    }
                } else {
                    lds_ld<SPL>(&s_bc[buf][i][n0], Bv[i]);
                }
            }
        };
        // the main pass reads in groups as well at one state per lane (it runs many waves per SIMD
        // too) and at four (reading the chunk up front would hold 160 VGPRs of operands: one wave per
        // SIMD instead of three, and twice the time per call at N=64)
        constexpr bool GROUPED = !HAS_OUT || SPL != 2;
        if constexpr (!GROUPED) read_steps(0, TC);
        // one workgroup-uniform decision per chunk: the loaders flag a chunk in which some |delta*A|
        // can exceed 88; the clamped path gives the same values whenever none does, so deciding for the
        // whole workgroup is exact
        const bool need_clamp = __builtin_amdgcn_readfirstlane(s_flag[buf]) == k;
        // the lane partials of y are reduce-scattered over the group every RV steps; the lane writes
        // the step's y the scatter leaves it (each step is held by two lanes of the group)
        constexpr int RV = LPC / 2;
        float ry[RV];
        float* const y_mine = &s_y[HAS_OUT ? buf : 0][HAS_OUT ? rs_index<LPC, RV>(lane) : 0][HAS_OUT ? c : 0];
        auto run = [&](auto clamp_tag) {
            constexpr bool CLAMP = decltype(clamp_tag)::value;
#pragma unroll
            for (int i = 0; i < TC; ++i) {
                if constexpr (GROUPED) {
                    if (i % 4 == 0) read_steps(i, 4);
                }
                float y = 0.f;
#pragma unroll
                for (int j = 0; j < SPL; ++j) {
                    float x = dt[i] * A2[j];
                    if constexpr (CLAMP) {
                        const float xc = __builtin_fminf(__builtin_fmaxf(x, -kExp2Clamp), kExp2Clamp);
                        if constexpr (CARRY) xs[j] += xc - x;  // the clamp's share of the exponent sum
                        x = xc;
                    }
                    h[j] = __builtin_fmaf(__builtin_amdgcn_exp2f(x), h[j], dtu[i] * Bv[i][j]);
                    if constexpr (HAS_OUT) y = __builtin_fmaf(Cv[i][j], h[j], y);
                }
                if constexpr (HAS_OUT) {
                    ry[i % RV] = y;
                    if (i % RV == RV - 1) y_mine[(i - (RV - 1)) * YS] = reduce_scatter<LPC, RV>(ry, lane);
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
            // the loader's (channel, steps) outputs: y from the tile plus D*u
            const uint32_t obytes = chunk_rows(k) * row_bytes;
            const rsrc_t ro = make_rsrc(ob + (int64_t)k * TC * D, ob != nullptr ? obytes : 0);
            const rsrc_t rz = make_rsrc(out_z + row0 * D + (int64_t)k * TC * D, XG ? obytes : 0);
#pragma unroll
            for (int s = 0; s < SPG; ++s) {
                const float y = s_y[buf][sg * SPG + s][lc] + du_cur[s];
                buf_st<T>(ro, lofs + s * row_bytes, y);  // size 0 when out is not wanted: dropped
                if constexpr (XG) buf_st<T>(rz, lofs + s * row_bytes, y * gz_cur[s]);
            }
        }
    }
    if constexpr (CARRY) {
        // summed exponent of each state: A2 * (the channel's delta summed by its NSG loader threads),
        // plus the clamp's share
        float* red = &s_in[0][0][0][0];  // free after the chunk loop; NSG*CPB = 256 floats
        red[sg * CPB + lc] = sdt_l;
        __syncthreads();
        float sdt = 0.f;
        for (int q = 0; q < NSG; ++q) sdt += red[q * CPB + c];
#pragma unroll
        for (int j = 0; j < SPL; ++j) xs[j] = __builtin_fmaf(A2[j], sdt, xs[j]);
        if (valid) {
            vst<SPL>(car_h + car0 + seg * car_seg, h);
            vst<SPL>(car_x + car0 + seg * car_seg, xs);
        }
    } else if (h_last != nullptr && valid && k1 == nck) {  // the row's last segment
#pragma unroll
        for (int j = 0; j < SPL; ++j) st(h_last + ((int64_t)b * D + d) * NS + n0 + j, h[j]);
    }
}

template <typename T, int NS, int SPL, int MODE, int XF>
static void fwd_launch(const FwdArgs& a, const SsmShape& s, int nseg_launched, hipStream_t st) {
    constexpr int CPB = 4 * 64 / (NS / SPL);
    const int nblk_d = (int)((s.dim + CPB - 1) / CPB);
    const int nck = (int)((s.seqlen + kCkptSteps - 1) / kCkptSteps);
    // a partly split plan launches its whole rows once and its split rows once per segment (carry pass: once
    // per carry segment)
    const int rows = nblk_d * (int)s.batch, split = a.nfull > 0 ? rows - a.nfull : rows;
    const int grid = MODE == kCarry ? split * nseg_launched : (a.nfull > 0 ? a.nfull : 0) + split * nseg_launched;
    hipLaunchKernelGGL((ssm_fwd_kernel<T, NS, SPL, MODE, XF>), dim3(grid), dim3(256), 0, st, (const T*)a.u,
                       (const T*)a.delta, (const T*)a.A, (const T*)a.B, (const T*)a.C, (const T*)a.Dv,
                       (const T*)a.h_prev, (T*)a.out, (T*)a.h_last, a.ckpt, a.car_h, a.car_x, (int)s.batch,
                       (int)s.seqlen, (int)s.dim, nck, nblk_d, a.nseg, MODE == kCarry ? a.cps / a.cfold : a.cps,
                       a.ncar, a.cfold, a.xf, (T*)a.out_z, a.nfull);
}

template <typename T, int NS, int SPL, int XF>
static hipError_t fwd_inst(const FwdArgs& a, const SsmShape& s, hipStream_t st) {
    // the state-only passes see only the delta transform
    if (a.nseg > 1) fwd_launch<T, NS, SPL, kCarry, XF & kXfDelta>(a, s, a.ncar, st);  // carries of all chunks before the last segment
    if (a.out != nullptr || a.out_z != nullptr)
        fwd_launch<T, NS, SPL, kMain, XF>(a, s, a.nseg, st);
    else
        fwd_launch<T, NS, SPL, kState, XF & kXfDelta>(a, s, a.nseg, st);
    return hipGetLastError();
}

template <typename T, int NS, int SPL>
static hipError_t fwd_inst(const FwdArgs& a, const SsmShape& s, hipStream_t st) {
    // the gate applies only to the gated output (z without out_z is unused)
    const int xf = (a.xf.delta_bias != nullptr || a.xf.softplus ? kXfDelta : 0) |
                   (a.xf.z != nullptr && a.out_z != nullptr ? kXfGate : 0);
    switch (xf) {
        case 0: return fwd_inst<T, NS, SPL, 0>(a, s, st);
        case kXfDelta: return fwd_inst<T, NS, SPL, kXfDelta>(a, s, st);
        case kXfGate: return fwd_inst<T, NS, SPL, kXfGate>(a, s, st);
        default: return fwd_inst<T, NS, SPL, kXfDelta | kXfGate>(a, s, st);
    }
}

int fwd_wgs_per_cu(int ns, int spl, int mode) {
    // the runtime's occupancy of the fp16, transform-free instance (registers and LDS differ little
    // across dtypes and transforms), queried once per (N, SPL, mode); 0 when it cannot be queried
    static std::atomic<int> cache[4][3][3];
    const int ni = ns == 8 ? 0 : ns == 16 ? 1 : ns == 32 ? 2 : 3, si = spl == 1 ? 0 : spl == 2 ? 1 : 2;
    int v = cache[ni][si][mode].load(std::memory_order_relaxed);
    if (v != 0) return v < 0 ? 0 : v;
    const void* k = nullptr;
#define MWC_FWD_K(N, S)                                                                                         \
    if (ns == N && spl == S)                                                                                    \
        k = mode == kCarry   ? reinterpret_cast<const void*>(&ssm_fwd_kernel<half_t, N, S, kCarry, 0>)        \
            : mode == kState ? reinterpret_cast<const void*>(&ssm_fwd_kernel<half_t, N, S, kState, 0>)        \
                             : reinterpret_cast<const void*>(&ssm_fwd_kernel<half_t, N, S, kMain, 0>);
    MWC_FOR_EACH_LANE_GROUP(MWC_FWD_K)
#undef MWC_FWD_K
    int n = 0;
    if (k == nullptr || hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, k, 256, 0) != hipSuccess || n <= 0) {
        (void)hipGetLastError();
        n = -1;
    }
    cache[ni][si][mode].store(n, std::memory_order_relaxed);
    return n < 0 ? 0 : n;
}

hipError_t launch_ssm_fwd(int dt, int ns, int spl, const FwdArgs& a, const SsmShape& s, hipStream_t st) {
#define MWC_FWD(N, S) \
    if (ns == N && spl == S) MWC_DISPATCH_DTYPE(dt, TT, return fwd_inst<TT, N, S>(a, s, st));
    MWC_FOR_EACH_LANE_GROUP(MWC_FWD)
#undef MWC_FWD
    return hipErrorInvalidValue;
}

}  // namespace mwc
