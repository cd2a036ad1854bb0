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
// Mapping: lane groups as in the forward (LPC lanes x SPL states per channel, 4
// waves = CPB channels of one batch row per workgroup), but with the channel in
// the low lane bits and the state group in the high ones. The sequence is walked
// in reverse in chunks of 16 steps; each chunk restarts from the fp32
// checkpoint the forward stored, recomputes the chunk's states and decay
// factors into VGPRs (one exp per state) and runs the reverse sweep. Inputs
// are staged through LDS as in the forward (fp32 delta, delta*u, dout rows
// per channel; B/C rows per step); the previous chunk's global loads are in
// flight during the sweep and land in LDS between the chunk's two barriers.
// Sums over n (S1 = sum g*B and S2 = sum g*A*dA*h_{t-1}) are DPP reduce-scatters
// inside the lane group; the storing threads finish du = D*dout + delta*S1 and
// ddelta = S2 + u*S1 once per element. Sums over
// channels (dB, dC) go through a wave-private LDS slab: each step a lane weights
// g_t by delta*u and h_t by dout, adds its channel partner's weighted values
// with one reduce-scatter level (keeping one of the two) and deposits the
// result; every 4 steps the wave folds the deposited channel-pair columns. Once
// per chunk the workgroup's waves are added and written as a per-group fp32
// partial, which a second small kernel sums in fixed order (deterministic, no
// atomics). dA and dD accumulate in registers
// over t and are summed over the segments and b by the finishing kernel.
//
// Parallelism over L: as in the forward, L is cut into segments of whole
// chunks. The adjoint entering a segment from its right is linear in the
// adjoint leaving the last step: g_in(s) = 2^xsum(s+1) * g_in(s+1) + G(s+1),
// where G(j) is segment j's reverse sweep of g -> dA_t*(g + dout_t*C_t) from
// g = 0 and xsum(j) the sum of its base-2 decay exponents. A carry kernel
// computes (G, xsum) for every segment but the first, each cut into cfold
// carry segments; the main kernel folds them, from dh_last, into its starting
// adjoint.
#include <atomic>
#include <type_traits>

#include "common.h"
#include "launch.h"

namespace mwc {

namespace {

constexpr int kRedSlots = 4;  // steps folded per in-wave LDS reduction

template <int K>
__device__ __forceinline__ void ldv(const float* p, float (&v)[K]) {
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

// Orders this wave's LDS traffic for the compiler; one wave's LDS operations
// are executed in issue order by the hardware.
__device__ __forceinline__ void wave_lds_fence() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

}  // namespace

// Adjoint carries of the chunks after the first segment, cut into ncar carry
// segments of cps chunks (carry segment j starts at chunk first + j*cps):
// car_g = the reverse sweep of g -> dA_t * (g + dout_t * C_t) over the carry
// segment from g = 0, car_x = its summed base-2 decay exponents (so it maps an
// adjoint g arriving from its right to 2^car_x * g + car_g).
template <typename T, int NS, int SPL, int XF>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(carry_min_waves(NS, SPL), 8)))
ssm_bwd_carry_kernel(const T* __restrict__ delta, const T* __restrict__ A, const T* __restrict__ Cm,
                     const T* __restrict__ dout, float* __restrict__ car_g, float* __restrict__ car_x, int Bsz,
                     int L, int D, int nck, int nblk_d, int ncar, int first, int cps, ScanXf xf, int nfull) {
    constexpr int LPC = NS / SPL;
    constexpr int CPW = 64 / LPC;
    constexpr int CPB = CPW * 4;
    constexpr int TC = kCkptSteps;
    constexpr int RS = TC + 4;
    constexpr int NSG = 256 / CPB;
    constexpr int SPG = TC / NSG;
    constexpr int BCN = TC * NS;                       // C values per chunk
    constexpr int BCPT = BCN >= 256 ? BCN / 256 : 1;   // of them per loader thread
    static_assert(NSG * SPG == TC && (BCN < 256 || BCN % 256 == 0), "tiling");

    __shared__ __align__(16) float s_in[2][2][CPB][RS];  // [buf][delta, dout][channel][step]
    __shared__ __align__(16) float s_c[2][TC][NS];
    // per staging buffer: the index of the last chunk staged there whose exponents can reach the clamp
    // ([2], [3]: sinks for the loaders' writes of the chunks that cannot)
    __shared__ int s_flag[4];

    const int tid = threadIdx.x;
    const int lid = xcd_remap(blockIdx.x, gridDim.x);
    const WorkItem wi = carry_item(lid, nblk_d * Bsz, nfull);  // carry segment wi.seg of a split row
    const int seg = wi.seg;
    const int b = wi.row / nblk_d;
    const int d0 = (wi.row % nblk_d) * CPB;
    const int k0 = first + seg * cps;
    const int k1 = min(nck, k0 + cps);

    const int wave = tid >> 6, lane = tid & 63;
    const int c = wave * CPW + lane / LPC;
    const int n0 = (lane % LPC) * SPL;
    const bool valid = d0 + c < D;
    const int d = valid ? d0 + c : D - 1;
    const int lc = tid % CPB, sg = tid / CPB;
    const bool lvalid = d0 + lc < D;
    const int ld_d = lvalid ? d0 + lc : D - 1;
    const int64_t row0 = (int64_t)b * L;

    float A2[SPL], gc[SPL], xs[SPL];
#pragma unroll
    for (int j = 0; j < SPL; ++j) {
        A2[j] = ld(A + (int64_t)d * NS + n0 + j) * kLog2e;
        gc[j] = 0.f;
        xs[j] = 0.f;  // the clamped exponents' departure from A2 * sum(delta)
    }
    float lamax2 = 0.f;  // max_n |A[ld_d][n]| * log2(e): the loader flags chunks that reach the clamp
#pragma unroll
    for (int n = 0; n < NS; ++n) lamax2 = __builtin_fmaxf(lamax2, __builtin_fabsf(ld(A + (int64_t)ld_d * NS + n)));
    lamax2 *= kLog2e;
    float sdt_l = 0.f;  // the sum of the loader's delta values over the carry segment

    // buffer resources per chunk: rows past L and channels past D read as 0 (see the main kernel)
    const uint32_t lofs = lvalid ? ((uint32_t)(sg * SPG) * (uint32_t)D + (uint32_t)ld_d) * sizeof(T) : kOob;
    const uint32_t row_bytes = (uint32_t)D * sizeof(T);
    constexpr bool XD = (XF & kXfDelta) != 0, XG = (XF & kXfGate) != 0;
    const T* zb = XG ? static_cast<const T*>(xf.z) : nullptr;
    const float lbias = XD && xf.delta_bias ? ld(static_cast<const T*>(xf.delta_bias) + ld_d) : 0.f;
    T pd[SPG], py[SPG], pz[SPG], pc[BCPT];
    auto issue = [&](int k) {
        const int64_t ck = (int64_t)k * TC;
        const uint32_t rows = (uint32_t)min(TC, L - k * TC);
        const rsrc_t rd = make_rsrc(delta + (row0 + ck) * D, rows * row_bytes);
        const rsrc_t ry = make_rsrc(dout + (row0 + ck) * D, rows * row_bytes);
#pragma unroll
        for (int s = 0; s < SPG; ++s) {
            pd[s] = buf_raw<T>(rd, lofs + s * row_bytes);
            py[s] = buf_raw<T>(ry, lofs + s * row_bytes);
        }
        if constexpr (XG) {
            const rsrc_t rz = make_rsrc(zb + (row0 + ck) * D, rows * row_bytes);
#pragma unroll
            for (int s = 0; s < SPG; ++s) pz[s] = buf_raw<T>(rz, lofs + s * row_bytes);
        }
        const rsrc_t rc = make_rsrc(Cm + (row0 + ck) * NS, rows * NS * sizeof(T));
#pragma unroll
        for (int q = 0; q < BCPT; ++q) pc[q] = buf_raw<T>(rc, (tid * BCPT + q) * sizeof(T));
    };
    auto commit = [&](int k, int buf) {
        float vd[SPG], vy[SPG];
        float vmax = 0.f;
#pragma unroll
        for (int s = 0; s < SPG; ++s) {
            vd[s] = static_cast<float>(pd[s]);
            vy[s] = static_cast<float>(py[s]);
            if constexpr (XG) {  // the scan sees dout * silu(z)
                const float zv = static_cast<float>(pz[s]);
                vy[s] *= zv * sigmoid_f(zv);
            }
        }
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
            sdt_l += vd[s];
        }
        s_flag[vmax * lamax2 > kExp2Clamp ? buf : 2 + buf] = k;  // branch-free: flag word or sink, all store k
        stv<SPG>(&s_in[buf][0][lc][sg * SPG], vd);
        stv<SPG>(&s_in[buf][1][lc][sg * SPG], vy);
#pragma unroll
        for (int q = 0; q < BCPT; ++q) {
            const int e = tid * BCPT + q;
            if (BCN >= 256 || e < BCN) s_c[buf][e / NS][e % NS] = static_cast<float>(pc[q]);
        }
    };

    if (tid < 2) s_flag[tid] = -1;
    __syncthreads();
    if (k0 < k1) {
        issue(k1 - 1);
        commit(k1 - 1, (k1 - 1) & 1);
    }
    __syncthreads();
    ProgressPrio prio(k1 - k0);
    for (int k = k1 - 1; k >= k0; --k) {
        const int buf = k & 1;
        const bool more = k > k0;
        prio.update(k1 - 1 - k);
        if (more) issue(k - 1);
        // operands are read four steps at a time, which keeps the pass to few enough registers for
        // twice the waves per SIMD (its chunks are short on arithmetic, so more waves in flight are
        // what covers the loads)
        float dt[TC], yo[TC], Cv[TC][SPL];
        auto read_steps = [&](int i0) {
            float t4[4], y4[4];
            ldv<4>(&s_in[buf][0][c][i0], t4);
            ldv<4>(&s_in[buf][1][c][i0], y4);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                dt[i0 + q] = t4[q];
                yo[i0 + q] = y4[q];
                ldv<SPL>(&s_c[buf][i0 + q][n0], Cv[i0 + q]);
            }
        };
        // one workgroup-uniform decision per chunk (exact: see the main kernel)
        const bool need_clamp = __builtin_amdgcn_readfirstlane(s_flag[buf]) == k;
        auto run = [&](auto clamp_tag) {
            constexpr bool CLAMP = decltype(clamp_tag)::value;
#pragma unroll
            for (int i = TC - 1; i >= 0; --i) {
                if (i % 4 == 3) read_steps(i - 3);
#pragma unroll
                for (int j = 0; j < SPL; ++j) {
                    float x = dt[i] * A2[j];
                    if constexpr (CLAMP) {
                        const float xc = __builtin_fminf(__builtin_fmaxf(x, -kExp2Clamp), kExp2Clamp);
                        xs[j] += xc - x;  // the clamp's share of the exponent sum
                        x = xc;
                    }
                    gc[j] = __builtin_amdgcn_exp2f(x) * __builtin_fmaf(yo[i], Cv[i][j], gc[j]);
                }
            }
        };
        if (need_clamp)
            run(std::true_type{});
        else
            run(std::false_type{});
        if (more) commit(k - 1, buf ^ 1);
        __syncthreads();
    }
    {  // summed exponent: A2 * (the channel's delta summed by its NSG loader threads), plus the clamp's share
        float* red = &s_in[0][0][0][0];  // free after the chunk loop; NSG*CPB = 256 floats
        red[sg * CPB + lc] = sdt_l;
        __syncthreads();
        float sdt = 0.f;
        for (int q = 0; q < NSG; ++q) sdt += red[q * CPB + c];
#pragma unroll
        for (int j = 0; j < SPL; ++j) xs[j] = __builtin_fmaf(A2[j], sdt, xs[j]);
    }
    if (valid) {
        const int64_t o = (((int64_t)b * ncar + seg) * D + d) * NS + n0;
        stv<SPL>(car_g + o, gc);
        stv<SPL>(car_x + o, xs);
    }
}

// XF: the transforms of ScanXf compiled in (kXfDelta, kXfGate bits).
template <typename T, int NS, int SPL, int XF>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(bwd_min_waves(NS, SPL), 8)))
ssm_bwd_kernel(
    const T* __restrict__ u, const T* __restrict__ delta, const T* __restrict__ A, const T* __restrict__ Bm,
    const T* __restrict__ Cm, const T* __restrict__ Dv, const T* __restrict__ dout, const T* __restrict__ dh_last,
    const float* __restrict__ ckpt, T* __restrict__ du, T* __restrict__ ddelta, T* __restrict__ dh_prev,
    float* __restrict__ dA_part, float* __restrict__ dD_part, float* __restrict__ dbc_part,
    const float* __restrict__ car_g, const float* __restrict__ car_x, int Bsz, int L, int D, int nck, int nblk_d,
    int nseg, int cps, int ncar, int cfold, ScanXf xf, const T* __restrict__ yb_out, T* __restrict__ dz,
    float* __restrict__ dbias_part, int nfull) {
    constexpr int LPC = NS / SPL;
    constexpr int CPW = 64 / LPC;
    constexpr int CPB = CPW * 4;
    constexpr int TC = kCkptSteps;
    constexpr int RS = TC + 4;
    constexpr int NSG = 256 / CPB;
    constexpr int SPG = TC / NSG;
    constexpr int OS = CPB + 4;
    constexpr int BCN = TC * NS;                       // B (and C) values per chunk
    constexpr int BCPT = BCN >= 256 ? BCN / 256 : 1;   // of them per loader thread
    // dB/dC over the wave's channels: each step a lane weights g_t (by delta*u) and h_t (by dout) in
    // registers and adds its channel partner's (the lane 2^PB away: channels c and c ^ CPW/2) with one
    // reduce-scatter level, keeping the g sums on one side and the h sums on the other, and deposits
    // that one vector. Every 4-step phase the 16 lanes of a slot each take one (plane, block of VB =
    // NS/8 states) row and add its CPW/2 channel-pair columns, so no lane pair combines partial sums
    // and the fold needs no weights.
    constexpr int VB = NS / 8;
    constexpr int PB = CPW >= 16 ? 3 : CPW >= 8 ? 2 : 1;  // lane bit of the channel partner (top channel bit)
    constexpr int NPC = CPW / 2;                           // channel-pair columns per row
    static_assert(NSG * SPG == TC && (BCN < 256 || BCN % 256 == 0) && VB >= 1, "tiling");

    // [delta, delta*u, dout] planes of [channel][step]; planes are AS floats apart
    // (AS = 16 mod 64 banks) so the delta*u and dout weights of one channel sit in different banks
    constexpr int AS = CPB * RS + 16;
    __shared__ __align__(16) float s_in_raw[3 * AS];
    // B/C rows of the chunk, [step][n / SPL][B x SPL, C x SPL]: a lane reads its B and C with one access
    __shared__ __align__(16) float s_bc[TC][2 * NS];
    // wave-private slabs of the weighted channel-pair sums of g_t (plane 0) and h_t (plane 1):
    // [wave][plane][slot][state block][channel pair][VB], a (slot, block) row holding the block's VB
    // states for every channel pair. Rows are packed and plane 1 starts 16 floats past a multiple of 64:
    // measured on gfx950 (N=16, 8 lanes per channel: rows of 8 floats), the deposits (ds_write_b64, the
    // two planes' lanes interleaved) are then conflict-free, and so are the fold's two ds_read_b128 of a
    // row when plane 1's lanes read the row's halves in swapped order (see the fold)
    constexpr int RW = NPC * VB;
    constexpr int PL = kRedSlots * 8 * RW + 16;
    __shared__ __align__(16) float s_red[4][2 * PL];
    auto s_in = [&](int plane, int ch) -> float* { return &s_in_raw[plane * AS + ch * RS]; };
    __shared__ __align__(16) float s_part[4][TC][2 * NS];
    __shared__ __align__(16) float s_out[2][TC][OS];  // [du, ddelta][step][channel]
    __shared__ int s_flag[2];  // [0]: index of the last staged chunk that needs the exponent clamp; [1]: sink

    const int tid = threadIdx.x;
    const int lid = xcd_remap(blockIdx.x, gridDim.x);
    const WorkItem wi = main_item(lid, nblk_d * Bsz, nfull, gridDim.x);  // segment wi.seg, or the whole row
    const int seg = wi.seg;
    const int b = wi.row / nblk_d;
    const int blk = wi.row % nblk_d;
    const int d0 = blk * CPB;
    const int k0 = wi.whole ? 0 : seg * cps;
    const int k1 = wi.whole ? nck : min(nck, k0 + cps);

    const int wave = tid >> 6, lane = tid & 63;
    // a wave's CPW channels take the low lane bits (channel lane % CPW, state group lane / CPW), so a
    // channel's lanes differ in the high bits the reduce-scatter exchanges cheaply
    const int cw = lane % CPW;  // channel within the wave
    const int c = wave * CPW + cw;
    const int g = lane / CPW;
    const int n0 = g * SPL;
    const bool valid = d0 + c < D;
    const int d = valid ? d0 + c : D - 1;

    const int lc = tid % CPB, sg = tid / CPB;
    const bool lvalid = d0 + lc < D;
    const int ld_d = lvalid ? d0 + lc : D - 1;
    const int64_t row0 = (int64_t)b * L;

    // folding roles: slot rs (step i+rs), plane rpl (0: dB from g, 1: dC from h), state block rb; with
    // rows of two 16-byte halves, plane 1's lanes read them in swapped order
    const int rs = lane >> 4, rpl = (lane >> 3) & 1, rb = lane & 7;
    constexpr bool kFoldRot = NPC * VB == 8;
    // depositing role: plane (the g sums on lanes whose bit PB is 0) and channel-pair column
    const int dpl = (lane >> PB) & 1;
    const int cwp = (cw & ((1 << PB) - 1)) | ((cw >> (PB + 1)) << PB);

    float A2[SPL], An[SPL], gc[SPL], dAacc[SPL];
#pragma unroll
    for (int j = 0; j < SPL; ++j) {
        An[j] = ld(A + (int64_t)d * NS + n0 + j);
        A2[j] = An[j] * kLog2e;
        gc[j] = dh_last != nullptr ? ld(dh_last + ((int64_t)b * D + d) * NS + n0 + j) : 0.f;
        dAacc[j] = 0.f;
    }
#pragma unroll 4
    for (int j = ncar - 1; j >= (wi.whole ? ncar : seg * cfold); --j) {  // g -> 2^xsum * g + G of each following carry segment
        const int64_t o = (((int64_t)b * ncar + j) * D + d) * NS + n0;
        float cg[SPL], cx[SPL];
        ldv<SPL>(car_g + o, cg);
        ldv<SPL>(car_x + o, cx);
#pragma unroll
        for (int q = 0; q < SPL; ++q) gc[q] = __builtin_fmaf(__builtin_amdgcn_exp2f(cx[q]), gc[q], cg[q]);
    }
    const float* ckb = ckpt + ((int64_t)b * nck * D + d) * NS + n0;

    // Chunk k's rows are read through buffer resources spanning exactly its min(16, L - 16k) rows:
    // rows past L and channels past D (offset kOob) read as 0 and their stores are dropped.
    const uint32_t lofs = lvalid ? ((uint32_t)(sg * SPG) * (uint32_t)D + (uint32_t)ld_d) * sizeof(T) : kOob;
    const uint32_t row_bytes = (uint32_t)D * sizeof(T);
    auto chunk_rows = [&](int k) { return (uint32_t)min(TC, L - k * TC); };
    const int64_t rowD = row0 * D;
    constexpr bool XD = (XF & kXfDelta) != 0, XG = (XF & kXfGate) != 0;
    const T* zb = XG ? static_cast<const T*>(xf.z) : nullptr;
    T pu[SPG], pd[SPG], py[SPG], pz[SPG], pyo[SPG], pb[BCPT], pc[BCPT];
    float hnext[SPL];
    auto issue = [&](int k) {
        const int64_t ck = (int64_t)k * TC;
        const uint32_t rows = chunk_rows(k);
        const rsrc_t ru = make_rsrc(u + rowD + ck * D, rows * row_bytes);
        const rsrc_t rd = make_rsrc(delta + rowD + ck * D, rows * row_bytes);
        const rsrc_t ry = make_rsrc(dout + rowD + ck * D, rows * row_bytes);
#pragma unroll
        for (int s = 0; s < SPG; ++s) {
            pu[s] = buf_raw<T>(ru, lofs + s * row_bytes);
            pd[s] = buf_raw<T>(rd, lofs + s * row_bytes);
            py[s] = buf_raw<T>(ry, lofs + s * row_bytes);
        }
        if constexpr (XG) {  // z and the ungated output, for dout * silu(z) and dz
            const rsrc_t rz = make_rsrc(zb + rowD + ck * D, rows * row_bytes);
            const rsrc_t ro = make_rsrc(yb_out + rowD + ck * D, rows * row_bytes);
#pragma unroll
            for (int s = 0; s < SPG; ++s) {
                pz[s] = buf_raw<T>(rz, lofs + s * row_bytes);
                pyo[s] = buf_raw<T>(ro, lofs + s * row_bytes);
            }
        }
        const uint32_t bc_bytes = rows * NS * sizeof(T);
        const rsrc_t rb = make_rsrc(Bm + (row0 + ck) * NS, bc_bytes);
        const rsrc_t rc = make_rsrc(Cm + (row0 + ck) * NS, bc_bytes);
#pragma unroll
        for (int q = 0; q < BCPT; ++q) {  // value e = tid*BCPT + q of the chunk's (step, n) rows
            pb[q] = buf_raw<T>(rb, (tid * BCPT + q) * sizeof(T));
            pc[q] = buf_raw<T>(rc, (tid * BCPT + q) * sizeof(T));
        }
        ldv<SPL>(ckb + (int64_t)k * D * NS, hnext);
    };
    float lamax2 = 0.f;  // max_n |A[ld_d][n]| * log2(e): the loader flags chunks that reach the clamp
#pragma unroll
    for (int n = 0; n < NS; ++n) lamax2 = __builtin_fmaxf(lamax2, __builtin_fabsf(ld(A + (int64_t)ld_d * NS + n)));
    lamax2 *= kLog2e;
    const float lbias = XD && xf.delta_bias ? ld(static_cast<const T*>(xf.delta_bias) + ld_d) : 0.f;
    // d delta' / d delta (softplus) of the loader's elements, for the chunk being stored and the next
    float dd_cur[XD ? SPG : 1], dd_nxt[XD ? SPG : 1];
    float dbias_acc = 0.f;
    // the loader's (channel, steps) elements of the chunk being stored and of the next one: delta and
    // dout (as the scan sees them), for du = D*dout + delta*sum_n g*B; dD accumulates here, once per
    // element
    const float Dl = ld(Dv + ld_d);
    float d_cur[SPG], d_nxt[SPG], y_cur[SPG], y_nxt[SPG], u_cur[SPG], u_nxt[SPG];
    float dDl = 0.f;
    auto commit = [&](int k) {
        float vd[SPG], vdu[SPG], vu[SPG], vy[SPG];
        float vmax = 0.f;
        [[maybe_unused]] float vdz[SPG];
#pragma unroll
        for (int s = 0; s < SPG; ++s) {
            vd[s] = static_cast<float>(pd[s]);
            vu[s] = static_cast<float>(pu[s]);
            vy[s] = static_cast<float>(py[s]);
            if constexpr (XG) {  // out_z = out * silu(z): the scan sees dout * silu(z)
                const float zv = static_cast<float>(pz[s]);
                const float sz = sigmoid_f(zv);
                const float a = vy[s] * sz;
                // silu'(z) = sigmoid(z) * (1 + z * (1 - sigmoid(z)))
                vdz[s] = a * static_cast<float>(pyo[s]) * __builtin_fmaf(zv, 1.f - sz, 1.f);
                vy[s] = a * zv;
            }
        }
        if constexpr (XD) {
#pragma unroll
            for (int s = 0; s < SPG; ++s) {
                vd[s] += lbias;  // 0 without a bias
                dd_nxt[s] = 1.f;
            }
            if (xf.softplus) {
#pragma unroll
                for (int s = 0; s < SPG; ++s) vd[s] = softplus_grad_f(vd[s], dd_nxt[s]);
            }
            if ((k + 1) * TC > L) {  // the ragged last chunk: padded steps keep delta' = 0
#pragma unroll
                for (int s = 0; s < SPG; ++s)
                    if (k * TC + sg * SPG + s >= L) vd[s] = 0.f;
            }
        }
#pragma unroll
        for (int s = 0; s < SPG; ++s) {
            vdu[s] = vd[s] * vu[s];
            vmax = __builtin_fmaxf(vmax, __builtin_fabsf(vd[s]));
            d_nxt[s] = vd[s];
            y_nxt[s] = vy[s];
            u_nxt[s] = vu[s];
            dDl = __builtin_fmaf(vy[s], vu[s], dDl);  // rows past L read as 0
        }
        if constexpr (XG) {  // dz = dout * out * silu'(z) needs no scan: store it now
            const rsrc_t rdz = make_rsrc(dz + rowD + (int64_t)k * TC * D, chunk_rows(k) * row_bytes);
#pragma unroll
            for (int s = 0; s < SPG; ++s) buf_st<T>(rdz, lofs + s * row_bytes, vdz[s]);
        }
        s_flag[vmax * lamax2 > kExp2Clamp ? 0 : 1] = k;  // branch-free: flag word or sink, all store k
        stv<SPG>((s_in(0, lc) + sg * SPG), vd);
        stv<SPG>((s_in(1, lc) + sg * SPG), vdu);
        stv<SPG>((s_in(2, lc) + sg * SPG), vy);
#pragma unroll
        for (int q = 0; q < BCPT; ++q) {
            const int e = tid * BCPT + q;
            if (BCN >= 256 || e < BCN) {
                const int n = e % NS;
                float* row = &s_bc[e / NS][(n / SPL) * 2 * SPL + n % SPL];
                row[0] = static_cast<float>(pb[q]);
                row[SPL] = static_cast<float>(pc[q]);
            }
        }
    };

    float hin[SPL];
    if (tid == 0) s_flag[0] = -1;
    __syncthreads();
    if (k0 < k1) {  // L == 0 has no chunk; the outputs below are then dh_prev = dh_last and zero partials
        issue(k1 - 1);
        commit(k1 - 1);
#pragma unroll
        for (int j = 0; j < SPL; ++j) hin[j] = hnext[j];
    }
    __syncthreads();

    float* red_g = &s_red[wave][0];   // [slot][state block][channel][VB]
    float* red_h = &s_red[wave][PL];

    ProgressPrio prio(k1 - k0);
    for (int k = k1 - 1; k >= k0; --k) {
        const int t0 = k * TC;
        const bool more = k > k0;
        prio.update(k1 - 1 - k);
#pragma unroll
        for (int s = 0; s < SPG; ++s) {
            d_cur[s] = d_nxt[s];
            u_cur[s] = u_nxt[s];
            y_cur[s] = y_nxt[s];
            if constexpr (XD) dd_cur[s] = dd_nxt[s];
        }
        if (more) issue(k - 1);
        // one workgroup-uniform decision per chunk: the clamped path gives the same values whenever
        // no exponent reaches the clamp, so deciding for the whole workgroup is exact
        const bool need_clamp = __builtin_amdgcn_readfirstlane(s_flag[0]) == k;

        // ---- recompute the chunk's states (one exp per state), 4 steps per operand read ----
        float H[TC][SPL], E[TC][SPL];
        {
            auto recompute = [&](auto clamp_tag) {
                constexpr bool CLAMP = decltype(clamp_tag)::value;
                float hh[SPL];
#pragma unroll
                for (int j = 0; j < SPL; ++j) hh[j] = hin[j];
#pragma unroll
                for (int i4 = 0; i4 < TC; i4 += 4) {
                    float dt4[4], dtu4[4];
                    ldv<4>(s_in(0, c) + i4, dt4);
                    ldv<4>(s_in(1, c) + i4, dtu4);
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const int i = i4 + q;
                        float Bv[SPL];
                        ldv<SPL>(&s_bc[i][2 * n0], Bv);
#pragma unroll
                        for (int j = 0; j < SPL; ++j) {
                            const float x = dt4[q] * A2[j];
                            const float e = CLAMP ? exp2_clamped(x) : __builtin_amdgcn_exp2f(x);
                            E[i][j] = e;
                            hh[j] = __builtin_fmaf(e, hh[j], dtu4[q] * Bv[j]);
                            H[i][j] = hh[j];
                        }
                    }
                }
            };
            if (need_clamp)
                recompute(std::true_type{});
            else
                recompute(std::false_type{});
        }
        // ---- reverse sweep ----
        // B/C are read one step ahead and delta/dout one 4-step group ahead of use; every 4 steps the
        // wave folds the phase's deposits over its channels.
        auto fold = [&](int phase) {
            // this lane's (slot, plane, block) row: the block's VB weighted sums for each channel pair
            float v[NPC * VB], acc[VB];
            const float* row = (rpl ? red_h : red_g) + (rs * 8 + rb) * RW;
            if constexpr (kFoldRot) {
                ldv<4>(row + 4 * rpl, *reinterpret_cast<float(*)[4]>(v));
                ldv<4>(row + 4 - 4 * rpl, *reinterpret_cast<float(*)[4]>(v + 4));
            } else {
                ldv<NPC * VB>(row, v);
            }
#pragma unroll
            for (int q = 0; q < VB; ++q) acc[q] = v[q];
#pragma unroll
            for (int p = 1; p < NPC; ++p) {
#pragma unroll
                for (int q = 0; q < VB; ++q) acc[q] += v[p * VB + q];
            }
            stv<VB>(&s_part[wave][phase * kRedSlots + rs][rpl * NS + rb * VB], acc);
        };
        {
            float yq[4], dq[4], uq[4], yqn[4], dqn[4], uqn[4], Bn[SPL], Cn[SPL];
            // The group sums over n of each step, S1 = sum g*B (for du) and S2 = sum g*A*dA*h_{t-1} (with
            // u*S1, ddelta), are reduce-scattered over the group every RST steps: the lane's partials of
            // RST steps x (S1, S2) go in, and the lane writes the one (step, sum) the scatter leaves it.
            // The storing threads add u*S1 once per element.
            constexpr int RV = LPC, RST = RV / 2;
            float rp[RV];
            const int ridx = rs_hi_index<CPW, RV>(lane);
            float* const s_mine = &s_out[ridx & 1][ridx >> 1][c];  // + the round's first step * OS
            ldv<4>(s_in(2, c) + TC - 4, yqn);
            ldv<4>(s_in(0, c) + TC - 4, dqn);
            ldv<4>(s_in(1, c) + TC - 4, uqn);
            auto ld_bc = [&](int i, float (&Bo)[SPL], float (&Co)[SPL]) {
                float bc[2 * SPL];
                ldv<2 * SPL>(&s_bc[i][2 * n0], bc);
#pragma unroll
                for (int j = 0; j < SPL; ++j) {
                    Bo[j] = bc[j];
                    Co[j] = bc[SPL + j];
                }
            };
            ld_bc(TC - 1, Bn, Cn);
#pragma unroll
            for (int i = TC - 1; i >= 0; --i) {
                const int slot = i % kRedSlots, phase = i / kRedSlots;
                if (slot == kRedSlots - 1) {
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        yq[q] = yqn[q];
                        dq[q] = dqn[q];
                        uq[q] = uqn[q];
                    }
                    if (i >= 4) {
                        ldv<4>(s_in(2, c) + i - 7, yqn);
                        ldv<4>(s_in(0, c) + i - 7, dqn);
                        ldv<4>(s_in(1, c) + i - 7, uqn);
                    }
                }
                float Bv[SPL], Cv[SPL];
#pragma unroll
                for (int j = 0; j < SPL; ++j) {
                    Bv[j] = Bn[j];
                    Cv[j] = Cn[j];
                }
                if (i > 0) {
                    ld_bc(i > 0 ? i - 1 : 0, Bn, Cn);
                }
                // keep the next step's operand reads here, a full step ahead of their use (the
                // scheduler would otherwise sink them next to the use and expose the LDS latency)
                __builtin_amdgcn_sched_barrier(0);
                const float yo = yq[slot], dti = dq[slot], dtui = uq[slot];
                float gt[SPL];
                float r1 = 0.f, r2 = 0.f;
#pragma unroll
                for (int j = 0; j < SPL; ++j) {
                    const float prev = (i > 0) ? H[i > 0 ? i - 1 : 0][j] : hin[j];
                    gt[j] = __builtin_fmaf(yo, Cv[j], gc[j]);
                    r1 = __builtin_fmaf(gt[j], Bv[j], r1);
                    gc[j] = E[i][j] * gt[j];
                    const float s = gc[j] * prev;  // g * dA_t * h_{t-1}
                    r2 = __builtin_fmaf(An[j], s, r2);
                    dAacc[j] = __builtin_fmaf(dti, s, dAacc[j]);
                }
                rp[2 * (i % RST)] = r1;
                rp[2 * (i % RST) + 1] = r2;
                if (i % RST == 0) s_mine[i * OS] = reduce_scatter_hi<CPW, RV>(rp);
                // dB/dC: weight g_t by delta*u and h_t by dout, add the channel partner's, deposit the side
                // this lane keeps: state n goes to row (slot, n / VB), column cwp * VB + n % VB
                float pw[2 * SPL], dv[SPL];
#pragma unroll
                for (int j = 0; j < SPL; ++j) {
                    pw[2 * j] = gt[j] * dtui;
                    pw[2 * j + 1] = H[i][j] * yo;
                }
                pair_level<PB, SPL>(pw, dv, lane);
                constexpr int DW = SPL < VB ? SPL : VB;  // floats per deposit write
                float* const dep = dpl ? red_h : red_g;
#pragma unroll
                for (int j0 = 0; j0 < SPL; j0 += DW) {
                    const int n = n0 + j0, o = (slot * 8 + n / VB) * RW + cwp * VB + n % VB;
                    float wv[DW];
#pragma unroll
                    for (int q = 0; q < DW; ++q) wv[q] = dv[j0 + q];
                    stv<DW>(dep + o, wv);
                }
                if (slot == 0) {
                    wave_lds_fence();
                    fold(phase);
                    wave_lds_fence();
                }
            }
        }
        __syncthreads();  // every wave is done with the staged chunk and has written s_out / s_part
        if (more) {
            commit(k - 1);
#pragma unroll
            for (int j = 0; j < SPL; ++j) hin[j] = hnext[j];
        }
        // du / ddelta of the loader's (channel, steps), read back from the tile
        {
            const rsrc_t rdu = make_rsrc(du + rowD + (int64_t)t0 * D, chunk_rows(k) * row_bytes);
            const rsrc_t rdd = make_rsrc(ddelta + rowD + (int64_t)t0 * D, chunk_rows(k) * row_bytes);
#pragma unroll
            for (int s = 0; s < SPG; ++s) {
                const float s1 = s_out[0][sg * SPG + s][lc];
                buf_st<T>(rdu, lofs + s * row_bytes, __builtin_fmaf(Dl, y_cur[s], d_cur[s] * s1));
                float dd = __builtin_fmaf(u_cur[s], s1, s_out[1][sg * SPG + s][lc]);  // + u * S1
                if constexpr (XD) {
                    dd *= dd_cur[s];  // through softplus (1 without it)
                    if (t0 + sg * SPG + s < L) dbias_acc += dd;
                }
                buf_st<T>(rdd, lofs + s * row_bytes, dd);
            }
        }
        {  // this workgroup's dB/dC partial for the chunk (sum of its 4 waves), PV consecutive values
           // per thread; the buffer spans the chunk's rows before L, so the stores of later rows drop
            constexpr int PV = TC * 2 * NS / 256;
            static_assert(PV * 256 == TC * 2 * NS && (PV <= 2 || PV % 4 == 0), "partial tiling");
            const int o = tid * PV, tt = o / (2 * NS), v = o % (2 * NS);
            float acc[PV], w[PV];
            ldv<PV>(&s_part[0][tt][v], acc);
#pragma unroll
            for (int q = 1; q < 4; ++q) {
                ldv<PV>(&s_part[q][tt][v], w);
#pragma unroll
                for (int p = 0; p < PV; ++p) acc[p] += w[p];
            }
            const rsrc_t rp = make_rsrc(dbc_part + (((int64_t)blk * Bsz + b) * L + t0) * (2 * NS),
                                        chunk_rows(k) * 2 * NS * sizeof(float));
            buf_st_f32<PV>(rp, o * sizeof(float), acc);
        }
        __syncthreads();  // the next chunk's tile is staged; s_out / s_part are free again
    }

    if (valid) {
        if (dh_prev != nullptr && seg == 0) {
#pragma unroll
            for (int j = 0; j < SPL; ++j) st(dh_prev + ((int64_t)b * D + d) * NS + n0 + j, gc[j]);
        }
        const int64_t pr = (int64_t)seg * Bsz + b;  // partial row
        stv<SPL>(dA_part + (pr * D + d) * NS + n0, dAacc);
        if (wi.whole) {  // a whole row of a partly split plan: its other segments' partial rows are zero
            float z[SPL];
#pragma unroll
            for (int j = 0; j < SPL; ++j) z[j] = 0.f;
            for (int s2 = 1; s2 < nseg; ++s2) stv<SPL>(dA_part + (((int64_t)s2 * Bsz + b) * D + d) * NS + n0, z);
        }
    }
    {  // dD (and delta_bias) partials: the NSG loader threads of a channel, in order
        const bool with_bias = XD && xf.delta_bias != nullptr;
        __syncthreads();
        float* red = &s_out[0][0][0];  // free after the chunk loop; 2*NSG*CPB <= 2*TC*OS floats
        red[sg * CPB + lc] = dDl;
        if (with_bias) red[NSG * CPB + sg * CPB + lc] = dbias_acc;
        __syncthreads();
        if (tid < CPB && d0 + tid < D) {
            const int64_t pr = (int64_t)seg * Bsz + b;
            float acc = 0.f, accb = 0.f;
            for (int q = 0; q < NSG; ++q) {
                acc += red[q * CPB + tid];
                if (with_bias) accb += red[NSG * CPB + q * CPB + tid];
            }
            dD_part[pr * D + d0 + tid] = acc;
            if (with_bias) dbias_part[pr * D + d0 + tid] = accb;
            for (int s2 = 1; wi.whole && s2 < nseg; ++s2) {  // as for dA
                dD_part[((int64_t)s2 * Bsz + b) * D + d0 + tid] = 0.f;
                if (with_bias) dbias_part[((int64_t)s2 * Bsz + b) * D + d0 + tid] = 0.f;
            }
        }
    }
}

// The backward's reductions, one launch: blocks [0, nblk_bc) sum the channel-group dB/dC partials
// (4 consecutive values per thread, groups in order), the rest sum the (segment, batch) dA/dD
// partials in order. Fixed summation orders: the results are deterministic.
template <typename T, int NS>
__global__ void __launch_bounds__(256) bwd_finish_kernel(const float* __restrict__ part, T* __restrict__ dB,
                                                         T* __restrict__ dC, int ngrp, int64_t rows, int nblk_bc,
                                                         const float* __restrict__ dA_part,
                                                         const float* __restrict__ dD_part, T* __restrict__ dA,
                                                         T* __restrict__ dD, int nrows, int D,
                                                         const float* __restrict__ dbias_part, T* __restrict__ dbias) {
    if ((int)blockIdx.x < nblk_bc) {
        const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;  // over rows*2NS, 4-aligned
        if (i >= rows * 2 * NS) return;
        const int64_t stride = rows * 2 * NS;
        const float* p = part + i;
        float acc[4] = {0.f, 0.f, 0.f, 0.f};
        int q = 0;
        for (; q + 4 <= ngrp; q += 4) {
            float4 v[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) v[u] = *reinterpret_cast<const float4*>(p + (int64_t)(q + u) * stride);
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                acc[0] += v[u].x;
                acc[1] += v[u].y;
                acc[2] += v[u].z;
                acc[3] += v[u].w;
            }
        }
        for (; q < ngrp; ++q) {
            const float4 v = *reinterpret_cast<const float4*>(p + (int64_t)q * stride);
            acc[0] += v.x;
            acc[1] += v.y;
            acc[2] += v.z;
            acc[3] += v.w;
        }
        const int64_t r = i / (2 * NS);
        const int col = (int)(i % (2 * NS));  // the 4 values are all dB (col < NS) or all dC
        T* dst = col < NS ? dB + r * NS + col : dC + r * NS + col - NS;
#pragma unroll
        for (int u = 0; u < 4; ++u) st(dst + u, acc[u]);
        return;
    }
    const int64_t i = (int64_t)(blockIdx.x - nblk_bc) * 256 + threadIdx.x;
    const int64_t nA = (int64_t)D * NS;
    // sum of rows 0..nrows-1 in order. Few threads do this part (D*NS of them), so it is latency-bound:
    // 32 loads are in flight before their adds (rows past nrows add 0, which leaves the sum unchanged).
    auto rows_sum = [nrows](const float* p, int64_t stride) {
        float s = 0.f;
        for (int r = 0; r < nrows; r += 32) {
            float v[32];
#pragma unroll
            for (int q = 0; q < 32; ++q) v[q] = r + q < nrows ? p[(int64_t)(r + q) * stride] : 0.f;
#pragma unroll
            for (int q = 0; q < 32; ++q) s += v[q];
        }
        return s;
    };
    if (i < nA) {
        st(dA + i, rows_sum(dA_part + i, nA));
    } else if (i < nA + D) {
        const int64_t dd = i - nA;
        st(dD + dd, rows_sum(dD_part + dd, D));
    } else if (dbias != nullptr && i < nA + 2 * D) {
        const int64_t dd = i - nA - D;
        st(dbias + dd, rows_sum(dbias_part + dd, D));
    }
}

int bwd_wgs_per_cu(int ns, int spl, bool carry) {
    // as fwd_wgs_per_cu: the fp16, transform-free instance's occupancy, queried once; 0 if unknown
    static std::atomic<int> cache[4][3][2];
    const int ni = ns == 8 ? 0 : ns == 16 ? 1 : ns == 32 ? 2 : 3, si = spl == 1 ? 0 : spl == 2 ? 1 : 2;
    int v = cache[ni][si][carry].load(std::memory_order_relaxed);
    if (v != 0) return v < 0 ? 0 : v;
    const void* k = nullptr;
#define MWC_BWD_K(N, S)                                                                                   \
    if (ns == N && spl == S)                                                                              \
        k = carry ? reinterpret_cast<const void*>(&ssm_bwd_carry_kernel<half_t, N, S, 0>)                 \
                  : reinterpret_cast<const void*>(&ssm_bwd_kernel<half_t, N, S, 0>);
    MWC_FOR_EACH_LANE_GROUP(MWC_BWD_K)
#undef MWC_BWD_K
    int n = 0;
    if (k == nullptr || hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, k, 256, 0) != hipSuccess || n <= 0) {
        (void)hipGetLastError();
        n = -1;
    }
    cache[ni][si][carry].store(n, std::memory_order_relaxed);
    return n < 0 ? 0 : n;
}

int bwd_groups(const SsmShape& s, int ns, int spl) {
    const int cpb = 4 * 64 / (ns / spl);
    return (int)((s.dim + cpb - 1) / cpb);
}

template <typename T, int NS, int SPL, int XF>
static hipError_t bwd_inst(const BwdArgs& a, const SsmShape& s, hipStream_t st) {
    const int nblk_d = bwd_groups(s, NS, SPL);
    const int nck = (int)((s.seqlen + kCkptSteps - 1) / kCkptSteps);
    // a partly split plan launches its whole rows once and its split rows once per (carry) segment
    const int rows = nblk_d * (int)s.batch, split = a.nfull > 0 ? rows - a.nfull : rows;
    if (a.nseg > 1)  // carries of every chunk after the first segment
        hipLaunchKernelGGL((ssm_bwd_carry_kernel<T, NS, SPL, XF>), dim3(split * a.ncar), dim3(256), 0, st,
                           (const T*)a.delta, (const T*)a.A, (const T*)a.C, (const T*)a.dout, a.car_g, a.car_x,
                           (int)s.batch, (int)s.seqlen, (int)s.dim, nck, nblk_d, a.ncar, a.cps, a.cps / a.cfold,
                           a.xf, a.nfull);
    hipLaunchKernelGGL((ssm_bwd_kernel<T, NS, SPL, XF>), dim3((a.nfull > 0 ? a.nfull : 0) + split * a.nseg),
                       dim3(256), 0, st, (const T*)a.u,
                       (const T*)a.delta, (const T*)a.A, (const T*)a.B, (const T*)a.C, (const T*)a.Dv,
                       (const T*)a.dout, (const T*)a.dh_last, a.ckpt, (T*)a.du, (T*)a.ddelta, (T*)a.dh_prev,
                       a.dA_part, a.dD_part, a.dbc_part, a.car_g, a.car_x, (int)s.batch, (int)s.seqlen, (int)s.dim,
                       nck, nblk_d, a.nseg, a.cps, a.ncar, a.cfold, a.xf, (const T*)a.y, (T*)a.dz, a.dbias_part,
                       a.nfull);
    return hipGetLastError();
}

template <typename T, int NS, int SPL>
static hipError_t bwd_inst(const BwdArgs& a, const SsmShape& s, hipStream_t st) {
    const int xf = (a.xf.delta_bias != nullptr || a.xf.softplus ? kXfDelta : 0) | (a.xf.z != nullptr ? kXfGate : 0);
    switch (xf) {
        case 0: return bwd_inst<T, NS, SPL, 0>(a, s, st);
        case kXfDelta: return bwd_inst<T, NS, SPL, kXfDelta>(a, s, st);
        case kXfGate: return bwd_inst<T, NS, SPL, kXfGate>(a, s, st);
        default: return bwd_inst<T, NS, SPL, kXfDelta | kXfGate>(a, s, st);
    }
}

hipError_t launch_ssm_bwd(int dt, int ns, int spl, const BwdArgs& a, const SsmShape& s, hipStream_t st) {
#define MWC_BWD(N, S) \
    if (ns == N && spl == S) MWC_DISPATCH_DTYPE(dt, TT, return bwd_inst<TT, N, S>(a, s, st));
    MWC_FOR_EACH_LANE_GROUP(MWC_BWD)
#undef MWC_BWD
    return hipErrorInvalidValue;
}

template <typename T, int NS>
static hipError_t finish_t(const float* dbc_part, const float* dA_part, const float* dD_part,
                           const float* dbias_part, void* dB, void* dC, void* dA, void* dD, void* dbias, int ngrp,
                           int nrows, const SsmShape& s, hipStream_t st) {
    const int64_t rows = s.batch * s.seqlen;
    const int nblk_bc = (int)((rows * 2 * NS / 4 + 255) / 256);
    const int64_t n2 = s.dim * NS + 2 * s.dim;
    const int nblk_ad = (int)((n2 + 255) / 256);
    hipLaunchKernelGGL((bwd_finish_kernel<T, NS>), dim3(nblk_bc + nblk_ad), dim3(256), 0, st, dbc_part, (T*)dB,
                       (T*)dC, ngrp, rows, nblk_bc, dA_part, dD_part, (T*)dA, (T*)dD, nrows, (int)s.dim, dbias_part,
                       (T*)dbias);
    return hipGetLastError();
}

hipError_t launch_bwd_finish(int dt, int ns, const float* dbc_part, const float* dA_part, const float* dD_part,
                             const float* dbias_part, void* dB, void* dC, void* dA, void* dD, void* dbias,
                             int ngroups, int nrows, const SsmShape& s, hipStream_t st) {
#define MWC_FIN(N)                                                                                              \
    if (ns == N)                                                                                                \
        MWC_DISPATCH_DTYPE(dt, TT,                                                                              \
                           return finish_t<TT, N>(dbc_part, dA_part, dD_part, dbias_part, dB, dC, dA, dD, dbias, \
                                                  ngroups, nrows, s, st));
    MWC_FIN(8)
    MWC_FIN(16)
    MWC_FIN(32)
    MWC_FIN(64)
#undef MWC_FIN
    return hipErrorInvalidValue;
}

}  // namespace mwc
