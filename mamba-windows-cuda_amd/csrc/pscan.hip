// Standalone first-order linear recurrence ("parallel_scan_fn") for gfx950.
//
// Semantics: parallel_scan_ref (pscan.py:153-171): over the middle axis of
// [nseq][L][ncols], H_0 = X_0 (A_0 unused), H_t = A_t*H_{t-1} + X_t, with fp32
// accumulation; and its adjoint (replacing PScan.backward, pscan.py:97-136,
// whose math is wrong for L >= 4): G_t = dH_t + A_{t+1}*G_{t+1}, dX = G,
// dA_t = G_t*H_{t-1} for t >= 1 and dA_0 = 0.
//
// Design: one pass over HBM (12 B/element forward, 20 B/element backward).
// A tile is TL consecutive steps x CW columns; each thread owns one column and
// RUN consecutive steps held in VGPRs. Thread runs are combined inside the
// tile through LDS; tiles along L are chained with a decoupled look-back:
// each tile publishes its aggregate map h -> a*h + b per column, then its
// inclusive prefix once known, as 64-bit (status << 32 | fp32 bits) words so
// a single relaxed agent-scope atomic carries both the flag and the value
// (no cache-wide release/acquire fences). Tiles are taken from an atomic
// ticket so every predecessor of a waiting tile is already resident, and each
// spin is bounded so a lost update can never hang the device. A wait that runs
// out of spins sets the workspace's error word (read by mwc_pscan_status) and
// gives the tile a NaN prefix, so its outputs, and every later tile's, are NaN
// rather than a plausible wrong value.
#include <algorithm>

#include "common.h"
#include "launch.h"

namespace mwc {

namespace {

constexpr int kThreads = 256;
constexpr int kTileSteps = 128;
constexpr uint32_t kStAgg = 1, kStInc = 2;

int pick_cw(int64_t ncols) { return ncols <= 16 ? 16 : (ncols <= 32 ? 32 : 64); }

struct PscanGeom {
    int cw, ncolblk, nltile;
    int64_t nchains, ntiles;
    size_t flag_bytes;
};

PscanGeom geom(int64_t nseq, int64_t seqlen, int64_t ncols) {
    PscanGeom g;
    g.cw = pick_cw(ncols);
    g.ncolblk = (int)((ncols + g.cw - 1) / g.cw);
    g.nltile = (int)((seqlen + kTileSteps - 1) / kTileSteps);
    g.nchains = nseq * g.ncolblk;
    g.ntiles = g.nchains * g.nltile;
    g.flag_bytes = (size_t)g.ntiles * g.cw * 2 * sizeof(uint64_t);
    return g;
}

__device__ __forceinline__ uint64_t pack(uint32_t st, float v) {
    return ((uint64_t)st << 32) | (uint64_t)__builtin_bit_cast(uint32_t, v);
}
__device__ __forceinline__ float unpack_v(uint64_t w) { return __builtin_bit_cast(float, (uint32_t)(w & 0xffffffffu)); }

__device__ __forceinline__ void publish(uint64_t* p, uint64_t w) {
    __hip_atomic_store(p, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Wait until *p carries a non-zero status; returns the word. If `limit` polls pass without one, the
// error word is set and an inclusive NaN is returned: the tile's prefix, and so its outputs, are NaN.
__device__ __forceinline__ uint64_t wait_word(const uint64_t* p, unsigned* err, unsigned limit) {
    for (unsigned it = 0; it < limit; ++it) {
        const uint64_t w = __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if ((w >> 32) != 0) return w;
        __builtin_amdgcn_s_sleep(2);
    }
    atomicOr(err, 1u);
    return pack(kStInc, __builtin_nanf(""));
}

}  // namespace

__global__ void __launch_bounds__(256) pscan_clear_kernel(uint64_t* __restrict__ p, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) p[i] = 0;
}

// REV = false: forward scan of X with coefficients A (A_0 ignored) into Out.
// REV = true : adjoint; X = dH, Out = dX, Hs = forward H, dAo = dA.
template <typename T, int CW, bool REV>
__global__ void __launch_bounds__(kThreads) pscan_kernel(const T* __restrict__ A, const T* __restrict__ X,
                                                         const T* __restrict__ Hs, T* __restrict__ Out,
                                                         T* __restrict__ dAo, uint64_t* __restrict__ flags,
                                                         unsigned* __restrict__ ticket, unsigned* __restrict__ err,
                                                         int L, int ncols, int ncolblk, int64_t nchains,
                                                         unsigned spin_limit) {
    constexpr int R = kThreads / CW;     // thread rows per tile
    constexpr int RUN = kTileSteps / R;  // steps per thread
    __shared__ int s_tile;
    __shared__ float s_a[R][CW], s_h[R][CW], s_p[CW];

    if (threadIdx.x == 0) s_tile = (int)atomicAdd(ticket, 1u);
    __syncthreads();
    const int64_t tile = s_tile;
    const int lt = (int)(tile / nchains);  // position of the tile along L (in scan order)
    const int64_t chain = tile % nchains;
    const int64_t seq = chain / ncolblk;
    const int cb = (int)(chain % ncolblk);
    const int cl = threadIdx.x % CW, r = threadIdx.x / CW;
    const int col = cb * CW + cl;
    const bool cvalid = col < ncols;
    const int64_t base = seq * L * ncols + (cvalid ? col : ncols - 1);
    const int p0 = lt * kTileSteps + r * RUN;

    // position p -> time index t (the adjoint runs from the end)
    float a[RUN], x[RUN];
#pragma unroll
    for (int i = 0; i < RUN; ++i) {
        const int p = p0 + i;
        if (p < L) {
            const int t = REV ? L - 1 - p : p;
            if constexpr (REV)
                a[i] = (t + 1 < L) ? ld(A + base + (int64_t)(t + 1) * ncols) : 0.f;
            else
                a[i] = (t > 0) ? ld(A + base + (int64_t)t * ncols) : 0.f;
            x[i] = ld(X + base + (int64_t)t * ncols);
        } else {
            a[i] = 1.f;
            x[i] = 0.f;
        }
    }
    // the run's map h -> ra*h + rh
    float ra = 1.f, rh = 0.f;
#pragma unroll
    for (int i = 0; i < RUN; ++i) {
        rh = __builtin_fmaf(a[i], rh, x[i]);
        ra *= a[i];
    }
    s_a[r][cl] = ra;
    s_h[r][cl] = rh;
    __syncthreads();

    if (r == 0) {
        float ta = 1.f, th = 0.f;  // the tile's map
#pragma unroll
        for (int q = 0; q < R; ++q) {
            th = __builtin_fmaf(s_a[q][cl], th, s_h[q][cl]);
            ta *= s_a[q][cl];
        }
        uint64_t* f = flags + ((chain * (int64_t)((L + kTileSteps - 1) / kTileSteps) + lt) * CW + cl) * 2;
        float prefix = 0.f;  // state entering the tile (the scan starts from 0; t = 0 ignores A_0)
        if (lt == 0) {
            publish(f, pack(kStInc, th));
        } else {
            publish(f + 1, pack(kStAgg, ta));
            publish(f, pack(kStAgg, th));
            float acc_a = 1.f, acc_h = 0.f;  // map of the tiles between the predecessor and this one
            uint64_t* pf = f - (int64_t)CW * 2;
            for (int j = lt - 1; j >= 0; --j, pf -= (int64_t)CW * 2) {
                const uint64_t w = wait_word(pf, err, spin_limit);
                if ((w >> 32) == kStInc) {
                    prefix = __builtin_fmaf(acc_a, unpack_v(w), acc_h);
                    break;
                }
                const uint64_t wa = wait_word(pf + 1, err, spin_limit);
                acc_h = __builtin_fmaf(acc_a, unpack_v(w), acc_h);
                acc_a *= unpack_v(wa);
            }
            publish(f, pack(kStInc, __builtin_fmaf(ta, prefix, th)));
        }
        s_p[cl] = prefix;
    }
    __syncthreads();

    // state entering this thread's run: rows 0..r-1 applied to the tile prefix
    float h = s_p[cl];
    for (int q = 0; q < r; ++q) h = __builtin_fmaf(s_a[q][cl], h, s_h[q][cl]);
#pragma unroll
    for (int i = 0; i < RUN; ++i) {
        const int p = p0 + i;
        h = __builtin_fmaf(a[i], h, x[i]);
        if (p < L && cvalid) {
            const int t = REV ? L - 1 - p : p;
            st(Out + base + (int64_t)t * ncols, h);
            if constexpr (REV) st(dAo + base + (int64_t)t * ncols, t > 0 ? h * ld(Hs + base + (int64_t)(t - 1) * ncols) : 0.f);
        }
    }
}

size_t pscan_workspace_bytes(int64_t nseq, int64_t seqlen, int64_t ncols) {
    if (nseq <= 0 || seqlen <= 0 || ncols <= 0) return 0;
    const PscanGeom g = geom(nseq, seqlen, ncols);
    return ((g.flag_bytes + 255) & ~(size_t)255) + 256;  // flags, then ticket + error word
}

size_t pscan_error_word_offset(int64_t nseq, int64_t seqlen, int64_t ncols) {
    const PscanGeom g = geom(nseq, seqlen, ncols);
    return ((g.flag_bytes + 255) & ~(size_t)255) + sizeof(unsigned);  // after the ticket
}

template <typename T, bool REV>
static hipError_t pscan_t(const void* A, const void* X, const void* Hs, void* Out, void* dAo, int64_t nseq,
                          int64_t seqlen, int64_t ncols, void* ws, unsigned spin_limit, hipStream_t st) {
    const PscanGeom g = geom(nseq, seqlen, ncols);
    uint64_t* flags = (uint64_t*)ws;
    const size_t fb = (g.flag_bytes + 255) & ~(size_t)255;
    unsigned* ticket = (unsigned*)((char*)ws + fb);
    unsigned* err = ticket + 1;
    const int64_t nwords = (int64_t)(fb + 256) / 8;
    const int cgrid = (int)std::min<int64_t>((nwords + 255) / 256, 4096);
    hipLaunchKernelGGL(pscan_clear_kernel, dim3(cgrid), dim3(256), 0, st, flags, nwords);
    if (g.ntiles > INT32_MAX) return hipErrorInvalidValue;
#define MWC_PSCAN_CW(CWV)                                                                                         \
    if (g.cw == CWV)                                                                                              \
        hipLaunchKernelGGL((pscan_kernel<T, CWV, REV>), dim3((unsigned)g.ntiles), dim3(kThreads), 0, st,          \
                           (const T*)A, (const T*)X, (const T*)Hs, (T*)Out, (T*)dAo, flags, ticket, err,           \
                           (int)seqlen, (int)ncols, g.ncolblk, g.nchains, spin_limit);
    MWC_PSCAN_CW(16)
    MWC_PSCAN_CW(32)
    MWC_PSCAN_CW(64)
#undef MWC_PSCAN_CW
    return hipGetLastError();
}

hipError_t launch_pscan_fwd(int dt, const void* A, const void* X, void* H, int64_t nseq, int64_t seqlen,
                            int64_t ncols, void* ws, unsigned spin_limit, hipStream_t st) {
    MWC_DISPATCH_DTYPE(dt, TT,
                       return pscan_t<TT, false>(A, X, nullptr, H, nullptr, nseq, seqlen, ncols, ws, spin_limit, st));
}

hipError_t launch_pscan_bwd(int dt, const void* A, const void* H, const void* dH, void* dA, void* dX,
                            int64_t nseq, int64_t seqlen, int64_t ncols, void* ws, unsigned spin_limit,
                            hipStream_t st) {
    MWC_DISPATCH_DTYPE(dt, TT, return pscan_t<TT, true>(A, dH, H, dX, dA, nseq, seqlen, ncols, ws, spin_limit, st));
}

}  // namespace mwc
