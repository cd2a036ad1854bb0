// Internal launcher interface between the C ABI (capi.hip) and the kernel files.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mwc {

struct SsmShape {
    int64_t batch, seqlen, dim;
    int nstate = 16;  // N: 8, 16, 32 or 64
};

// The (state count NS, states per lane SPL) pairs the lane-group kernels are built for: NS/SPL lanes
// per channel, a power of two from 4 to 16 (the DPP reductions stay inside a 16-lane row).
#define MWC_FOR_EACH_LANE_GROUP(X) X(8, 1) X(8, 2) X(16, 1) X(16, 2) X(16, 4) X(32, 2) X(32, 4) X(64, 4)
bool lane_group_supported(int ns, int spl);

// Waves per SIMD the lane-group kernels are compiled to fit (each lane then has 512/W VGPRs). The
// forward at four states per lane fits three waves without transforms and two with them.
// At N=8 and two states per lane a loader thread holds 4 steps of each staged operand (twice N=16's):
// the carry passes get 5 waves per SIMD instead of 6, which keeps them from spilling at no measured
// cost. The backward main kernel keeps 3 waves and spills 20-96 bytes per lane there: at 2 waves it
// does not spill but takes 27% longer (B=8, L=2048, D=1536, N=8: 203.6 against 160.0 us per call).
constexpr int fwd_min_waves(int spl) { return spl == 4 ? 2 : spl == 1 ? 6 : 3; }
constexpr int bwd_min_waves(int ns, int spl) { return spl == 4 ? 1 : 3; }
constexpr int carry_min_waves(int ns, int spl) { return spl == 4 ? 1 : (ns == 8 && spl == 2) ? 5 : 6; }

// Launch plan of the lane-group kernels: SPL = states held per lane (16/SPL lanes per channel),
// nseg = segments L is cut into (cps chunks of kCkptSteps steps each), cfold = carry segments per
// segment (the carry passes run cps/cfold chunks per workgroup), ncar = carry segments in all.
// nfull > 0 marks a partly split plan (nseg = 2): the first nfull rows -- a row is one (batch, channel
// group) -- run whole, the others as two segments with carries.
struct SegPlan {
    int spl, nseg, cps, cfold, ncar;
    int nfull = 0;
};

// A main-pass workgroup's row (b * nblk_d + channel group) and segment.
// Uniform plans (nfull == 0) number the (row, segment) items segment-major, k = seg * rows + row. Each
// XCD deals its contiguous share of the grid (see xcd_remap) to its 32 CUs breadth-first: logical
// block j of the share runs on CU j % 32 of that XCD, as its (j / 32)-th workgroup (measured on MI355X
// with a probe that records each workgroup's hardware CU id). When the grid is whole rounds of all 256
// CUs, item k = round * 256 + XCD * 32 + CU, so every CU holds items from different parts of the
// segment order: segments late in the order fold more carries before their first chunk, and a CU that
// mixes them keeps computing while one of its workgroups folds (1-3% per call at the fill plans'
// shapes, none at config 2). Otherwise the items follow the block order.
// In a partly split plan the workgroups are nfull whole rows and two halves of each other row; when the
// counts allow, each XCD's contiguous share of the grid holds its whole rows first and its halves after
// them, so that each CU receives whole rows and halves in the same proportion.
struct WorkItem {
    int row, seg;
    bool whole;  // the row runs unsplit in a partly split plan
};
__device__ __forceinline__ WorkItem main_item(int lid, int rows, int nfull, int total) {
    constexpr int kXcds = 8, kCusPerXcd = 32;
    if (nfull <= 0) {
        int k = lid;
        if (total % (kXcds * kCusPerXcd) == 0) {
            const int per = total / kXcds, x = lid / per, j = lid % per;
            k = (j / kCusPerXcd) * (kXcds * kCusPerXcd) + x * kCusPerXcd + j % kCusPerXcd;
        }
        return WorkItem{k % rows, k / rows, false};
    }
    int h = lid - nfull;  // half index, or negative for a whole row
    int f = lid;
    if (nfull % 8 == 0 && total % 8 == 0) {
        const int per = total / 8, fx = nfull / 8, x = lid / per, i = lid % per;
        f = x * fx + i;
        h = i < fx ? -1 : x * ((total - nfull) / 8) + (i - fx);
    }
    if (h < 0) return WorkItem{f, 0, true};
    return WorkItem{nfull + h / 2, h % 2, false};
}
// A carry-pass workgroup's row and carry segment: the carries exist for the split rows only.
__device__ __forceinline__ WorkItem carry_item(int lid, int rows, int nfull) {
    const int first = nfull > 0 ? nfull : 0, n = rows - first;
    return WorkItem{first + lid % n, lid / n, false};
}
SegPlan plan_fwd(const SsmShape& s);
SegPlan plan_bwd(const SsmShape& s);
// Workgroups per CU of a lane-group kernel instance (the HIP runtime's occupancy query, cached), or 0 when
// no device can be queried. fwd mode: 0 main, 1 state-only, 2 carry.
int fwd_wgs_per_cu(int ns, int spl, int mode);
int bwd_wgs_per_cu(int ns, int spl, bool carry);

// Workspace carve-up (bytes, 256-aligned pieces).
size_t fwd_workspace_bytes(const SsmShape& s);
size_t bwd_workspace_bytes(const SsmShape& s);
int bwd_groups(const SsmShape& s, int ns, int spl);  // channel groups that write dB/dC partials

// Optional elementwise transforms fused around the scan (all NULL / 0: the plain scan).
//   delta' = softplus(delta + delta_bias) (bias and softplus each optional; rows past L stay 0)
//   out_z  = out * silu(z)
struct ScanXf {
    const void* delta_bias;  // (dim,)
    const void* z;           // (batch, seqlen, dim)
    int softplus;
};
// The scan kernels are compiled per set of transforms (a template bit mask), so the plain scan
// carries none of their registers and no kernel tests for a transform it does not apply inside its
// chunk loop: kXfDelta = delta' = softplus?(delta + delta_bias?) (bias and softplus stay run-time
// flags), kXfGate = the z gate.
constexpr int kXfDelta = 1, kXfGate = 2;

struct FwdArgs {
    const void *u, *delta, *A, *B, *C, *Dv, *h_prev;
    void *out, *h_last;        // out == NULL: state-only pass (checkpoints and/or h_last)
    float* ckpt;               // [batch][nck][dim][16] or NULL
    float *car_h, *car_x;      // [batch][ncar][dim][16] carries (nseg > 1)
    int nseg, cps, cfold, ncar;
    ScanXf xf;
    void* out_z;               // gated output (xf.z != NULL); `out` then receives the ungated one
    int nfull;                 // rows run whole in a partly split plan (SegPlan::nfull)
};

struct BwdArgs {
    const void *u, *delta, *A, *B, *C, *Dv, *dout, *dh_last;
    const float* ckpt;
    void *du, *ddelta, *dh_prev;
    float* dA_part;            // [nseg][batch][dim][16]
    float* dD_part;            // [nseg][batch][dim]
    float* dbc_part;           // [groups][batch][seqlen][32]
    float *car_g, *car_x;      // [batch][ncar][dim][16] adjoint carries (nseg > 1)
    int nseg, cps, cfold, ncar;
    ScanXf xf;
    const void* y;             // ungated forward output (xf.z != NULL)
    void* dz;                  // gradient of z (xf.z != NULL)
    float* dbias_part;         // [nseg][batch][dim] delta_bias partials (xf.delta_bias != NULL)
    int nfull;                 // rows run whole in a partly split plan (SegPlan::nfull)
};

// Kernel launchers; `dt` is the storage dtype (mwc_dtype). They only enqueue work.
hipError_t launch_ssm_fwd(int dt, int ns, int spl, const FwdArgs& a, const SsmShape& s, hipStream_t st);
hipError_t launch_ssm_bwd(int dt, int ns, int spl, const BwdArgs& a, const SsmShape& s, hipStream_t st);
// Sums the dB/dC partials of `ngroups` channel groups and the dA/dD (and, when dbias is not NULL,
// delta_bias) partials of `nrows` rows.
hipError_t launch_bwd_finish(int dt, int ns, const float* dbc_part, const float* dA_part,
                             const float* dD_part, const float* dbias_part, void* dB, void* dC, void* dA,
                             void* dD, void* dbias, int ngroups, int nrows, const SsmShape& s, hipStream_t st);

// One decode step (ssm_step.hip): u, delta, z, y, y_z (batch, dim); B, C (batch, ns); h (batch, dim, ns).
hipError_t launch_ssm_step(int dt, int ns, const void* u, const void* delta, const void* A, const void* B,
                           const void* C, const void* Dv, const void* h_in, const ScanXf& xf, void* y, void* y_z,
                           void* h_out, int64_t batch, int64_t dim, hipStream_t st);

// spin_limit bounds every look-back wait (polls); a wait that runs out sets the workspace's error
// word and poisons the tile's outputs with NaN.
hipError_t launch_pscan_fwd(int dt, const void* A, const void* X, void* H, int64_t nseq,
                            int64_t seqlen, int64_t ncols, void* ws, unsigned spin_limit, hipStream_t st);
hipError_t launch_pscan_bwd(int dt, const void* A, const void* H, const void* dH, void* dA,
                            void* dX, int64_t nseq, int64_t seqlen, int64_t ncols, void* ws,
                            unsigned spin_limit, hipStream_t st);
size_t pscan_workspace_bytes(int64_t nseq, int64_t seqlen, int64_t ncols);
size_t pscan_error_word_offset(int64_t nseq, int64_t seqlen, int64_t ncols);  // byte offset in the workspace
constexpr unsigned kPscanSpinLimit = 1u << 22;  // default bound of a look-back wait (polls of ~128 clocks)

// Grid helper: map hardware block ids so that consecutive logical blocks run on
// the same XCD (the dispatcher deals block i to XCD i % 8), which keeps blocks
// sharing cache lines inside one XCD's L2.
__device__ __forceinline__ int xcd_remap(int bid, int nblocks) {
    constexpr int kXcd = 8;
    if (nblocks % kXcd != 0) return bid;
    return (bid % kXcd) * (nblocks / kXcd) + bid / kXcd;
}

}  // namespace mwc
