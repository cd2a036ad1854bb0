// extern "C" entry points declared in include/mwc_ssm.h.
//
// Argument validation restates the reference host wrappers' contract
// (mamba_cuda.py:185-238, 281-326): N must be 16, dtypes fp32/fp16, shapes
// consistent. Everything is checked before the first launch; the functions
// only enqueue work on the caller's stream and never allocate.
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>

#include "common.h"
#include "launch.h"

namespace {

thread_local char g_err[512] = "";

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

int spl_override() {
    static const int v = [] {
        const char* e = getenv("MWC_SPL");
        if (!e) return 0;
        const int s = atoi(e);
        return (s == 1 || s == 2 || s == 4) ? s : 0;
    }();
    return v;
}

int fail(int status, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return status;
}

int check_dims(int dtype, int64_t batch, int64_t seqlen, int64_t dim, int64_t dstate) {
    if (dtype != MWC_DTYPE_F32 && dtype != MWC_DTYPE_F16)
        return fail(MWC_ERR_INVALID_ARGUMENT, "dtype must be MWC_DTYPE_F32 or MWC_DTYPE_F16 (got %d)", dtype);
    if (dstate != mwc::kNState) return fail(MWC_ERR_INVALID_ARGUMENT, "Only N=16 is supported (got N=%lld)", (long long)dstate);
    if (batch < 0 || seqlen < 0 || dim < 0)
        return fail(MWC_ERR_INVALID_ARGUMENT, "negative size (batch=%lld, seqlen=%lld, dim=%lld)", (long long)batch,
                    (long long)seqlen, (long long)dim);
    if (seqlen > INT32_MAX / 2 || dim > INT32_MAX / 2 || batch > 65535)
        return fail(MWC_ERR_UNSUPPORTED, "sizes beyond the supported range (batch=%lld, seqlen=%lld, dim=%lld)",
                    (long long)batch, (long long)seqlen, (long long)dim);
    return MWC_OK;
}

}  // namespace

int mwc_set_error(int status, const char* msg) { return fail(status, "%s", msg); }

int mwc_set_hip_error(hipError_t e, const char* what) {
    return fail(MWC_ERR_HIP, "%s failed: %s", what, hipGetErrorString(e));
}

namespace mwc {

// States per lane. Measured on MI355X at B=8, L=2048, D=1536 (fp16): SPL=2 (8 lanes per
// channel, 1.5 waves per SIMD) beats SPL=4 (one wave per SIMD, every stall exposed) and SPL=1
// (4x the per-lane overhead). Small problems use SPL=1 for parallelism.
int choose_spl(int64_t channels) {
    if (const int o = spl_override()) return o;
    return channels >= 2048 ? 2 : 1;
}

// Kernel family: 2 = lane groups (ssm_fwd.hip / ssm_bwd.hip, the default), 3 = state groups across
// waves (ssm_v3.hip; selectable with MWC_IMPL=3 while it is slower at the benchmark shapes).
int impl_choice() {
    static const int v = [] {
        const char* e = getenv("MWC_IMPL");
        return (e && atoi(e) == 3) ? 3 : 2;
    }();
    return v;
}

size_t fwd_workspace_bytes(const SsmShape& s) {
    // the state-group kernels read a packed fp32 copy of B/C; the lane-group kernels need nothing
    return impl_choice() == 3 ? v3_bcp_bytes(s) : 0;
}

size_t bwd_workspace_bytes(const SsmShape& s) {
    const int ngrp = impl_choice() == 3 ? v3_groups(s) : bwd_groups(s, choose_spl(s.batch * s.dim));
    size_t n = fwd_workspace_bytes(s);
    n += align256((size_t)ngrp * s.batch * s.seqlen * 32 * sizeof(float));  // dB/dC partials
    n += align256((size_t)s.batch * s.dim * kNState * sizeof(float));         // dA partials
    n += align256((size_t)s.batch * s.dim * sizeof(float));                   // dD partials
    return n;
}

}  // namespace mwc

extern "C" {

int mwc_abi_version(void) { return MWC_ABI_VERSION; }

const char* mwc_status_string(int status) {
    switch (status) {
        case MWC_OK: return "MWC_OK";
        case MWC_ERR_INVALID_ARGUMENT: return "MWC_ERR_INVALID_ARGUMENT";
        case MWC_ERR_UNSUPPORTED: return "MWC_ERR_UNSUPPORTED";
        case MWC_ERR_WORKSPACE: return "MWC_ERR_WORKSPACE";
        case MWC_ERR_HIP: return "MWC_ERR_HIP";
        default: return "MWC_ERR_UNKNOWN";
    }
}

const char* mwc_last_error(void) { return g_err; }

int64_t mwc_ssm_ckpt_count(int64_t seqlen) {
    return seqlen <= 0 ? 0 : (seqlen + mwc::kCkptSteps - 1) / mwc::kCkptSteps;
}

size_t mwc_ssm_fwd_workspace_size(int64_t batch, int64_t seqlen, int64_t dim, int64_t dstate) {
    (void)dstate;
    return mwc::fwd_workspace_bytes({batch, seqlen, dim});
}

size_t mwc_ssm_bwd_workspace_size(int64_t batch, int64_t seqlen, int64_t dim, int64_t dstate) {
    (void)dstate;
    return mwc::bwd_workspace_bytes({batch, seqlen, dim});
}

int mwc_ssm_fwd(int dtype, const void* u, const void* delta, const void* A, const void* B_ssm, const void* C_ssm,
                const void* D_ssm, const void* h_prev, void* out, void* h_last, float* ckpt, int64_t batch,
                int64_t seqlen, int64_t dim, int64_t dstate, void* workspace, size_t workspace_bytes,
                void* stream) {
    g_err[0] = 0;
    if (int st = check_dims(dtype, batch, seqlen, dim, dstate)) return st;
    if (batch == 0 || dim == 0) return MWC_OK;
    if (!A || !D_ssm) return fail(MWC_ERR_INVALID_ARGUMENT, "A and D_ssm must not be NULL");
    if (seqlen > 0 && (!u || !delta || !B_ssm || !C_ssm))
        return fail(MWC_ERR_INVALID_ARGUMENT, "u, delta, B_ssm and C_ssm must not be NULL");
    const mwc::SsmShape s{batch, seqlen, dim};
    const bool half = dtype == MWC_DTYPE_F16;
    hipStream_t st = (hipStream_t)stream;
    if (mwc::impl_choice() == 3) {
        const size_t need = mwc::fwd_workspace_bytes(s);
        if (seqlen > 0 && (workspace == nullptr || workspace_bytes < need))
            return fail(MWC_ERR_WORKSPACE, "forward workspace too small: need %zu bytes, got %zu", need,
                        workspace_bytes);
        float* bcp = (float*)workspace;
        if (seqlen > 0) MWC_HIP_TRY(mwc::launch_v3_pack(half, B_ssm, C_ssm, bcp, s, st));
        MWC_HIP_TRY(mwc::launch_v3_fwd(half, u, delta, A, bcp, D_ssm, h_prev, out, h_last, ckpt, s, st));
        return MWC_OK;
    }
    const int spl = mwc::choose_spl(batch * dim);
    MWC_HIP_TRY(mwc::launch_ssm_fwd(half, spl, u, delta, A, B_ssm, C_ssm, D_ssm, h_prev, out, h_last, ckpt, s, st));
    return MWC_OK;
}

int mwc_ssm_bwd(int dtype, const void* u, const void* delta, const void* A, const void* B_ssm, const void* C_ssm,
                const void* D_ssm, const void* h_prev, const void* dout, const void* dh_last, const float* ckpt,
                void* du, void* ddelta, void* dA, void* dB, void* dC, void* dD, void* dh_prev, int64_t batch,
                int64_t seqlen, int64_t dim, int64_t dstate, void* workspace, size_t workspace_bytes,
                void* stream) {
    g_err[0] = 0;
    (void)h_prev;  // the checkpoints already carry h_prev (checkpoint 0)
    if (int st = check_dims(dtype, batch, seqlen, dim, dstate)) return st;
    if (batch == 0 || dim == 0) return MWC_OK;
    if (!A || !D_ssm || !dA || !dD) return fail(MWC_ERR_INVALID_ARGUMENT, "A, D_ssm, dA and dD must not be NULL");
    if (seqlen > 0 && (!u || !delta || !B_ssm || !C_ssm || !dout || !ckpt || !du || !ddelta || !dB || !dC))
        return fail(MWC_ERR_INVALID_ARGUMENT,
                    "u, delta, B_ssm, C_ssm, dout, ckpt, du, ddelta, dB and dC must not be NULL");
    const mwc::SsmShape s{batch, seqlen, dim};
    const size_t need = mwc::bwd_workspace_bytes(s);
    if (workspace == nullptr || workspace_bytes < need)
        return fail(MWC_ERR_WORKSPACE, "backward workspace too small: need %zu bytes, got %zu", need, workspace_bytes);
    const bool half = dtype == MWC_DTYPE_F16;
    hipStream_t st = (hipStream_t)stream;
    const bool v3 = mwc::impl_choice() == 3;
    const int spl = mwc::choose_spl(batch * dim);
    const int ngrp = v3 ? mwc::v3_groups(s) : mwc::bwd_groups(s, spl);
    char* w = (char*)workspace;
    float* bcp = (float*)w;
    w += mwc::fwd_workspace_bytes(s);
    float* dbc_part = (float*)w;
    w += align256((size_t)ngrp * batch * seqlen * 32 * sizeof(float));
    float* dA_part = (float*)w;
    w += align256((size_t)batch * dim * mwc::kNState * sizeof(float));
    float* dD_part = (float*)w;
    if (v3) {
        if (seqlen > 0) MWC_HIP_TRY(mwc::launch_v3_pack(half, B_ssm, C_ssm, bcp, s, st));
        MWC_HIP_TRY(mwc::launch_v3_bwd(half, u, delta, A, bcp, D_ssm, dout, dh_last, ckpt, du, ddelta, dh_prev,
                                       dA_part, dD_part, dbc_part, s, st));
    } else {
        MWC_HIP_TRY(mwc::launch_ssm_bwd(half, spl, u, delta, A, B_ssm, C_ssm, D_ssm, dout, dh_last, ckpt, du,
                                        ddelta, dh_prev, dA_part, dD_part, dbc_part, s, st));
    }
    MWC_HIP_TRY(mwc::launch_bwd_finish(half, dbc_part, dA_part, dD_part, dB, dC, dA, dD, ngrp, s, st));
    return MWC_OK;
}

size_t mwc_pscan_workspace_size(int64_t nseq, int64_t seqlen, int64_t ncols) {
    return mwc::pscan_workspace_bytes(nseq, seqlen, ncols);
}

static int check_pscan(int dtype, int64_t nseq, int64_t seqlen, int64_t ncols) {
    if (dtype != MWC_DTYPE_F32 && dtype != MWC_DTYPE_F16)
        return fail(MWC_ERR_INVALID_ARGUMENT, "dtype must be MWC_DTYPE_F32 or MWC_DTYPE_F16 (got %d)", dtype);
    if (nseq < 0 || seqlen < 0 || ncols < 0)
        return fail(MWC_ERR_INVALID_ARGUMENT, "negative size (nseq=%lld, seqlen=%lld, ncols=%lld)", (long long)nseq,
                    (long long)seqlen, (long long)ncols);
    if (nseq > INT32_MAX / 2 || seqlen > INT32_MAX / 2 || ncols > INT32_MAX / 2)
        return fail(MWC_ERR_UNSUPPORTED, "sizes beyond the supported range");
    return MWC_OK;
}

int mwc_pscan_fwd(int dtype, const void* A, const void* X, void* H, int64_t nseq, int64_t seqlen, int64_t ncols,
                  void* workspace, size_t workspace_bytes, void* stream) {
    g_err[0] = 0;
    if (int st = check_pscan(dtype, nseq, seqlen, ncols)) return st;
    if (nseq == 0 || seqlen == 0 || ncols == 0) return MWC_OK;
    if (!A || !X || !H) return fail(MWC_ERR_INVALID_ARGUMENT, "A, X and H must not be NULL");
    const size_t need = mwc::pscan_workspace_bytes(nseq, seqlen, ncols);
    if (need && (workspace == nullptr || workspace_bytes < need))
        return fail(MWC_ERR_WORKSPACE, "scan workspace too small: need %zu bytes, got %zu", need, workspace_bytes);
    MWC_HIP_TRY(mwc::launch_pscan_fwd(dtype == MWC_DTYPE_F16, A, X, H, nseq, seqlen, ncols, workspace,
                                      (hipStream_t)stream));
    return MWC_OK;
}

int mwc_pscan_bwd(int dtype, const void* A, const void* H, const void* dH, void* dA, void* dX, int64_t nseq,
                  int64_t seqlen, int64_t ncols, void* workspace, size_t workspace_bytes, void* stream) {
    g_err[0] = 0;
    if (int st = check_pscan(dtype, nseq, seqlen, ncols)) return st;
    if (nseq == 0 || seqlen == 0 || ncols == 0) return MWC_OK;
    if (!A || !H || !dH || !dA || !dX) return fail(MWC_ERR_INVALID_ARGUMENT, "A, H, dH, dA and dX must not be NULL");
    const size_t need = mwc::pscan_workspace_bytes(nseq, seqlen, ncols);
    if (need && (workspace == nullptr || workspace_bytes < need))
        return fail(MWC_ERR_WORKSPACE, "scan workspace too small: need %zu bytes, got %zu", need, workspace_bytes);
    MWC_HIP_TRY(mwc::launch_pscan_bwd(dtype == MWC_DTYPE_F16, A, H, dH, dA, dX, nseq, seqlen, ncols, workspace,
                                      (hipStream_t)stream));
    return MWC_OK;
}

}  // extern "C"
