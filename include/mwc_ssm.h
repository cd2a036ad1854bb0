/*
 * mwc_ssm.h -- C ABI of the MI355X (gfx950) selective-scan engine.
 *
 * Drop-in boundary for the native layer of zouyuanqing/mamba-windows-cuda.
 * The reference binds its CUDA code through pybind/load_inline
 * (mamba_windows_cuda/mamba_cuda.py:793-830, 862-871;
 * mamba_windows_cuda/selective_scan_cuda_ext.py:517-528, 551-558); here the
 * same operations are plain extern "C" functions over device pointers, so any
 * FFI (ctypes in mamba_windows_cuda/_lib.py) can bind them.
 *
 * Conventions
 *  - Every pointer is a device pointer on the current HIP device, C-contiguous
 *    in the reference's layouts: u, delta, out, dout, du, ddelta (B,L,D);
 *    A, dA (D,N); B_ssm, C_ssm, dB, dC (B,L,N); D_ssm, dD (D,);
 *    h_prev, h_last, dh_last, dh_prev (B,D,N).
 *  - dtype selects the element type of every tensor argument: MWC_DTYPE_F32
 *    (float), MWC_DTYPE_F16 (IEEE binary16) or MWC_DTYPE_BF16 (bfloat16; not in
 *    the reference, which rejects it). Arithmetic is fp32 throughout; fp16 and
 *    bf16 are storage only, rounded to nearest-even on store (the reference's
 *    load_to_float/store_from_float, mamba_cuda.py:72-90).
 *  - N (dstate) must be 16 (mamba_cuda.py:215) or, not in the reference, 8, 32
 *    or 64.
 *  - Work is enqueued on `stream` (a hipStream_t; NULL = default stream);
 *    nothing synchronises the host. The library never allocates device
 *    memory: scratch space comes from the caller through `workspace`, whose
 *    required size the *_workspace_size functions return.
 *  - Return value: MWC_OK or an mwc_status; mwc_last_error() gives a message
 *    for the calling thread's last failure. Argument errors are detected
 *    before any device work is enqueued.
 */
#ifndef MWC_SSM_H
#define MWC_SSM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MWC_ABI_VERSION 1
/* Steps between the fp32 state checkpoints written by the forward and read by
 * the backward. */
#define MWC_CKPT_STEPS 16

enum mwc_dtype { MWC_DTYPE_F32 = 0, MWC_DTYPE_F16 = 1, MWC_DTYPE_BF16 = 2 };

enum mwc_status {
    MWC_OK = 0,
    MWC_ERR_INVALID_ARGUMENT = 1, /* shape/pointer/dtype contract violated */
    MWC_ERR_UNSUPPORTED = 2,      /* valid request the build does not handle */
    MWC_ERR_WORKSPACE = 3,        /* workspace missing or too small */
    MWC_ERR_HIP = 4,              /* a HIP runtime call failed */
    MWC_ERR_INCOMPLETE = 5        /* device work gave up a bounded wait; its results are NaN */
};

/* Library version (MWC_ABI_VERSION). */
int mwc_abi_version(void);

/* Human-readable name of a status code. */
const char* mwc_status_string(int status);

/* Message describing the calling thread's most recent failure ("" if none). */
const char* mwc_last_error(void);

/* Number of checkpoints for a sequence of `seqlen` steps: ceil(seqlen / MWC_CKPT_STEPS). */
int64_t mwc_ssm_ckpt_count(int64_t seqlen);

/* Workspace bytes needed by mwc_ssm_fwd for these sizes (0 when the sequence is not split into
 * segments; otherwise the segment carries). dim is limited to 2^24, batch*dim to 2^31 and
 * batch*seqlen to 2^33; for sizes the entry points reject it returns 0 and sets mwc_last_error(). */
size_t mwc_ssm_fwd_workspace_size(int64_t batch, int64_t seqlen, int64_t dim, int64_t dstate);

/*
 * Fused forward: dA = exp(clamp(delta*A, -88, 88)); h_t = dA*h_{t-1} + delta*u*B;
 * out = sum_n C*h + D*u; h_{-1} = h_prev (zeros when NULL); h_last = h_{L-1}.
 *
 * Replaces selective_scan_cuda_forward (mamba_cuda.py:176-269),
 * selective_scan_cuda_forward_with_state (mamba_cuda.py:271-359),
 * selective_scan_cuda_forward_store (mamba_cuda.py:747-764) and
 * fused_selective_scan_forward (selective_scan_cuda_ext.py:389-452).
 *
 * out     may be NULL (state-only pass, used to regenerate checkpoints).
 * h_last  may be NULL.
 * ckpt    may be NULL; otherwise fp32 [batch][mwc_ssm_ckpt_count(seqlen)][dim][N]
 *         receiving the state before steps 0, 16, 32, ... (checkpoint 0 = h_prev).
 */
int mwc_ssm_fwd(int dtype, const void* u, const void* delta, const void* A, const void* B_ssm,
                const void* C_ssm, const void* D_ssm, const void* h_prev, void* out, void* h_last,
                float* ckpt, int64_t batch, int64_t seqlen, int64_t dim, int64_t dstate,
                void* workspace, size_t workspace_bytes, void* stream);

/*
 * mwc_ssm_fwd with the elementwise transforms a Mamba block applies around the scan, fused into
 * the scan's loads and stores (no reference counterpart: the reference rejects them; they are the
 * delta_bias / delta_softplus / z options of the official Mamba selective scan):
 *   delta' = softplus(delta + delta_bias)   (delta_bias (dim,) may be NULL; delta_softplus 0/1)
 *   out    = the scan of delta' (as mwc_ssm_fwd)          may be NULL
 *   out_z  = out * silu(z)                  (z (batch, seqlen, dim) may be NULL; then out_z NULL;
 *                                            out_z may be NULL with z, e.g. to rebuild checkpoints)
 * Checkpoints, workspace and the other arguments are as for mwc_ssm_fwd.
 */
int mwc_ssm_fwd_ex(int dtype, const void* u, const void* delta, const void* A, const void* B_ssm,
                   const void* C_ssm, const void* D_ssm, const void* h_prev, const void* delta_bias,
                   int delta_softplus, const void* z, void* out, void* out_z, void* h_last, float* ckpt,
                   int64_t batch, int64_t seqlen, int64_t dim, int64_t dstate, void* workspace,
                   size_t workspace_bytes, void* stream);

/*
 * mwc_ssm_fwd_ex without a workspace argument: it allocates nothing and takes no workspace, for
 * callers that cannot allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid allocation). No counterpart in the reference. The segment carries that
 * mwc_ssm_fwd_ex keeps in its workspace live in a static device array of MWC_NOALLOC_SCRATCH_BYTES
 * per GPU (held until the process ends); sizes whose carries need more (mwc_ssm_fwd_workspace_size)
 * return MWC_ERR_UNSUPPORTED before anything is enqueued. Calls that overlap on one GPU share that
 * array and race: serialise them (one stream, or events). Results equal mwc_ssm_fwd_ex's bitwise.
 */
#define MWC_NOALLOC_SCRATCH_BYTES ((size_t)32 << 20)
int mwc_ssm_fwd_noalloc(int dtype, const void* u, const void* delta, const void* A, const void* B_ssm,
                        const void* C_ssm, const void* D_ssm, const void* h_prev, const void* delta_bias,
                        int delta_softplus, const void* z, void* out, void* out_z, void* h_last, float* ckpt,
                        int64_t batch, int64_t seqlen, int64_t dim, int64_t dstate, void* stream);

/* Workspace bytes needed by mwc_ssm_bwd for these sizes (0, with mwc_last_error() set, for sizes
 * the entry points reject). */
size_t mwc_ssm_bwd_workspace_size(int64_t batch, int64_t seqlen, int64_t dim, int64_t dstate);

/*
 * Fused backward of mwc_ssm_fwd given dout (and dh_last, zeros when NULL):
 * du, ddelta (B,L,D); dA (D,N); dB, dC (B,L,N); dD (D,); dh_prev (B,D,N) when
 * not NULL. All gradients are accumulated in fp32 and stored in `dtype`.
 * `ckpt` must hold the checkpoints mwc_ssm_fwd wrote for the same inputs and
 * h_prev. Reductions are deterministic (fixed order, no atomics).
 *
 * Replaces selective_scan_cuda_backward (mamba_cuda.py:564-604),
 * selective_scan_cuda_backward_direct (mamba_cuda.py:766-790), the Python
 * stateful backward selective_scan_backward (mamba_cuda.py:949-1041) and
 * selective_scan_backward (selective_scan_cuda_ext.py:454-514).
 */
int mwc_ssm_bwd(int dtype, const void* u, const void* delta, const void* A, const void* B_ssm,
                const void* C_ssm, const void* D_ssm, const void* h_prev, const void* dout,
                const void* dh_last, const float* ckpt, void* du, void* ddelta, void* dA, void* dB,
                void* dC, void* dD, void* dh_prev, int64_t batch, int64_t seqlen, int64_t dim,
                int64_t dstate, void* workspace, size_t workspace_bytes, void* stream);

/*
 * The adjoint of mwc_ssm_fwd_ex (no reference counterpart, see there). With z, `out` is the ungated
 * forward output (mwc_ssm_fwd_ex's `out`) and dout the gradient of out_z; dz receives
 * dout * out * silu'(z). ddelta is the gradient of the raw delta (through the bias and softplus),
 * ddelta_bias (dim,) the gradient of delta_bias (may be NULL). Checkpoints (from mwc_ssm_fwd_ex with
 * the same transforms), workspace and the other arguments are as for mwc_ssm_bwd.
 */
int mwc_ssm_bwd_ex(int dtype, const void* u, const void* delta, const void* A, const void* B_ssm,
                   const void* C_ssm, const void* D_ssm, const void* h_prev, const void* delta_bias,
                   int delta_softplus, const void* z, const void* out, const void* dout, const void* dh_last,
                   const float* ckpt, void* du, void* ddelta, void* dA, void* dB, void* dC, void* dD,
                   void* ddelta_bias, void* dz, void* dh_prev, int64_t batch, int64_t seqlen, int64_t dim,
                   int64_t dstate, void* workspace, size_t workspace_bytes, void* stream);

/*
 * One decode step (inference): mwc_ssm_fwd_ex at seqlen 1 with the state carried in and out, in a
 * batched layout without the length axis:
 *   u, delta, z, out, out_z (batch, dim); B_ssm, C_ssm (batch, N); h, h_new (batch, dim, N).
 * h_new may alias h (in-place update). out may be NULL; out_z must be given with z (and only then).
 * A, B_ssm, C_ssm, h and h_new must be aligned to 16 bytes.
 * Replaces selective_scan_cuda_forward_with_state (mamba_cuda.py:271-359) called with seqlen 1,
 * the reference's only way to advance one step; needs no workspace.
 */
int mwc_ssm_step(int dtype, const void* u, const void* delta, const void* A, const void* B_ssm, const void* C_ssm,
                 const void* D_ssm, const void* h, const void* delta_bias, int delta_softplus, const void* z,
                 void* out, void* out_z, void* h_new, int64_t batch, int64_t dim, int64_t dstate, void* stream);

/* Workspace bytes needed by mwc_pscan_fwd / mwc_pscan_bwd for these sizes. */
size_t mwc_pscan_workspace_size(int64_t nseq, int64_t seqlen, int64_t ncols);

/*
 * Linear recurrence over the middle axis of [nseq][seqlen][ncols] tensors:
 * H_0 = X_0 (A_0 unused); H_t = A_t*H_{t-1} + X_t. fp32 accumulation.
 * Replaces PScan.forward (pscan.py:74-95) behind parallel_scan_fn
 * (pscan.py:139-150), with the semantics of parallel_scan_ref (pscan.py:153-171).
 */
int mwc_pscan_fwd(int dtype, const void* A, const void* X, void* H, int64_t nseq, int64_t seqlen,
                  int64_t ncols, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Adjoint of mwc_pscan_fwd: G_t = dH_t + A_{t+1}*G_{t+1}; dX = G;
 * dA_t = G_t*H_{t-1} (t >= 1), dA_0 = 0. Replaces PScan.backward (pscan.py:97-136).
 */
int mwc_pscan_bwd(int dtype, const void* A, const void* H, const void* dH, void* dA, void* dX,
                  int64_t nseq, int64_t seqlen, int64_t ncols, void* workspace,
                  size_t workspace_bytes, void* stream);

/*
 * Outcome of the last mwc_pscan_fwd / mwc_pscan_bwd that used `workspace` with these sizes: waits
 * for `stream`, then returns MWC_OK, or MWC_ERR_INCOMPLETE if a bounded look-back wait between
 * tiles ran out (the affected outputs are then NaN, never a silently wrong value). No reference
 * counterpart: the reference's PScan (pscan.py:16-136) runs elementwise torch ops with no waits.
 */
int mwc_pscan_status(const void* workspace, size_t workspace_bytes, int64_t nseq, int64_t seqlen,
                     int64_t ncols, void* stream);

/*
 * The same outcome without waiting: enqueues on `stream` a copy of the scan's status word into
 * `*host_word` (pinned host memory, so the copy does not block the caller) and returns. Once the
 * stream has passed that point, *host_word is 0 if every wait completed and non-zero if one gave
 * up (MWC_ERR_INCOMPLETE). No reference counterpart, as mwc_pscan_status.
 */
int mwc_pscan_status_async(const void* workspace, size_t workspace_bytes, int64_t nseq, int64_t seqlen,
                           int64_t ncols, uint32_t* host_word, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MWC_SSM_H */
