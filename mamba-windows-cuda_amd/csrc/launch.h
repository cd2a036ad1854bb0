// Internal launcher interface between the C ABI (capi.hip) and the kernel files.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mwc {

struct SsmShape {
    int64_t batch, seqlen, dim;
};

// Channel-grouping choice: SPL = states held per lane (4 lanes x 4 states per
// channel by default). Returns 1, 2 or 4.
int choose_spl(int64_t channels);

// Workspace carve-up (bytes, 256-aligned pieces).
size_t fwd_workspace_bytes(const SsmShape& s);
size_t bwd_workspace_bytes(const SsmShape& s);
int bwd_groups(const SsmShape& s, int spl);  // channel groups that write dB/dC partials

// Kernel launchers; `is_half` selects fp16 storage. They only enqueue work.
hipError_t launch_ssm_fwd(bool is_half, int spl, const void* u, const void* delta, const void* A,
                          const void* B, const void* C, const void* Dv, const void* h_prev, void* out,
                          void* h_last, float* ckpt, const SsmShape& s, hipStream_t st);
hipError_t launch_ssm_bwd(bool is_half, int spl, const void* u, const void* delta, const void* A,
                          const void* B, const void* C, const void* Dv, const void* dout, const void* dh_last,
                          const float* ckpt, void* du, void* ddelta, void* dh_prev, float* dA_part,
                          float* dD_part, float* dbc_part, const SsmShape& s, hipStream_t st);
hipError_t launch_bwd_finish(bool is_half, const float* dbc_part, const float* dA_part,
                             const float* dD_part, void* dB, void* dC, void* dA, void* dD,
                             int ngroups, const SsmShape& s, hipStream_t st);

// "state groups across waves" kernels (ssm_v3.hip)
int impl_choice();  // 2 = lane groups (default), 3 = state groups across waves
size_t v3_bcp_bytes(const SsmShape& s);
int v3_groups(const SsmShape& s);
hipError_t launch_v3_pack(bool is_half, const void* B, const void* C, float* bcp, const SsmShape& s,
                          hipStream_t st);
hipError_t launch_v3_fwd(bool is_half, const void* u, const void* delta, const void* A, const float* bcp,
                         const void* Dv, const void* h_prev, void* out, void* h_last, float* ckpt,
                         const SsmShape& s, hipStream_t st);
hipError_t launch_v3_bwd(bool is_half, const void* u, const void* delta, const void* A, const float* bcp,
                         const void* Dv, const void* dout, const void* dh_last, const float* ckpt, void* du,
                         void* ddelta, void* dh_prev, float* dA_part, float* dD_part, float* dbc_part,
                         const SsmShape& s, hipStream_t st);

hipError_t launch_pscan_fwd(bool is_half, const void* A, const void* X, void* H, int64_t nseq,
                            int64_t seqlen, int64_t ncols, void* ws, hipStream_t st);
hipError_t launch_pscan_bwd(bool is_half, const void* A, const void* H, const void* dH, void* dA,
                            void* dX, int64_t nseq, int64_t seqlen, int64_t ncols, void* ws,
                            hipStream_t st);
size_t pscan_workspace_bytes(int64_t nseq, int64_t seqlen, int64_t ncols);

// Grid helper: map hardware block ids so that consecutive logical blocks run on
// the same XCD (the dispatcher deals block i to XCD i % 8), which keeps blocks
// sharing cache lines inside one XCD's L2.
__device__ __forceinline__ int xcd_remap(int bid, int nblocks) {
    constexpr int kXcd = 8;
    if (nblocks % kXcd != 0) return bid;
    return (bid % kXcd) * (nblocks / kXcd) + bid / kXcd;
}

}  // namespace mwc
