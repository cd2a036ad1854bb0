// extern "C" entry points declared in include/mwc_ssm.h.
//
// Argument validation restates the reference host wrappers' contract
// (mamba_cuda.py:185-238, 281-326: N = 16, fp32/fp16, consistent shapes), widened
// to N = 8, 32, 64 and bf16 storage. Everything is checked before the first
// launch; the functions only enqueue work on the caller's stream and never
// allocate.
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>

#include <algorithm>
#include <atomic>
#include <mutex>

#include "common.h"
#include "launch.h"

namespace {

thread_local char g_err[512] = "";

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

int spl_override() {
    const char* e = getenv("MWC_SPL");
    if (!e) return 0;
    const int s = atoi(e);
    return (s == 1 || s == 2 || s == 4) ? s : 0;
}

int fail(int status, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return status;
}

int check_dims(int dtype, int64_t batch, int64_t seqlen, int64_t dim, int64_t dstate) {
    if (dtype != MWC_DTYPE_F32 && dtype != MWC_DTYPE_F16 && dtype != MWC_DTYPE_BF16)
        return fail(MWC_ERR_INVALID_ARGUMENT, "dtype must be MWC_DTYPE_F32, MWC_DTYPE_F16 or MWC_DTYPE_BF16 (got %d)",
                    dtype);
    if (dstate != 8 && dstate != 16 && dstate != 32 && dstate != 64)
        return fail(MWC_ERR_INVALID_ARGUMENT, "Only N=16 (or 8, 32, 64) is supported (got N=%lld)", (long long)dstate);
    if (batch < 0 || seqlen < 0 || dim < 0)
        return fail(MWC_ERR_INVALID_ARGUMENT, "negative size (batch=%lld, seqlen=%lld, dim=%lld)", (long long)batch,
                    (long long)seqlen, (long long)dim);
    // the launchers count workgroups (rows of channels, rows of the dB/dC partials) in 32-bit ints
    if (seqlen > INT32_MAX / 2 || dim > (int64_t(1) << 24) || batch > 65535 || batch * dim > (int64_t(1) << 31) ||
        batch * seqlen > (int64_t(1) << 33))
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

// States per lane. Measured on MI355X at B=8, L=2048, D=1536, fp16 fwd+bwd step: at N=16, SPL=2 (8
// lanes per channel, 0.389 ms) beats SPL=1 (0.464 ms: twice the per-lane overhead of the n-reductions)
// and SPL=4 (one wave per SIMD); at N=32, SPL=2 takes 0.751 ms and SPL=4 0.966 ms (its forward needs
// 267 VGPRs, one wave per SIMD); at N=8, SPL=2 takes 0.293 ms and SPL=1 0.330 ms. N=64 is built at
// SPL=4 only. Small problems use 16 lanes per channel, for parallelism.
int choose_spl(int64_t channels, int ns) {
    const int o = spl_override();
    if (o && lane_group_supported(ns, o)) return o;
    if (ns == 64) return 4;
    if (channels >= 2048) return 2;
    return ns / 16 < 1 ? 1 : ns / 16;
}

bool lane_group_supported(int ns, int spl) {
#define MWC_LG(N, S) \
    if (ns == N && spl == S) return true;
    MWC_FOR_EACH_LANE_GROUP(MWC_LG)
#undef MWC_LG
    return false;
}

namespace {

constexpr int kCUs = 256;  // MI355X compute units (4 SIMDs each); a workgroup is 4 waves on one CU

int env_int(const char* name, int lo, int hi) {
    const char* e = getenv(name);
    if (!e) return 0;
    const int v = atoi(e);
    return (v >= lo && v <= hi) ? v : 0;
}

// Relative throughput of a SIMD running q of these waves at once. Measured with the main kernels at
// 2 states per lane, B=8, L=2048, one segment and D = 1024, 2048, 3072 (1, 2, 3 workgroups per CU):
// 1 : 1.65-1.7 : 2.0 for the forward and the backward. Four or more waves (the carry passes, one
// state per lane) keep earlier estimates.
double simd_throughput(int64_t q) {
    static const double t[] = {0.0, 1.0, 1.7, 2.0, 2.3};
    return q < 5 ? t[q] : 2.4;
}

// Duration, in units of one chunk of one lone wave, of a pass of `wgs` equal workgroups of
// `chunks` chunks each when a CU holds at most `cap` of them at once: full rounds of `cap`, then
// a last round as deep as its busiest CU. (Counting the rounds one after the other matches the
// measured plans; an earlier 4% discount for grids of several rounds overrated split plans.)
double pass_time(int64_t wgs, int64_t chunks, int cap) {
    if (wgs <= 0 || chunks <= 0) return 0.0;
    const int64_t full = wgs / (kCUs * cap);
    const int64_t rem = wgs - full * kCUs * cap;
    double t = (double)full * ((double)chunks * cap / simd_throughput(cap) + 1.0);  // +1: prologue, first loads
    if (rem > 0) {
        const int64_t q = (rem + kCUs - 1) / kCUs;
        t += (double)chunks * q / simd_throughput(q) + 1.0;
    }
    return t;
}

int cpb_of(int ns, int spl) { return 4 * 64 / (ns / spl); }

constexpr int kMinSegChunks = 8;  // shortest (carry) segment the fill and partly split plans make

// Picks the segment count (and the carry split) minimising the modelled time of carry pass + main
// pass. caps = workgroups per CU each kernel fits (registers, LDS); carry_rel = cost of a carry-pass
// chunk relative to a main-pass chunk.
SegPlan plan(const SsmShape& s, bool bwd, int spl, int cap_main, int cap_carry, double carry_rel,
             double* t_out = nullptr) {
    const int64_t nck = (s.seqlen + kCkptSteps - 1) / kCkptSteps;
    const int64_t w1 = s.batch * ((s.dim + cpb_of(s.nstate, spl) - 1) / cpb_of(s.nstate, spl));
    SegPlan best{spl, 1, (int)nck, 1, 0};
    double best_t = pass_time(w1, nck, cap_main);
    // MWC_NSEG / MWC_CFOLD force the segment count / carry split (tuning and tests)
    const int force_n = env_int("MWC_NSEG", 1, 1 << 20), force_f = env_int("MWC_CFOLD", 1, 64);
    if (force_n == 1 || nck < 2) {
        if (t_out) *t_out = best_t;
        return best;
    }
    const int n_lo = force_n ? force_n : 2, n_hi = force_n ? force_n : 16;
    for (int n = n_lo; n <= n_hi; ++n) {
        // finer carry splits first: they are measured as fast or faster than the model says
        for (int f = force_f ? force_f : 4; f >= (force_f ? force_f : 1); f /= 2) {
            const int64_t cps = ((nck + n - 1) / n + f - 1) / f * f;  // chunks per segment, a multiple of f
            const int64_t nseg = (nck + cps - 1) / cps;                 // non-empty segments
            if (nseg < 2) continue;
            const int64_t ccps = cps / f;
            const int64_t ncar = bwd ? (nck - cps + ccps - 1) / ccps : (nseg - 1) * f;
            const double t = pass_time(w1 * nseg, cps, cap_main) + carry_rel * pass_time(w1 * ncar, ccps, cap_carry);
            if (t < best_t * 0.98 || force_n) {
                best_t = t;
                best = SegPlan{spl, (int)nseg, (int)cps, f, (int)ncar};
            }
        }
    }
    if (t_out) *t_out = best_t;
    return best;
}

// Partly split plans: only some rows are split into two segments (and need carries); the others run
// whole. Two cases, with slots = cap * CUs workgroups in one round:
// - rows between slots - CUs and slots (one round in which some CUs are one workgroup short of their
//   cap): x = slots - rows split rows make the grid fill one round, each CU running cap - 1 whole rows
//   and one half. The halves finish at half time and the CU then runs cap - 1 workgroups to the end,
//   instead of the busiest CUs running cap whole rows throughout;
// - rows = m full rounds plus r <= slots / 2 more (m >= 1): an unsplit grid's last round runs r whole
//   rows on a part-empty chip. Splitting just those x = r rows puts m rounds of whole rows first (the
//   whole rows come first in the block order) and the 2r halves in one last round of half length.
// `x_forced` (MWC_NSPLIT) sets x for tests; returns nseg = 0 when no such plan applies. *t_out receives
// the modelled time.
SegPlan split_plan(const SsmShape& s, bool bwd, int spl, int cap_main, int cap_carry, double carry_rel, int x_forced,
                   double* t_out) {
    const int64_t nck = (s.seqlen + kCkptSteps - 1) / kCkptSteps;
    const int64_t rows = s.batch * ((s.dim + cpb_of(s.nstate, spl) - 1) / cpb_of(s.nstate, spl));
    const int64_t slots = (int64_t)kCUs * cap_main;
    const int64_t m = rows / slots, r = rows - m * slots;
    const bool one_round = m == 0;
    const SegPlan none{spl, 0, 0, 0, 0};
    int64_t x = x_forced;
    if (x_forced <= 0) {
        if (one_round) {
            if (rows <= slots - kCUs || 2 * rows - slots > (int64_t)kCUs * (cap_main - 1)) return none;
            x = slots - rows;
        } else {
            if (r == 0 || 2 * r > slots) return none;
            x = r;
        }
    }
    if (nck < 2 || x < 1 || x >= rows) return none;
    for (int f = 8; f >= 1; f /= 2) {
        const int64_t cps = ((nck + 1) / 2 + f - 1) / f * f;
        const int64_t ccps = cps / f;
        if ((nck + cps - 1) / cps != 2) continue;
        if (f > 1 && (ccps < kMinSegChunks || x * f > (int64_t)kCUs * cap_carry)) continue;
        const int64_t ncar = bwd ? (nck - cps + ccps - 1) / ccps : f;
        const double carry = carry_rel * pass_time(x * ncar, ccps, cap_carry);
        // one round: a CU with cap - 1 whole rows and one half runs all cap until the half ends, then
        // cap - 1; several rounds: the whole rows' rounds, then the halves'
        const double t = one_round && x == slots - rows
                             ? (double)cps * cap_main / simd_throughput(cap_main) +
                                   (double)(nck - cps) * (cap_main - 1) / simd_throughput(cap_main - 1) + 1.0 + carry
                             : pass_time(rows - x, nck, cap_main) + pass_time(2 * x, cps, cap_main) + carry;
        if (t_out) *t_out = t;
        return SegPlan{spl, 2, (int)cps, f, (int)ncar, (int)(rows - x)};
    }
    return none;
}

// Workgroups per CU each kernel fits: the runtime's occupancy query for the instance (registers and LDS
// of the gfx950 build), or, when no device can be queried, min(512 / VGPRs, 160 KiB / LDS) of the
// N=16 instances.
int cap_or(int queried, int fallback) { return queried > 0 ? queried : fallback; }
int fwd_cap(int ns, int spl) { return cap_or(fwd_wgs_per_cu(ns, spl, 0), spl == 1 ? 7 : spl == 2 ? 3 : 1); }
int fwd_carry_cap(int ns, int spl) { return cap_or(fwd_wgs_per_cu(ns, spl, 2), spl == 1 ? 8 : spl == 2 ? 6 : 4); }
int bwd_cap(int ns, int spl) { return cap_or(bwd_wgs_per_cu(ns, spl, false), spl == 1 ? 4 : spl == 2 ? 3 : 1); }
int bwd_carry_cap(int ns, int spl) { return cap_or(bwd_wgs_per_cu(ns, spl, true), spl == 1 ? 8 : spl == 2 ? 6 : 4); }

size_t carry_bytes(const SsmShape& s, const SegPlan& p) {
    return p.nseg > 1 ? align256((size_t)s.batch * p.ncar * s.dim * s.nstate * sizeof(float)) : 0;
}

// Small problems at N=16 (an unsplit two-states-per-lane grid fills under 1.5 waves per SIMD). Measured
// sweeps of every (states per lane, segments, carry split) at B=8, L=2048 and D = 192, 384, 768 (fp16,
// interleaved event timing) put the fastest plan of each shape, forward and backward alike, at two
// states per lane with exactly one round of full CUs (segments = cap x CUs / workgroups per segment) and
// the most carry segments that keep each at least 8 chunks long and the carry grid in one round (the
// planner's cost model picked shorter segments and finer carry splits there: 8-12% slower). Where two
// states per lane cannot fill 2.25 workgroups per CU with segments of at least 8 chunks, the cost model
// above decides, at choose_spl's states per lane.
bool small_problem(const SsmShape& s) {
    return s.nstate == 16 && s.batch * ((s.dim + cpb_of(16, 2) - 1) / cpb_of(16, 2)) < (int64_t)kCUs * 3 / 2;
}

// The one-round plan at `spl` states per lane, or nseg = 0 when it does not fill the chip
SegPlan fill_plan(const SsmShape& s, bool bwd, int spl, int cap_main, int cap_carry) {
    const int64_t nck = (s.seqlen + kCkptSteps - 1) / kCkptSteps;
    const int64_t w1 = s.batch * ((s.dim + cpb_of(s.nstate, spl) - 1) / cpb_of(s.nstate, spl));
    if (w1 <= 0) return SegPlan{spl, 0, 0, 0, 0};  // nothing to launch (empty batch or channels)
    int64_t n = std::min<int64_t>((int64_t)kCUs * cap_main / w1, nck / kMinSegChunks);
    if (n < 2 || w1 * n * 4 < (int64_t)kCUs * cap_main * 3) return SegPlan{spl, 0, 0, 0, 0};
    for (int f = 8; f >= 1; f /= 2) {
        const int64_t cps = ((nck + n - 1) / n + f - 1) / f * f;
        const int64_t nseg = (nck + cps - 1) / cps;
        const int64_t ccps = cps / f;
        const int64_t ncar = bwd ? (nck - cps + ccps - 1) / ccps : (nseg - 1) * f;
        if (nseg < 2) continue;
        if (f > 1 && (ccps < kMinSegChunks || w1 * ncar > (int64_t)kCUs * cap_carry)) continue;
        return SegPlan{spl, (int)nseg, (int)cps, f, (int)ncar};
    }
    return SegPlan{spl, 0, 0, 0, 0};
}

SegPlan plan_dir(const SsmShape& s, bool bwd) {
    auto caps = [&](int spl, int& cm, int& cc) {
        cm = bwd ? bwd_cap(s.nstate, spl) : fwd_cap(s.nstate, spl);
        cc = bwd ? bwd_carry_cap(s.nstate, spl) : fwd_carry_cap(s.nstate, spl);
    };
    int cm = 0, cc = 0;
    const int o = spl_override();
    const bool forced = env_int("MWC_NSEG", 1, 1 << 20) || env_int("MWC_CFOLD", 1, 64);
    if (small_problem(s) && !forced && (o == 0 || o == 2)) {
        caps(2, cm, cc);
        const SegPlan p = fill_plan(s, bwd, 2, cm, cc);
        if (p.nseg > 0) return p;
    }
    const int spl = choose_spl(s.batch * s.dim, s.nstate);
    caps(spl, cm, cc);
    const double rel = bwd ? 0.3 : 0.75;
    const char* e = getenv("MWC_NSPLIT");
    const int x_forced = e ? atoi(e) : -1;  // MWC_NSPLIT=0 turns partly split plans off
    double t = 0.0, th = 0.0;
    const SegPlan p = plan(s, bwd, spl, cm, cc, rel, &t);
    if (x_forced == 0 || (forced && x_forced < 0)) return p;
    // the one-round case competes with an unsplit uniform plan only; the several-rounds case with any
    const int64_t rows = s.batch * ((s.dim + cpb_of(s.nstate, spl) - 1) / cpb_of(s.nstate, spl));
    if (p.nseg > 1 && x_forced < 0 && rows < (int64_t)kCUs * cm) return p;
    const SegPlan h = split_plan(s, bwd, spl, cm, cc, rel, x_forced, &th);
    return h.nseg > 0 && (x_forced > 0 || th < t * 0.98) ? h : p;
}

}  // namespace

SegPlan plan_fwd(const SsmShape& s) { return plan_dir(s, false); }

SegPlan plan_bwd(const SsmShape& s) { return plan_dir(s, true); }

size_t fwd_workspace_bytes(const SsmShape& s) {
    // the segment carries when L is split
    return 2 * carry_bytes(s, plan_fwd(s));
}

size_t bwd_workspace_bytes(const SsmShape& s) {
    const SegPlan p = plan_bwd(s);
    size_t n = align256((size_t)bwd_groups(s, s.nstate, p.spl) * s.batch * s.seqlen * 2 * s.nstate *
                        sizeof(float));                                                          // dB/dC
    n += align256((size_t)p.nseg * s.batch * s.dim * s.nstate * sizeof(float));                  // dA
    n += align256((size_t)p.nseg * s.batch * s.dim * sizeof(float));                                // dD
    n += align256((size_t)p.nseg * s.batch * s.dim * sizeof(float));                                // d bias
    n += 2 * carry_bytes(s, p);
    return n;
}

}  // namespace mwc

// Scratch of mwc_ssm_fwd_noalloc: the forward's segment carries (h_end and the summed decay exponents
// of every carry segment, fp32), for callers that cannot allocate. Each GPU the library runs on holds
// its own copy until the process ends. The carry pass writes every value the main pass reads, so
// nothing needs clearing; calls that overlap on one GPU share it and race.
namespace {
constexpr size_t kScratchBytes = MWC_NOALLOC_SCRATCH_BYTES;
constexpr int kMaxDevices = 64;
__device__ __align__(256) unsigned char scratch[kScratchBytes];
std::mutex g_scratch_mu;
std::atomic<void*> g_scratch_ptr[kMaxDevices];

// The current device's address of `scratch` (the symbol's name is only a host-side stand-in), looked
// up once per device with that device current and kept for later calls.
int device_scratch(void** out) {
    int dev = -1;
    MWC_HIP_TRY(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxDevices) return fail(MWC_ERR_UNSUPPORTED, "device index %d beyond %d", dev, kMaxDevices);
    void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
    if (p == nullptr) {
        std::lock_guard<std::mutex> lock(g_scratch_mu);
        p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
        if (p == nullptr) {
            MWC_HIP_TRY(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
            if (p == nullptr) return fail(MWC_ERR_HIP, "hipGetSymbolAddress(scratch) returned NULL");
            g_scratch_ptr[dev].store(p, std::memory_order_release);
        }
    }
    *out = p;
    return MWC_OK;
}
}  // namespace

extern "C" {

int mwc_abi_version(void) { return MWC_ABI_VERSION; }

const char* mwc_status_string(int status) {
    switch (status) {
        case MWC_OK: return "MWC_OK";
        case MWC_ERR_INVALID_ARGUMENT: return "MWC_ERR_INVALID_ARGUMENT";
        case MWC_ERR_UNSUPPORTED: return "MWC_ERR_UNSUPPORTED";
        case MWC_ERR_WORKSPACE: return "MWC_ERR_WORKSPACE";
        case MWC_ERR_HIP: return "MWC_ERR_HIP";
        case MWC_ERR_INCOMPLETE: return "MWC_ERR_INCOMPLETE";
        default: return "MWC_ERR_UNKNOWN";
    }
}

const char* mwc_last_error(void) { return g_err; }

int64_t mwc_ssm_ckpt_count(int64_t seqlen) {
    return seqlen <= 0 ? 0 : (seqlen + mwc::kCkptSteps - 1) / mwc::kCkptSteps;
}

// Sizes the entry points would reject need no workspace: 0, with the reason in mwc_last_error().
size_t mwc_ssm_fwd_workspace_size(int64_t batch, int64_t seqlen, int64_t dim, int64_t dstate) {
    if (check_dims(MWC_DTYPE_F32, batch, seqlen, dim, dstate) != MWC_OK) return 0;
    return mwc::fwd_workspace_bytes({batch, seqlen, dim, (int)dstate});
}

size_t mwc_ssm_bwd_workspace_size(int64_t batch, int64_t seqlen, int64_t dim, int64_t dstate) {
    if (check_dims(MWC_DTYPE_F32, batch, seqlen, dim, dstate) != MWC_OK) return 0;
    return mwc::bwd_workspace_bytes({batch, seqlen, dim, (int)dstate});
}

// The forward's one body: validation, workspace check and launch. With `scratch_only`, the segment
// carries live in this device's static scratch array (mwc_ssm_fwd_noalloc) instead of a caller
// workspace; sizes whose carries exceed it are rejected before anything is enqueued.
static int fwd_impl(int dtype, const void* u, const void* delta, const void* A, const void* B_ssm,
                    const void* C_ssm, const void* D_ssm, const void* h_prev, const void* delta_bias,
                    int delta_softplus, const void* z, void* out, void* out_z, void* h_last, float* ckpt,
                    int64_t batch, int64_t seqlen, int64_t dim, int64_t dstate, void* workspace,
                    size_t workspace_bytes, bool scratch_only, void* stream);

int mwc_ssm_fwd_ex(int dtype, const void* u, const void* delta, const void* A, const void* B_ssm,
                   const void* C_ssm, const void* D_ssm, const void* h_prev, const void* delta_bias,
                   int delta_softplus, const void* z, void* out, void* out_z, void* h_last, float* ckpt,
                   int64_t batch, int64_t seqlen, int64_t dim, int64_t dstate, void* workspace,
                   size_t workspace_bytes, void* stream) {
    return fwd_impl(dtype, u, delta, A, B_ssm, C_ssm, D_ssm, h_prev, delta_bias, delta_softplus, z, out, out_z,
                    h_last, ckpt, batch, seqlen, dim, dstate, workspace, workspace_bytes, false, stream);
}

int mwc_ssm_fwd_noalloc(int dtype, const void* u, const void* delta, const void* A, const void* B_ssm,
                        const void* C_ssm, const void* D_ssm, const void* h_prev, const void* delta_bias,
                        int delta_softplus, const void* z, void* out, void* out_z, void* h_last, float* ckpt,
                        int64_t batch, int64_t seqlen, int64_t dim, int64_t dstate, void* stream) {
    return fwd_impl(dtype, u, delta, A, B_ssm, C_ssm, D_ssm, h_prev, delta_bias, delta_softplus, z, out, out_z,
                    h_last, ckpt, batch, seqlen, dim, dstate, nullptr, 0, true, stream);
}

int mwc_ssm_fwd(int dtype, const void* u, const void* delta, const void* A, const void* B_ssm, const void* C_ssm,
                const void* D_ssm, const void* h_prev, void* out, void* h_last, float* ckpt, int64_t batch,
                int64_t seqlen, int64_t dim, int64_t dstate, void* workspace, size_t workspace_bytes,
                void* stream) {
    return mwc_ssm_fwd_ex(dtype, u, delta, A, B_ssm, C_ssm, D_ssm, h_prev, nullptr, 0, nullptr, out, nullptr,
                          h_last, ckpt, batch, seqlen, dim, dstate, workspace, workspace_bytes, stream);
}

static int fwd_impl(int dtype, const void* u, const void* delta, const void* A, const void* B_ssm,
                    const void* C_ssm, const void* D_ssm, const void* h_prev, const void* delta_bias,
                    int delta_softplus, const void* z, void* out, void* out_z, void* h_last, float* ckpt,
                    int64_t batch, int64_t seqlen, int64_t dim, int64_t dstate, void* workspace,
                    size_t workspace_bytes, bool scratch_only, void* stream) {
    g_err[0] = 0;
    if (int st = check_dims(dtype, batch, seqlen, dim, dstate)) return st;
    if (batch == 0 || dim == 0) return MWC_OK;
    if (!A || !D_ssm) return fail(MWC_ERR_INVALID_ARGUMENT, "A and D_ssm must not be NULL");
    if (seqlen > 0 && (!u || !delta || !B_ssm || !C_ssm))
        return fail(MWC_ERR_INVALID_ARGUMENT, "u, delta, B_ssm and C_ssm must not be NULL");
    if (z == nullptr && out_z != nullptr) return fail(MWC_ERR_INVALID_ARGUMENT, "out_z needs z");
    const mwc::SsmShape s{batch, seqlen, dim, (int)dstate};
    hipStream_t st = (hipStream_t)stream;
    const size_t need = seqlen > 0 ? mwc::fwd_workspace_bytes(s) : 0;
    if (scratch_only && need > 0) {
        if (need > kScratchBytes)
            return fail(MWC_ERR_UNSUPPORTED,
                        "mwc_ssm_fwd_noalloc: these sizes need %zu bytes of segment carries, more than its static "
                        "scratch of %zu bytes; call mwc_ssm_fwd_ex with a workspace instead",
                        need, (size_t)kScratchBytes);
        if (int e = device_scratch(&workspace)) return e;
        workspace_bytes = kScratchBytes;
    }
    if (need > 0 && (workspace == nullptr || workspace_bytes < need))
        return fail(MWC_ERR_WORKSPACE, "forward workspace too small: need %zu bytes, got %zu", need, workspace_bytes);
    const mwc::SegPlan p = mwc::plan_fwd(s);
    float* car_h = (float*)workspace;
    float* car_x = (float*)((char*)workspace + need / 2);
    const mwc::FwdArgs a{u, delta, A, B_ssm, C_ssm, D_ssm, h_prev, out, h_last, ckpt, car_h, car_x,
                         p.nseg, p.cps, p.cfold, p.ncar, mwc::ScanXf{delta_bias, z, delta_softplus != 0}, out_z,
                         p.nfull};
    MWC_HIP_TRY(mwc::launch_ssm_fwd(dtype, s.nstate, p.spl, a, s, st));
    return MWC_OK;
}

int mwc_ssm_bwd_ex(int dtype, const void* u, const void* delta, const void* A, const void* B_ssm,
                   const void* C_ssm, const void* D_ssm, const void* h_prev, const void* delta_bias,
                   int delta_softplus, const void* z, const void* out, const void* dout, const void* dh_last,
                   const float* ckpt, void* du, void* ddelta, void* dA, void* dB, void* dC, void* dD,
                   void* ddelta_bias, void* dz, void* dh_prev, int64_t batch, int64_t seqlen, int64_t dim,
                   int64_t dstate, void* workspace, size_t workspace_bytes, void* stream) {
    g_err[0] = 0;
    (void)h_prev;  // the checkpoints already carry h_prev (checkpoint 0)
    if (int st = check_dims(dtype, batch, seqlen, dim, dstate)) return st;
    if (batch == 0 || dim == 0) {
        // nothing to scan, but sums over an empty batch (dA, dD, d delta_bias) or over no channels
        // (dB, dC) are zeros: the finishing kernel writes them from zero partials
        const bool sums_d = dim > 0, sums_bl = batch > 0 && seqlen > 0;
        if (!sums_d && !sums_bl) return MWC_OK;
        if (sums_d && (!dA || !dD)) return fail(MWC_ERR_INVALID_ARGUMENT, "dA and dD must not be NULL");
        if (sums_bl && (!dB || !dC)) return fail(MWC_ERR_INVALID_ARGUMENT, "dB and dC must not be NULL");
        const mwc::SsmShape s{batch, seqlen, dim, (int)dstate};
        MWC_HIP_TRY(mwc::launch_bwd_finish(dtype, s.nstate, nullptr, nullptr, nullptr, nullptr, dB, dC, dA, dD,
                                           delta_bias != nullptr ? ddelta_bias : nullptr, 0, 0, s,
                                           (hipStream_t)stream));
        return MWC_OK;
    }
    if (!A || !D_ssm || !dA || !dD) return fail(MWC_ERR_INVALID_ARGUMENT, "A, D_ssm, dA and dD must not be NULL");
    if (seqlen > 0 && (!u || !delta || !B_ssm || !C_ssm || !dout || !ckpt || !du || !ddelta || !dB || !dC))
        return fail(MWC_ERR_INVALID_ARGUMENT,
                    "u, delta, B_ssm, C_ssm, dout, ckpt, du, ddelta, dB and dC must not be NULL");
    if (seqlen > 0 && z != nullptr && (out == nullptr || dz == nullptr))
        return fail(MWC_ERR_INVALID_ARGUMENT, "out (ungated) and dz must not be NULL when z is given");
    if (ddelta_bias != nullptr && delta_bias == nullptr)
        return fail(MWC_ERR_INVALID_ARGUMENT, "ddelta_bias needs delta_bias");
    const mwc::SsmShape s{batch, seqlen, dim, (int)dstate};
    const size_t need = mwc::bwd_workspace_bytes(s);
    if (workspace == nullptr || workspace_bytes < need)
        return fail(MWC_ERR_WORKSPACE, "backward workspace too small: need %zu bytes, got %zu", need, workspace_bytes);
    hipStream_t st = (hipStream_t)stream;
    char* w = (char*)workspace;
    const mwc::SegPlan p = mwc::plan_bwd(s);
    const int ngrp = mwc::bwd_groups(s, s.nstate, p.spl);
    float* dbc_part = (float*)w;
    w += align256((size_t)ngrp * batch * seqlen * 2 * dstate * sizeof(float));
    float* dA_part = (float*)w;
    w += align256((size_t)p.nseg * batch * dim * dstate * sizeof(float));
    float* dD_part = (float*)w;
    w += align256((size_t)p.nseg * batch * dim * sizeof(float));
    float* dbias_part = (float*)w;
    w += align256((size_t)p.nseg * batch * dim * sizeof(float));
    float* car_g = (float*)w;
    w += mwc::carry_bytes(s, p);
    float* car_x = (float*)w;
    const mwc::BwdArgs a{u, delta, A, B_ssm, C_ssm, D_ssm, dout, dh_last, ckpt, du, ddelta, dh_prev,
                         dA_part, dD_part, dbc_part, car_g, car_x, p.nseg, p.cps, p.cfold, p.ncar,
                         mwc::ScanXf{delta_bias, z, delta_softplus != 0}, out, dz, dbias_part, p.nfull};
    MWC_HIP_TRY(mwc::launch_ssm_bwd(dtype, s.nstate, p.spl, a, s, st));
    MWC_HIP_TRY(mwc::launch_bwd_finish(dtype, s.nstate, dbc_part, dA_part, dD_part, dbias_part, dB, dC, dA, dD,
                                       delta_bias != nullptr ? ddelta_bias : nullptr, ngrp, p.nseg * (int)batch, s,
                                       st));
    return MWC_OK;
}

int mwc_ssm_bwd(int dtype, const void* u, const void* delta, const void* A, const void* B_ssm, const void* C_ssm,
                const void* D_ssm, const void* h_prev, const void* dout, const void* dh_last, const float* ckpt,
                void* du, void* ddelta, void* dA, void* dB, void* dC, void* dD, void* dh_prev, int64_t batch,
                int64_t seqlen, int64_t dim, int64_t dstate, void* workspace, size_t workspace_bytes,
                void* stream) {
    return mwc_ssm_bwd_ex(dtype, u, delta, A, B_ssm, C_ssm, D_ssm, h_prev, nullptr, 0, nullptr, nullptr, dout, dh_last,
                          ckpt, du, ddelta, dA, dB, dC, dD, nullptr, nullptr, dh_prev, batch, seqlen, dim, dstate,
                          workspace, workspace_bytes, stream);
}

int mwc_ssm_step(int dtype, const void* u, const void* delta, const void* A, const void* B_ssm, const void* C_ssm,
                 const void* D_ssm, const void* h, const void* delta_bias, int delta_softplus, const void* z,
                 void* out, void* out_z, void* h_new, int64_t batch, int64_t dim, int64_t dstate, void* stream) {
    g_err[0] = 0;
    if (int st = check_dims(dtype, batch, 1, dim, dstate)) return st;
    if (batch == 0 || dim == 0) return MWC_OK;
    if (!u || !delta || !A || !B_ssm || !C_ssm || !D_ssm || !h || !h_new)
        return fail(MWC_ERR_INVALID_ARGUMENT, "u, delta, A, B_ssm, C_ssm, D_ssm, h and h_new must not be NULL");
    if (z != nullptr && out_z == nullptr) return fail(MWC_ERR_INVALID_ARGUMENT, "out_z must not be NULL when z is given");
    if (z == nullptr && out_z != nullptr) return fail(MWC_ERR_INVALID_ARGUMENT, "out_z needs z");
    const uintptr_t align = 16;  // the kernel moves a lane's states as one 16-byte vector
    for (const void* p : {A, B_ssm, C_ssm, h, static_cast<const void*>(h_new)})
        if ((uintptr_t)p % align != 0)
            return fail(MWC_ERR_INVALID_ARGUMENT, "A, B_ssm, C_ssm, h and h_new must be aligned to 16 bytes");
    MWC_HIP_TRY(mwc::launch_ssm_step(dtype, (int)dstate, u, delta, A, B_ssm, C_ssm, D_ssm, h,
                                     mwc::ScanXf{delta_bias, z, delta_softplus != 0}, out, out_z, h_new, batch, dim,
                                     (hipStream_t)stream));
    return MWC_OK;
}

size_t mwc_pscan_workspace_size(int64_t nseq, int64_t seqlen, int64_t ncols) {
    return mwc::pscan_workspace_bytes(nseq, seqlen, ncols);
}

// Bound of each look-back wait of the scan (polls). MWC_PSCAN_SPIN_LIMIT overrides it (tests force a
// give-up with 0: every wait then fails at once and every kernel still exits normally).
static unsigned pscan_spin_limit() {
    const char* e = getenv("MWC_PSCAN_SPIN_LIMIT");
    if (!e || !*e) return mwc::kPscanSpinLimit;
    const long long v = atoll(e);
    return v < 0 ? mwc::kPscanSpinLimit : (unsigned)(v > (long long)mwc::kPscanSpinLimit ? mwc::kPscanSpinLimit : v);
}

static int check_pscan(int dtype, int64_t nseq, int64_t seqlen, int64_t ncols) {
    if (dtype != MWC_DTYPE_F32 && dtype != MWC_DTYPE_F16 && dtype != MWC_DTYPE_BF16)
        return fail(MWC_ERR_INVALID_ARGUMENT, "dtype must be MWC_DTYPE_F32, MWC_DTYPE_F16 or MWC_DTYPE_BF16 (got %d)",
                    dtype);
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
    MWC_HIP_TRY(mwc::launch_pscan_fwd(dtype, A, X, H, nseq, seqlen, ncols, workspace, pscan_spin_limit(),
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
    MWC_HIP_TRY(mwc::launch_pscan_bwd(dtype, A, H, dH, dA, dX, nseq, seqlen, ncols, workspace, pscan_spin_limit(),
                                      (hipStream_t)stream));
    return MWC_OK;
}

int mwc_pscan_status(const void* workspace, size_t workspace_bytes, int64_t nseq, int64_t seqlen, int64_t ncols,
                     void* stream) {
    g_err[0] = 0;
    if (nseq <= 0 || seqlen <= 0 || ncols <= 0) return MWC_OK;  // nothing was scanned
    const size_t need = mwc::pscan_workspace_bytes(nseq, seqlen, ncols);
    if (workspace == nullptr || workspace_bytes < need)
        return fail(MWC_ERR_WORKSPACE, "scan workspace too small: need %zu bytes, got %zu", need, workspace_bytes);
    unsigned err = 0;
    hipStream_t st = (hipStream_t)stream;
    MWC_HIP_TRY(hipMemcpyAsync(&err, (const char*)workspace + mwc::pscan_error_word_offset(nseq, seqlen, ncols),
                               sizeof(err), hipMemcpyDeviceToHost, st));
    MWC_HIP_TRY(hipStreamSynchronize(st));
    if (err != 0)
        return fail(MWC_ERR_INCOMPLETE,
                    "a look-back wait of the parallel scan ran out of spins: the affected tiles' outputs are NaN");
    return MWC_OK;
}

int mwc_pscan_status_async(const void* workspace, size_t workspace_bytes, int64_t nseq, int64_t seqlen,
                           int64_t ncols, uint32_t* host_word, void* stream) {
    g_err[0] = 0;
    if (host_word == nullptr) return fail(MWC_ERR_INVALID_ARGUMENT, "host_word must not be NULL");
    if (nseq <= 0 || seqlen <= 0 || ncols <= 0) {  // nothing was scanned
        *host_word = 0;
        return MWC_OK;
    }
    const size_t need = mwc::pscan_workspace_bytes(nseq, seqlen, ncols);
    if (workspace == nullptr || workspace_bytes < need)
        return fail(MWC_ERR_WORKSPACE, "scan workspace too small: need %zu bytes, got %zu", need, workspace_bytes);
    MWC_HIP_TRY(hipMemcpyAsync(host_word, (const char*)workspace + mwc::pscan_error_word_offset(nseq, seqlen, ncols),
                               sizeof(uint32_t), hipMemcpyDeviceToHost, (hipStream_t)stream));
    return MWC_OK;
}

}  // extern "C"
