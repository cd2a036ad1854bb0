// PyTorch operators over the C ABI: the eager host path of SelectiveScanCuda / FusedSelectiveScan
// (mamba_cuda.py:1172-1219, selective_scan_cuda_ext.py:636-677) in C++. The reference validates
// and launches from C++ too (its pybind functions, mamba_cuda.py:185-238 and 281-326); here the
// argument checks keep its TORCH_CHECK messages, outputs and workspace come from the torch caching
// allocator, the kernels of libmwc_ssm.so are enqueued on the current HIP stream, and the gradient
// is a C++ autograd Function, so no Python runs per call besides the operator call itself.
//
//   torch.ops.mwc.ssm_scan(u, delta, A, B_ssm, C_ssm, D_ssm, h_prev=None, checkpoint_lvl=0,
//                          z=None, delta_bias=None, delta_softplus=False) -> (out, h_last)
//   torch.ops.mwc.ssm_step(u, delta, A, B_ssm, C_ssm, D_ssm, h, z=None, delta_bias=None,
//                          delta_softplus=False, out_state=None) -> (out, h_new)   (decode, inference)
//
// checkpoint_lvl 0 keeps the forward's fp32 state checkpoints (every 16 steps) for the backward; 1
// keeps only the inputs and rebuilds them with a state-only forward pass in the backward. Nothing
// is kept when no input needs a gradient. The backward returns the exact adjoint, with dh_prev when
// h_prev is given, and dz / ddelta_bias for the fused transforms.
#include <ATen/ATen.h>
#include <ATen/hip/impl/HIPGuardImplMasqueradingAsCUDA.h>
#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>
#include <torch/autograd.h>
#include <torch/library.h>

#include <algorithm>
#include <optional>
#include <sstream>
#include <tuple>

#include "mwc_ssm.h"

namespace {

using at::Tensor;
using OptT = std::optional<Tensor>;
using torch::autograd::AutogradContext;
using torch::autograd::variable_list;

int dtype_code(const Tensor& t) {
    switch (t.scalar_type()) {
        case at::kHalf: return MWC_DTYPE_F16;
        case at::kBFloat16: return MWC_DTYPE_BF16;
        default: return MWC_DTYPE_F32;
    }
}

void check_status(int st, const char* what) {
    TORCH_CHECK(st == MWC_OK, what, ": ", mwc_status_string(st), ": ", mwc_last_error());
}

void* ptr(const Tensor& t) { return t.defined() ? t.data_ptr() : nullptr; }

// torch on ROCm gives HIP devices the CUDA device type, so its guard and stream accessors for them
// are the "masquerading" ones
hipStream_t stream_of(const Tensor& t) {
    return c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(t.device().index()).stream();
}

std::string shape_str(at::IntArrayRef s) {  // as Python prints a shape tuple: (3,) or (2, 5, 3)
    std::ostringstream o;
    o << '(';
    for (size_t i = 0; i < s.size(); ++i) o << (i ? ", " : "") << s[i];
    o << (s.size() == 1 ? ",)" : ")");
    return o.str();
}

bool last_dim_contiguous(const Tensor& t) { return t.dim() == 0 || t.stride(-1) == 1 || t.size(-1) == 1; }

// The reference's input contract (mamba_cuda.py:281-326; N widened to 8, 16, 32, 64, bf16 storage
// accepted), with the same messages.
// require_device = false skips the device-type checks (the contract can then be exercised with host
// tensors).
void check_ssm_inputs(const Tensor& u, const Tensor& delta, const Tensor& A, const Tensor& B, const Tensor& C,
                      const Tensor& D, const OptT& h_prev, bool require_device = true) {
    const std::pair<const char*, const Tensor*> named[] = {{"u", &u}, {"delta", &delta}, {"A", &A},
                                                           {"B_ssm", &B}, {"C_ssm", &C}, {"D_ssm", &D}};
    if (require_device)
        for (const auto& [name, t] : named) TORCH_CHECK(t->is_cuda(), name, " must be a CUDA tensor");
    const auto dt = u.scalar_type();
    TORCH_CHECK(dt == at::kFloat || dt == at::kHalf || dt == at::kBFloat16, "u must be float32/float16 (or bfloat16)");
    for (size_t i = 1; i < 6; ++i)
        TORCH_CHECK(named[i].second->scalar_type() == dt, named[i].first, " dtype must match u dtype");
    for (const auto& [name, t] : named) TORCH_CHECK(last_dim_contiguous(*t), name, " must be contiguous in the last dimension");
    TORCH_CHECK(A.dim() == 2, "A must be 2D (dim, state)");
    const int64_t n = A.size(1);
    TORCH_CHECK(n == 8 || n == 16 || n == 32 || n == 64, "Only N=16 (or 8, 32, 64) is supported");
    TORCH_CHECK(u.dim() == 3, "u must be 3D (batch, seqlen, dim)");
    TORCH_CHECK(delta.dim() == 3, "delta must be 3D (batch, seqlen, dim)");
    TORCH_CHECK(B.dim() == 3, "B_ssm must be 3D (batch, seqlen, state)");
    TORCH_CHECK(C.dim() == 3, "C_ssm must be 3D (batch, seqlen, state)");
    TORCH_CHECK(D.dim() == 1, "D_ssm must be 1D (dim)");
    const int64_t bsz = u.size(0), L = u.size(1), dm = u.size(2);
    TORCH_CHECK(delta.sizes() == u.sizes(), "delta shape mismatch");
    TORCH_CHECK(A.size(0) == dm, "A shape mismatch");
    TORCH_CHECK(B.size(0) == bsz && B.size(1) == L && B.size(2) == n, "B_ssm shape mismatch");
    TORCH_CHECK(C.size(0) == bsz && C.size(1) == L && C.size(2) == n, "C_ssm shape mismatch");
    TORCH_CHECK(D.size(0) == dm, "D_ssm shape mismatch");
    for (size_t i = 1; i < 6; ++i)
        TORCH_CHECK(named[i].second->device() == u.device(), "all inputs must be on the same device");
    if (h_prev.has_value()) {
        const Tensor& h = *h_prev;
        TORCH_CHECK(!require_device || h.is_cuda(), "h_prev must be a CUDA tensor");
        TORCH_CHECK(h.scalar_type() == dt, "h_prev dtype must match u dtype");
        TORCH_CHECK(last_dim_contiguous(h), "h_prev must be contiguous in the last dimension");
        TORCH_CHECK(h.dim() == 3, "h_prev must be 3D (batch, dim, state)");
        TORCH_CHECK(h.size(0) == bsz && h.size(1) == dm && h.size(2) == n, "h_prev shape must be (B, D, N)");
        TORCH_CHECK(h.device() == u.device(), "h_prev must be on the same device as u");
    }
}

// delta_bias (D,) and z (B, L, D).
void check_transforms(const Tensor& u, const OptT& delta_bias, const OptT& z) {
    const std::tuple<const char*, const OptT*, std::vector<int64_t>> items[] = {
        {"delta_bias", &delta_bias, {u.size(2)}}, {"z", &z, {u.size(0), u.size(1), u.size(2)}}};
    for (const auto& [name, t, shape] : items) {
        if (!t->has_value()) continue;
        const Tensor& v = t->value();
        TORCH_CHECK(v.device() == u.device(), name, " must be on the same device as u");
        TORCH_CHECK(v.scalar_type() == u.scalar_type(), name, " dtype must match u dtype");
        TORCH_CHECK(v.sizes() == at::IntArrayRef(shape), name, " shape must be ", shape_str(shape));
    }
}

Tensor contig(const OptT& t) { return t.has_value() ? t->contiguous() : Tensor(); }

struct FwdOut {
    Tensor out, out_ungated, h_last, ckpt;
};

// mwc_ssm_fwd_ex on contiguous copies of the inputs. `out` is the gated
// output when z is given, out_ungated the scan's own output (with z and want_ungated).
FwdOut fwd_raw(const Tensor& u_, const Tensor& delta_, const Tensor& A_, const Tensor& B_, const Tensor& C_,
               const Tensor& D_, const OptT& h_prev_, const OptT& delta_bias_, bool softplus, const OptT& z_,
               bool want_out, bool want_ungated, bool want_h_last, bool want_ckpt) {
    check_ssm_inputs(u_, delta_, A_, B_, C_, D_, h_prev_);
    check_transforms(u_, delta_bias_, z_);
    const Tensor u = u_.contiguous(), delta = delta_.contiguous(), A = A_.contiguous(), B = B_.contiguous(),
                 C = C_.contiguous(), D = D_.contiguous();
    const Tensor h_prev = contig(h_prev_), delta_bias = contig(delta_bias_), z = contig(z_);
    const int64_t bsz = u.size(0), L = u.size(1), dm = u.size(2), n = A.size(1);
    const bool gated = z.defined();
    c10::hip::HIPGuardMasqueradingAsCUDA guard(u.device());
    FwdOut r;
    Tensor out = (want_out && !gated) || (gated && want_ungated) ? at::empty_like(u) : Tensor();
    Tensor out_z = gated && want_out ? at::empty_like(u) : Tensor();
    if (want_h_last) r.h_last = at::empty({bsz, dm, n}, u.options());
    if (want_ckpt) r.ckpt = at::empty({bsz, mwc_ssm_ckpt_count(L), dm, n}, u.options().dtype(at::kFloat));
    const size_t nbytes = mwc_ssm_fwd_workspace_size(bsz, L, dm, n);
    const Tensor ws = at::empty({(int64_t)std::max<size_t>(nbytes, 1)}, u.options().dtype(at::kByte));
    check_status(mwc_ssm_fwd_ex(dtype_code(u), ptr(u), ptr(delta), ptr(A), ptr(B), ptr(C), ptr(D), ptr(h_prev),
                                ptr(delta_bias), softplus ? 1 : 0, ptr(z), ptr(out), ptr(out_z), ptr(r.h_last),
                                static_cast<float*>(ptr(r.ckpt)), bsz, L, dm, n, ws.data_ptr(), nbytes, stream_of(u)),
                 "mwc_ssm_fwd_ex");
    r.out = gated ? out_z : out;
    r.out_ungated = gated ? out : Tensor();
    return r;
}

struct BwdOut {
    Tensor du, ddelta, dA, dB, dC, dD, dh_prev, dbias, dz;
};

// mwc_ssm_bwd_ex: dout and dh_last in u's dtype, the checkpoints of the
// same inputs, the ungated forward output when z is given.
BwdOut bwd_raw(const Tensor& u_, const Tensor& delta_, const Tensor& A_, const Tensor& B_, const Tensor& C_,
               const Tensor& D_, const Tensor& dout_, const Tensor& ckpt, const Tensor& dh_last_, bool want_dh_prev,
               const OptT& delta_bias_, bool softplus, const OptT& z_, const Tensor& out_ungated_) {
    check_ssm_inputs(u_, delta_, A_, B_, C_, D_, std::nullopt);
    const Tensor u = u_.contiguous(), delta = delta_.contiguous(), A = A_.contiguous(), B = B_.contiguous(),
                 C = C_.contiguous(), D = D_.contiguous();
    const int64_t bsz = u.size(0), L = u.size(1), dm = u.size(2), n = A.size(1);
    // every operand the kernels read must live on u's device
    for (const auto& [name, t] : {std::pair<const char*, const Tensor*>{"dout", &dout_}, {"dh_last", &dh_last_},
                                  {"ckpt", &ckpt}, {"out_ungated", &out_ungated_}})
        TORCH_CHECK(!t->defined() || t->device() == u_.device(), name, " must be on the same device as u");
    const Tensor dout = dout_.to(u.scalar_type()).contiguous();
    TORCH_CHECK(dout.sizes() == u.sizes(), "dout shape mismatch");
    Tensor dh_last;
    if (dh_last_.defined()) {
        dh_last = dh_last_.to(u.scalar_type()).contiguous();
        TORCH_CHECK(dh_last.dim() == 3 && dh_last.size(0) == bsz && dh_last.size(1) == dm && dh_last.size(2) == n,
                    "dh_last shape must be (B, D, N)");
    }
    TORCH_CHECK(ckpt.defined() && ckpt.scalar_type() == at::kFloat && ckpt.is_contiguous() && ckpt.dim() == 4 &&
                    ckpt.size(0) == bsz && ckpt.size(1) == mwc_ssm_ckpt_count(L) && ckpt.size(2) == dm &&
                    ckpt.size(3) == n,
                "ckpt does not match the inputs");
    check_transforms(u, delta_bias_, z_);
    const Tensor delta_bias = contig(delta_bias_), z = contig(z_);
    Tensor out_ungated;
    if (z.defined()) {
        TORCH_CHECK(out_ungated_.defined() && out_ungated_.sizes() == u.sizes(),
                    "the ungated forward output is needed with z");
        out_ungated = out_ungated_.to(u.scalar_type()).contiguous();
    }
    c10::hip::HIPGuardMasqueradingAsCUDA guard(u.device());
    BwdOut g;
    g.du = at::empty_like(u);
    g.ddelta = at::empty_like(u);
    g.dA = at::empty_like(A);
    g.dB = at::empty_like(B);
    g.dC = at::empty_like(C);
    g.dD = at::empty_like(D);
    if (want_dh_prev) g.dh_prev = at::empty({bsz, dm, n}, u.options());
    if (delta_bias.defined()) g.dbias = at::empty_like(delta_bias);
    if (z.defined()) g.dz = at::empty_like(z);
    const size_t nbytes = mwc_ssm_bwd_workspace_size(bsz, L, dm, n);
    const Tensor ws = at::empty({(int64_t)std::max<size_t>(nbytes, 1)}, u.options().dtype(at::kByte));
    check_status(mwc_ssm_bwd_ex(dtype_code(u), ptr(u), ptr(delta), ptr(A), ptr(B), ptr(C), ptr(D), nullptr,
                                ptr(delta_bias), softplus ? 1 : 0, ptr(z), ptr(out_ungated), ptr(dout), ptr(dh_last),
                                static_cast<const float*>(ptr(ckpt)), ptr(g.du), ptr(g.ddelta), ptr(g.dA), ptr(g.dB),
                                ptr(g.dC), ptr(g.dD), ptr(g.dbias), ptr(g.dz), ptr(g.dh_prev), bsz, L, dm, n,
                                ws.data_ptr(), nbytes, stream_of(u)),
                 "mwc_ssm_bwd_ex");
    return g;
}

void check_level(int64_t lvl) { TORCH_CHECK(lvl == 0 || lvl == 1, "checkpoint_lvl must be 0 or 1 (got ", lvl, ")"); }

// Saved-tensor slots of the autograd Function.
enum Saved { kU, kDelta, kA, kB, kC, kD, kHprev, kCkpt, kZ, kBias, kUngated, kNSaved };

struct ScanFunction : public torch::autograd::Function<ScanFunction> {
    static variable_list forward(AutogradContext* ctx, const Tensor& u, const Tensor& delta, const Tensor& A,
                                 const Tensor& B, const Tensor& C, const Tensor& D, const OptT& h_prev,
                                 int64_t lvl, const OptT& z, const OptT& delta_bias, bool softplus) {
        check_level(lvl);
        FwdOut r = fwd_raw(u, delta, A, B, C, D, h_prev, delta_bias, softplus, z, true, z.has_value(), true, lvl == 0);
        ctx->save_for_backward({u, delta, A, B, C, D, h_prev.value_or(Tensor()), r.ckpt, z.value_or(Tensor()),
                                delta_bias.value_or(Tensor()), r.out_ungated});
        ctx->saved_data["softplus"] = softplus;
        ctx->saved_data["h_prev_edge"] = h_prev.has_value() ? int64_t(6) : int64_t(-1);
        ctx->set_materialize_grads(false);
        return {r.out, r.h_last};
    }

    static variable_list backward(AutogradContext* ctx, variable_list grads) {
        const variable_list s = ctx->get_saved_variables();
        const bool softplus = ctx->saved_data["softplus"].toBool();
        const int64_t h_edge = ctx->saved_data["h_prev_edge"].toInt();
        const OptT h_prev = s[kHprev].defined() ? OptT(s[kHprev]) : std::nullopt;
        const OptT z = s[kZ].defined() ? OptT(s[kZ]) : std::nullopt;
        const OptT bias = s[kBias].defined() ? OptT(s[kBias]) : std::nullopt;
        Tensor ckpt = s[kCkpt], ungated = s[kUngated];
        if (!ckpt.defined()) {  // recompute level: rebuild the checkpoints (and the ungated output for dz)
            FwdOut r = fwd_raw(s[kU], s[kDelta], s[kA], s[kB], s[kC], s[kD], h_prev, bias, softplus, z, false,
                               z.has_value(), false, true);
            ckpt = r.ckpt;
            ungated = r.out_ungated;
        }
        const Tensor dout = grads[0].defined() ? grads[0] : at::zeros_like(s[kU]);
        const bool want_dh_prev = h_edge >= 0 && ctx->needs_input_grad(h_edge);
        BwdOut g = bwd_raw(s[kU], s[kDelta], s[kA], s[kB], s[kC], s[kD], dout, ckpt, grads[1], want_dh_prev, bias,
                           softplus, z, ungated);
        // one entry per forward argument: u, delta, A, B, C, D, h_prev, checkpoint_lvl, z, delta_bias, softplus
        return {g.du, g.ddelta, g.dA, g.dB, g.dC, g.dD, g.dh_prev, Tensor(), g.dz, g.dbias, Tensor()};
    }
};

// Without gradients (grad mode off, or no input requiring one) nothing is kept for a backward.
std::tuple<Tensor, Tensor> scan_nograd(const Tensor& u, const Tensor& delta, const Tensor& A, const Tensor& B,
                                       const Tensor& C, const Tensor& D, const OptT& h_prev, int64_t lvl, const OptT& z,
                                       const OptT& delta_bias, bool softplus) {
    check_level(lvl);
    FwdOut r = fwd_raw(u, delta, A, B, C, D, h_prev, delta_bias, softplus, z, true, false, true, false);
    return {r.out, r.h_last};
}

std::tuple<Tensor, Tensor> scan_autograd(const Tensor& u, const Tensor& delta, const Tensor& A, const Tensor& B,
                                         const Tensor& C, const Tensor& D, const OptT& h_prev, int64_t lvl,
                                         const OptT& z, const OptT& delta_bias, bool softplus) {
    bool need_grad = false;
    if (at::GradMode::is_enabled()) {
        for (const Tensor* t : {&u, &delta, &A, &B, &C, &D}) need_grad = need_grad || t->requires_grad();
        for (const OptT* t : {&h_prev, &z, &delta_bias}) need_grad = need_grad || (t->has_value() && (*t)->requires_grad());
    }
    if (!need_grad) return scan_nograd(u, delta, A, B, C, D, h_prev, lvl, z, delta_bias, softplus);
    variable_list r = ScanFunction::apply(u, delta, A, B, C, D, h_prev, lvl, z, delta_bias, softplus);
    return {r[0], r[1]};
}

// The raw operators behind ops.py (the Python host path of the reference-named autograd Functions):
// no autograd of their own, outputs that a call does not ask for come back as None.
void check_inputs_op(const Tensor& u, const Tensor& delta, const Tensor& A, const Tensor& B, const Tensor& C,
                     const Tensor& D, const OptT& h_prev, bool require_device) {
    check_ssm_inputs(u, delta, A, B, C, D, h_prev, require_device);
}

void check_transforms_op(const Tensor& u, const OptT& delta_bias, const OptT& z) {
    TORCH_CHECK(u.dim() == 3, "u must be 3D (batch, seqlen, dim)");
    check_transforms(u, delta_bias, z);
}

std::tuple<Tensor, Tensor, Tensor, Tensor> fwd_op(const Tensor& u, const Tensor& delta, const Tensor& A,
                                                  const Tensor& B, const Tensor& C, const Tensor& D,
                                                  const OptT& h_prev, const OptT& delta_bias, bool softplus,
                                                  const OptT& z, bool want_out, bool want_ungated, bool want_h_last,
                                                  bool want_ckpt) {
    FwdOut r = fwd_raw(u, delta, A, B, C, D, h_prev, delta_bias, softplus, z, want_out, want_ungated, want_h_last,
                       want_ckpt);
    return {r.out, r.out_ungated, r.h_last, r.ckpt};
}

using Grads9 = std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor>;

Grads9 bwd_op(const Tensor& u, const Tensor& delta, const Tensor& A, const Tensor& B, const Tensor& C, const Tensor& D,
              const Tensor& dout, const OptT& ckpt, const OptT& dh_last, bool want_dh_prev, const OptT& delta_bias,
              bool softplus, const OptT& z, const OptT& out_ungated) {
    BwdOut g = bwd_raw(u, delta, A, B, C, D, dout, ckpt.value_or(Tensor()), dh_last.value_or(Tensor()), want_dh_prev,
                       delta_bias, softplus, z, out_ungated.value_or(Tensor()));
    return {g.du, g.ddelta, g.dA, g.dB, g.dC, g.dD, g.dh_prev, g.dbias, g.dz};
}

// One decode step: u, delta, z (B, D); A (D, N); B_ssm, C_ssm (B, N); D_ssm (D,);
// h (B, D, N). Returns (out (B, D), gated by silu(z) when z is given, h_new); out_state, when given,
// receives h_new and may be h itself (an in-place update). Inference only.
std::tuple<Tensor, Tensor> step_impl(const Tensor& u_, const Tensor& delta_, const Tensor& A_, const Tensor& B_,
                                     const Tensor& C_, const Tensor& D_, const Tensor& h_, const OptT& z_,
                                     const OptT& delta_bias_, bool softplus, const OptT& out_state) {
    const std::pair<const char*, const Tensor*> named[] = {{"u", &u_}, {"delta", &delta_}, {"A", &A_}, {"B_ssm", &B_},
                                                           {"C_ssm", &C_}, {"D_ssm", &D_}, {"h", &h_}};
    for (const auto& [name, t] : named) {
        TORCH_CHECK(t->is_cuda(), name, " must be a CUDA tensor");
        TORCH_CHECK(t->scalar_type() == u_.scalar_type(), name, " dtype must match u dtype");
    }
    const auto dt = u_.scalar_type();
    TORCH_CHECK(dt == at::kFloat || dt == at::kHalf || dt == at::kBFloat16, "u must be float32/float16 (or bfloat16)");
    TORCH_CHECK(u_.dim() == 2, "u must be 2D (batch, dim) for a step");
    const int64_t bsz = u_.size(0), dm = u_.size(1);
    TORCH_CHECK(A_.dim() == 2 && (A_.size(1) == 8 || A_.size(1) == 16 || A_.size(1) == 32 || A_.size(1) == 64),
                "Only N=16 (or 8, 32, 64) is supported");
    const int64_t n = A_.size(1);
    const std::tuple<const char*, const Tensor*, std::vector<int64_t>> shaped[] = {
        {"delta", &delta_, {bsz, dm}}, {"A", &A_, {dm, n}}, {"B_ssm", &B_, {bsz, n}}, {"C_ssm", &C_, {bsz, n}},
        {"D_ssm", &D_, {dm}}, {"h", &h_, {bsz, dm, n}},
        {"delta_bias", delta_bias_.has_value() ? &*delta_bias_ : nullptr, {dm}},
        {"z", z_.has_value() ? &*z_ : nullptr, {bsz, dm}}};
    for (const auto& [name, t, shape] : shaped) {
        if (t == nullptr) continue;
        TORCH_CHECK(t->sizes() == at::IntArrayRef(shape), name, " shape must be ", shape_str(shape));
        TORCH_CHECK(t->scalar_type() == dt && t->device() == u_.device(), name, " must match u's dtype and device");
    }
    // the kernel moves a lane's states as one 16-byte vector
    auto aligned = [](const Tensor& t) {
        Tensor c = t.contiguous();
        return reinterpret_cast<uintptr_t>(c.data_ptr()) % 16 == 0 ? c : c.clone();
    };
    const Tensor u = u_.contiguous(), delta = delta_.contiguous(), D = D_.contiguous();
    const Tensor A = aligned(A_), B = aligned(B_), C = aligned(C_), h = aligned(h_);
    const Tensor delta_bias = contig(delta_bias_), z = contig(z_);
    Tensor h_new = out_state.has_value() ? *out_state : at::empty_like(h);
    TORCH_CHECK(h_new.device() == u_.device() && h_new.is_contiguous() && h_new.dim() == 3 && h_new.size(0) == bsz &&
                    h_new.size(1) == dm && h_new.size(2) == n && h_new.scalar_type() == dt &&
                    reinterpret_cast<uintptr_t>(h_new.data_ptr()) % 16 == 0,
                "out_state must be a contiguous, 16-byte-aligned (B, D, N) tensor of u's dtype and device");
    c10::hip::HIPGuardMasqueradingAsCUDA guard(u.device());
    const Tensor out = at::empty_like(u);
    check_status(mwc_ssm_step(dtype_code(u), ptr(u), ptr(delta), ptr(A), ptr(B), ptr(C), ptr(D), ptr(h),
                              ptr(delta_bias), softplus ? 1 : 0, ptr(z), z.defined() ? nullptr : ptr(out),
                              z.defined() ? ptr(out) : nullptr, ptr(h_new), bsz, dm, n, stream_of(u)),
                 "mwc_ssm_step");
    // the kernel wrote out_state through a raw pointer: bump its version counter as an in-place op
    // would, so autograd sees the overwrite of a state some other op saved (the op is eager-only: no
    // Meta kernel or aliasing information for functionalization / torch.compile)
    if (out_state.has_value()) torch::autograd::impl::bump_version(*out_state);
    return {out, h_new};
}

std::tuple<Tensor, Tensor> step_autograd(const Tensor& u, const Tensor& delta, const Tensor& A, const Tensor& B,
                                         const Tensor& C, const Tensor& D, const Tensor& h, const OptT& z,
                                         const OptT& delta_bias, bool softplus, const OptT& out_state) {
    if (at::GradMode::is_enabled()) {
        bool req = false;
        for (const Tensor* t : {&u, &delta, &A, &B, &C, &D, &h}) req = req || t->requires_grad();
        for (const OptT* t : {&z, &delta_bias}) req = req || (t->has_value() && (*t)->requires_grad());
        TORCH_CHECK(!req, "SelectiveScanCuda.step is inference-only; use forward_with_state for gradients");
    }
    return step_impl(u, delta, A, B, C, D, h, z, delta_bias, softplus, out_state);
}

}  // namespace

TORCH_LIBRARY(mwc, m) {
    m.def("ssm_scan(Tensor u, Tensor delta, Tensor A, Tensor B_ssm, Tensor C_ssm, Tensor D_ssm, Tensor? h_prev=None, "
          "int checkpoint_lvl=0, Tensor? z=None, Tensor? delta_bias=None, bool delta_softplus=False) -> (Tensor, Tensor)");
    m.def("check_ssm_inputs(Tensor u, Tensor delta, Tensor A, Tensor B_ssm, Tensor C_ssm, Tensor D_ssm, "
          "Tensor? h_prev=None, bool require_device=True) -> ()");
    m.def("check_transforms(Tensor u, Tensor? delta_bias=None, Tensor? z=None) -> ()");
    m.def("ssm_fwd(Tensor u, Tensor delta, Tensor A, Tensor B_ssm, Tensor C_ssm, Tensor D_ssm, Tensor? h_prev, "
          "Tensor? delta_bias, bool delta_softplus, Tensor? z, bool want_out, bool want_ungated, bool want_h_last, "
          "bool want_ckpt) -> (Tensor, Tensor, Tensor, Tensor)");
    m.def("ssm_bwd(Tensor u, Tensor delta, Tensor A, Tensor B_ssm, Tensor C_ssm, Tensor D_ssm, Tensor dout, "
          "Tensor? ckpt, Tensor? dh_last, bool want_dh_prev, Tensor? delta_bias, bool delta_softplus, Tensor? z, "
          "Tensor? out_ungated) -> (Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor)");
    m.def("ssm_step(Tensor u, Tensor delta, Tensor A, Tensor B_ssm, Tensor C_ssm, Tensor D_ssm, Tensor h, "
          "Tensor? z=None, Tensor? delta_bias=None, bool delta_softplus=False, Tensor(a!)? out_state=None) "
          "-> (Tensor, Tensor)");
}

// the raw operators run below autograd on every backend (host tensors reach the checks and are refused)
TORCH_LIBRARY_IMPL(mwc, CompositeImplicitAutograd, m) {
    m.impl("check_ssm_inputs", &check_inputs_op);
    m.impl("check_transforms", &check_transforms_op);
    m.impl("ssm_fwd", &fwd_op);
    m.impl("ssm_bwd", &bwd_op);
}

TORCH_LIBRARY_IMPL(mwc, Autograd, m) {
    m.impl("ssm_scan", &scan_autograd);
    m.impl("ssm_step", &step_autograd);
}
// HIP tensors carry torch's CUDA dispatch key; host tensors reach the same checks and are refused.
TORCH_LIBRARY_IMPL(mwc, CUDA, m) {
    m.impl("ssm_scan", &scan_nograd);
    m.impl("ssm_step", &step_impl);
}
TORCH_LIBRARY_IMPL(mwc, CPU, m) {
    m.impl("ssm_scan", &scan_nograd);
    m.impl("ssm_step", &step_impl);
}
