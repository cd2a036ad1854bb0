"""CPU-only checks of the C-ABI library and the host layer (no kernel launches)."""
import ctypes
import os
import re

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "mwc_ssm.h")


def _declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(mwc_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    from mamba_windows_cuda import _lib

    L = _lib.lib()
    names = _declared()
    assert len(names) >= 11
    for n in names:
        assert hasattr(L, n), n
    assert set(names) == set(_lib.EXPORTED)
    assert L.mwc_abi_version() == 1


def test_torch_operator_library_registers_ssm_scan():
    """libmwc_torch.so (the C++ host path) loads and registers torch.ops.mwc.ssm_scan with the
    reference's argument names; host tensors are refused by its checks in every dispatch mode."""
    from mamba_windows_cuda import _lib

    ops = _lib.torch_ops()
    schema = str(ops.ssm_scan.default._schema)
    for arg in ("Tensor u", "Tensor delta", "Tensor A", "Tensor B_ssm", "Tensor C_ssm", "Tensor D_ssm",
                "Tensor? h_prev=None", "int checkpoint_lvl=0", "Tensor? z=None", "Tensor? delta_bias=None",
                "bool delta_softplus=False"):
        assert arg in schema, arg
    x = _valid()
    args = [x["u"], x["delta"], x["A"], x["B_ssm"], x["C_ssm"], x["D_ssm"]]
    with pytest.raises(RuntimeError, match="u must be a CUDA tensor"):
        ops.ssm_scan(*args)
    with pytest.raises(RuntimeError, match="u must be a CUDA tensor"):
        ops.ssm_scan(*[t.clone().requires_grad_(True) for t in args])
    with torch.inference_mode(), pytest.raises(RuntimeError, match="u must be a CUDA tensor"):
        ops.ssm_scan(*args)
    assert "Tensor(a!)? out_state=None" in str(ops.ssm_step.default._schema)
    with pytest.raises(RuntimeError, match="u must be a CUDA tensor"):
        ops.ssm_step(x["u"][:, 0], x["delta"][:, 0], x["A"], x["B_ssm"][:, 0], x["C_ssm"][:, 0], x["D_ssm"],
                     torch.zeros(2, 3, 16))


def test_library_override_maps_one_copy(tmp_path):
    """With MWC_SSM_LIB pointing at another copy of libmwc_ssm.so, the ctypes binding and the PyTorch
    operators (whose dependency resolves through the library's SONAME) share that one copy: the
    process maps a single libmwc_ssm.so, the override."""
    import shutil
    import subprocess
    import sys

    from mamba_windows_cuda import _lib

    alt = tmp_path / "libmwc_ssm.so"
    shutil.copy(_lib.LIB_PATH, alt)
    code = (
        "import sys; sys.path[:0] = %r\n"
        "from mamba_windows_cuda import _lib\n"
        "_lib.torch_ops(); _lib.lib()\n"
        "maps = {l.split()[-1] for l in open('/proc/self/maps') if l.rstrip().endswith('libmwc_ssm.so')}\n"
        "print(sorted(maps))\n" % (sys.path[:3],))
    env = dict(os.environ, MWC_SSM_LIB=str(alt))
    r = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr
    assert r.stdout.strip() == str([str(alt)]), r.stdout


# Instances that may use per-lane scratch (register spills), from the code object metadata of the build:
# the N=8 backward main kernel at two states per lane (3 waves per SIMD; at 2 it does not spill but
# is 27% slower) and the two-states-per-lane backward with both transforms at N=16 and 32.
SPILL_ALLOWED = re.compile(r"ssm_bwd_kernelI.*Li8ELi2ELi\dE|ssm_bwd_kernelI.*Li(16|32)ELi2ELi3E")


def _kernel_scratch(lib_path, tmp_path):
    """{kernel symbol: private segment bytes} of the gfx950 code objects bundled in the library."""
    import shutil
    import subprocess

    tools = ("objcopy", "/opt/rocm/llvm/bin/clang-offload-bundler", "/opt/rocm/llvm/bin/llvm-readelf")
    if not all(shutil.which(t) or os.path.exists(t) for t in tools):
        pytest.skip("objcopy / ROCm LLVM tools not available")
    fat = tmp_path / "fatbin.bin"
    subprocess.run(["objcopy", "-O", "binary", "--only-section=.hip_fatbin", lib_path, str(fat)], check=True)
    data = fat.read_bytes()
    starts = [m.start() for m in re.finditer(re.escape(b"__CLANG_OFFLOAD_BUNDLE__"), data)]
    out = {}
    for i, s0 in enumerate(starts):
        part = tmp_path / f"b{i}.bin"
        part.write_bytes(data[s0:starts[i + 1] if i + 1 < len(starts) else len(data)])
        co = tmp_path / f"co{i}.o"
        subprocess.run([tools[1], "--unbundle", "--type=o", f"--input={part}",
                        "--targets=hipv4-amdgcn-amd-amdhsa--gfx950", f"--output={co}"], check=True)
        notes = subprocess.run([tools[2], "--notes", str(co)], capture_output=True, text=True, check=True).stdout
        name = None
        for line in notes.splitlines():
            m = re.match(r"\s+\.name:\s+(\S+)", line)
            if m:
                name = m.group(1)
            m = re.match(r"\s+\.private_segment_fixed_size:\s+(\d+)", line)
            if m and name:
                out[name] = int(m.group(1))
    return out


def test_kernels_do_not_spill(tmp_path):
    """Every kernel instance of libmwc_ssm.so builds without per-lane scratch (register spills), except
    the listed backward instances; in particular every forward instance (mwc_ssm_fwd_noalloc's kernels)
    and the config-2 path."""
    from mamba_windows_cuda import _lib

    sizes = _kernel_scratch(_lib.LIB_PATH, tmp_path)
    assert len(sizes) > 300  # every template instance is there
    bad = sorted(k for k, v in sizes.items() if v > 0 and not SPILL_ALLOWED.search(k))
    assert not bad, f"{len(bad)} instances spill: {bad[:4]}"
    assert all(v == 0 for k, v in sizes.items() if "ssm_fwd_kernel" in k or "ssm_step" in k or "pscan" in k)


def test_workspace_sizes_of_empty_and_tiny_shapes():
    """The planner behind the workspace queries handles empty batches, channels and sequences (host
    code only: these sizes launch nothing)."""
    from mamba_windows_cuda import _lib

    L = _lib.lib()
    for B, Lq, D in ((0, 100, 64), (2, 0, 64), (2, 100, 0), (0, 0, 0), (1, 1, 1), (1, 16, 1), (3, 255, 158)):
        for n in (8, 16, 32, 64):
            assert L.mwc_ssm_fwd_workspace_size(B, Lq, D, n) >= 0
            assert L.mwc_ssm_bwd_workspace_size(B, Lq, D, n) >= 0


def test_workspace_sizes_of_rejected_shapes():
    """Sizes the entry points reject (unsupported state counts, negative sizes, beyond the supported
    range) need no workspace: the queries return 0 and name the reason, instead of planning them (a
    state count of 4 or 0 used to divide by zero in the planner)."""
    from mamba_windows_cuda import _lib

    L = _lib.lib()
    for B, Lq, D, n in ((2, 100, 64, 0), (2, 100, 64, 4), (2, 100, 64, 128), (-1, 100, 64, 16), (2, -5, 64, 16),
                        (2, 100, -1, 16), (65535, 16, 1 << 24, 16), (65536, 16, 64, 16), (1 << 14, 1 << 20, 64, 16)):
        for query in (L.mwc_ssm_fwd_workspace_size, L.mwc_ssm_bwd_workspace_size):
            assert query(B, Lq, D, n) == 0, (B, Lq, D, n)
            assert L.mwc_last_error(), (B, Lq, D, n)


def test_status_strings_and_ckpt_count():
    from mamba_windows_cuda import _lib

    L = _lib.lib()
    assert L.mwc_status_string(0) == b"MWC_OK"
    assert L.mwc_status_string(1) == b"MWC_ERR_INVALID_ARGUMENT"
    assert L.mwc_ssm_ckpt_count(0) == 0
    assert L.mwc_ssm_ckpt_count(1) == 1
    assert L.mwc_ssm_ckpt_count(16) == 1
    assert L.mwc_ssm_ckpt_count(17) == 2
    assert L.mwc_ssm_ckpt_count(2048) == 128


def test_argument_errors_before_any_launch():
    """Contract violations return a status before the library touches the device."""
    from mamba_windows_cuda import _lib

    L = _lib.lib()
    fake = ctypes.c_void_p(16)
    # N outside {8, 16, 32, 64} (the reference accepts N=16 only, mamba_cuda.py:215)
    for bad_n in (15, 4, 128):
        st = L.mwc_ssm_fwd(1, fake, fake, fake, fake, fake, fake, None, fake, None, None, 1, 8, 8, bad_n, fake,
                           1 << 20, None)
        assert st == 1 and b"N=16" in L.mwc_last_error()
    # bad dtype
    st = L.mwc_ssm_fwd(7, fake, fake, fake, fake, fake, fake, None, fake, None, None, 1, 8, 8, 16, fake, 1 << 20, None)
    assert st == 1
    # backward workspace too small
    st = L.mwc_ssm_bwd(0, fake, fake, fake, fake, fake, fake, None, fake, None, fake, fake, fake, fake, fake, fake,
                       fake, None, 1, 8, 8, 16, fake, 4, None)
    assert st == 3 and b"workspace" in L.mwc_last_error()
    # backward without checkpoints
    st = L.mwc_ssm_bwd(0, fake, fake, fake, fake, fake, fake, None, fake, None, None, fake, fake, fake, fake, fake,
                       fake, None, 1, 8, 8, 16, fake, 1 << 20, None)
    assert st == 1
    # scan: negative size, missing pointer
    assert L.mwc_pscan_fwd(0, fake, fake, fake, -1, 8, 8, fake, 1 << 20, None) == 1
    assert L.mwc_pscan_fwd(0, None, fake, fake, 1, 8, 8, fake, 1 << 20, None) == 1
    # empty problems are no-ops
    assert L.mwc_ssm_fwd(0, None, None, fake, None, None, fake, None, None, None, None, 0, 8, 8, 16, None, 0, None) == 0
    assert L.mwc_pscan_fwd(0, None, None, None, 0, 8, 8, None, 0, None) == 0
    # the non-waiting scan status: no host word, workspace too small; an empty scan reports 0 at once
    word = ctypes.c_uint32(7)
    assert L.mwc_pscan_status_async(fake, 1 << 20, 1, 8, 8, None, None) == 1
    assert L.mwc_pscan_status_async(fake, 4, 2, 1000, 64, ctypes.byref(word), None) == 3
    assert L.mwc_pscan_status_async(None, 0, 0, 8, 8, ctypes.byref(word), None) == 0 and word.value == 0


def test_transform_entry_points_argument_errors():
    """The fused-transform entry points reject inconsistent optional arguments before any launch."""
    from mamba_windows_cuda import _lib

    L = _lib.lib()
    fake = ctypes.c_void_p(16)
    # out_z without z
    st = L.mwc_ssm_fwd_ex(0, fake, fake, fake, fake, fake, fake, None, None, 0, None, fake, fake, None, None,
                          1, 8, 8, 16, fake, 1 << 20, None)
    assert st == 1 and b"out_z" in L.mwc_last_error()
    # backward with z but no ungated output
    st = L.mwc_ssm_bwd_ex(0, fake, fake, fake, fake, fake, fake, None, None, 0, fake, None, fake, None, fake,
                          fake, fake, fake, fake, fake, fake, None, fake, None, 1, 8, 8, 16, fake, 1 << 20, None)
    assert st == 1 and b"ungated" in L.mwc_last_error()
    # ddelta_bias without delta_bias
    st = L.mwc_ssm_bwd_ex(0, fake, fake, fake, fake, fake, fake, None, None, 0, None, None, fake, None, fake,
                          fake, fake, fake, fake, fake, fake, fake, None, None, 1, 8, 8, 16, fake, 1 << 20, None)
    assert st == 1


def test_transform_validation():
    from mamba_windows_cuda import ops

    u = torch.randn(2, 5, 3)
    with pytest.raises(RuntimeError, match="delta_bias shape"):
        ops.check_transforms(u, torch.randn(4), None)
    with pytest.raises(RuntimeError, match="z dtype"):
        ops.check_transforms(u, None, torch.randn(2, 5, 3).double())


def test_step_argument_errors():
    from mamba_windows_cuda import _lib

    L = _lib.lib()
    fake = ctypes.c_void_p(16)
    # missing state
    st = L.mwc_ssm_step(0, fake, fake, fake, fake, fake, fake, None, None, 0, None, fake, None, fake, 2, 8, 16, None)
    assert st == 1 and b"h_new" in L.mwc_last_error()
    # z without out_z; an unsupported N
    assert L.mwc_ssm_step(0, fake, fake, fake, fake, fake, fake, fake, None, 0, fake, fake, None, fake, 2, 8, 16,
                          None) == 1
    assert L.mwc_ssm_step(0, fake, fake, fake, fake, fake, fake, fake, None, 0, None, fake, None, fake, 2, 8, 12,
                          None) == 1
    assert b"N=16" in L.mwc_last_error()


def test_workspace_sizes_monotone():
    from mamba_windows_cuda import _lib

    L = _lib.lib()
    a = L.mwc_ssm_bwd_workspace_size(8, 2048, 1536, 16)
    b = L.mwc_ssm_bwd_workspace_size(8, 4096, 1536, 16)
    assert 0 < a < b
    # the forward needs workspace only for the carries of a split sequence
    assert L.mwc_ssm_fwd_workspace_size(1, 16, 64, 16) == 0
    assert L.mwc_ssm_fwd_workspace_size(8, 2048, 1536, 16) % 256 == 0
    assert L.mwc_ssm_fwd_workspace_size(1, 131072, 2048, 16) > 0
    assert L.mwc_pscan_workspace_size(4, 65536, 1024) > 0
    # the carries and the dB/dC/dA partials scale with N
    assert L.mwc_ssm_bwd_workspace_size(8, 2048, 1536, 8) < a < L.mwc_ssm_bwd_workspace_size(8, 2048, 1536, 64)


def _valid(dtype=torch.float32, B=2, L=5, D=3):
    return dict(u=torch.randn(B, L, D, dtype=dtype), delta=torch.rand(B, L, D, dtype=dtype),
                A=-torch.rand(D, 16, dtype=dtype), B_ssm=torch.randn(B, L, 16, dtype=dtype),
                C_ssm=torch.randn(B, L, 16, dtype=dtype), D_ssm=torch.ones(D, dtype=dtype))


@pytest.mark.parametrize("mutate,msg", [
    (lambda x: x.update(A=torch.randn(3, 15)), "Only N=16"),
    (lambda x: x.update(A=torch.randn(3, 32)), "B_ssm shape mismatch"),
    (lambda x: x.update(u=x["u"].double()), "float32/float16"),
    (lambda x: x.update(delta=x["delta"].half()), "delta dtype must match"),
    (lambda x: x.update(u=x["u"][0]), "u must be 3D"),
    (lambda x: x.update(B_ssm=torch.randn(2, 4, 16)), "B_ssm shape mismatch"),
    (lambda x: x.update(D_ssm=torch.ones(4)), "D_ssm shape mismatch"),
    (lambda x: x.update(C_ssm=torch.randn(2, 16, 5).transpose(1, 2)), "C_ssm must be contiguous"),
    (lambda x: x.update(h_prev=torch.randn(2, 3, 17)), "h_prev shape must be"),
    (lambda x: x.update(h_prev=torch.randn(3, 3, 16)), "h_prev shape must be"),
    (lambda x: x.update(h_prev=torch.randn(2, 3, 16).half()), "h_prev dtype"),
])
def test_validation_contract(mutate, msg):
    """Same failures as the reference's TORCH_CHECKs (mamba_cuda.py:281-326), as RuntimeError."""
    from mamba_windows_cuda import ops

    x = _valid()
    mutate(x)
    with pytest.raises(RuntimeError, match=msg):
        ops.check_ssm_inputs(x["u"], x["delta"], x["A"], x["B_ssm"], x["C_ssm"], x["D_ssm"], x.get("h_prev"),
                             require_device=False)


def test_cpu_tensors_are_rejected_not_computed():
    """No CPU fallback: host tensors raise like the reference's is_cuda checks."""
    from mamba_windows_cuda import FusedSelectiveScan, SelectiveScanCuda, parallel_scan_fn

    x = _valid()
    with pytest.raises(RuntimeError, match="must be a CUDA tensor"):
        SelectiveScanCuda()(x["u"], x["delta"], x["A"], x["B_ssm"], x["C_ssm"], x["D_ssm"])
    with pytest.raises(RuntimeError, match="must be a CUDA tensor"):
        FusedSelectiveScan(1).forward_with_state(x["u"], x["delta"], x["A"], x["B_ssm"], x["C_ssm"], x["D_ssm"])
    with pytest.raises(RuntimeError, match="CUDA"):
        parallel_scan_fn(torch.rand(1, 2, 8, 4), torch.rand(1, 2, 8, 4))
    with pytest.raises(RuntimeError, match="must be a CUDA tensor"):
        SelectiveScanCuda().step(x["u"][:, 0], x["delta"][:, 0], x["A"], x["B_ssm"][:, 0], x["C_ssm"][:, 0],
                                 x["D_ssm"], torch.zeros(2, 3, 16))


def test_reference_api_functions_on_cpu():
    """selective_scan_ref / parallel_scan_ref are plain-PyTorch API functions (any device)."""
    import numpy as np

    from mamba_windows_cuda import parallel_scan_ref, selective_scan_ref
    from oracle import oracle as orc

    x = _valid(B=2, L=9, D=4)
    hp = torch.randn(2, 4, 16)
    out, hl = selective_scan_ref(x["u"], x["delta"], x["A"], x["B_ssm"], x["C_ssm"], x["D_ssm"], hp)
    ro, rh = orc.ssm_fwd(x["u"], x["delta"], x["A"], x["B_ssm"], x["C_ssm"], x["D_ssm"], hp)
    np.testing.assert_allclose(out.numpy(), ro, rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(hl.numpy(), rh, rtol=1e-4, atol=1e-5)
    _, _, inter = selective_scan_ref(x["u"], x["delta"], x["A"], x["B_ssm"], x["C_ssm"], x["D_ssm"],
                                     return_intermediates=True)
    assert inter["h_states"].shape == (2, 4, 16, 9)
    A = torch.rand(2, 3, 11, 5)
    X = torch.randn(2, 3, 11, 5)
    np.testing.assert_allclose(parallel_scan_ref(A, X).numpy(), orc.pscan_fwd(A, X), rtol=1e-5, atol=1e-6)


def test_selective_scan_backward_is_the_true_adjoint():
    """selective_scan_backward (the reference's API, mamba_cuda.py:949-1041) on selective_scan_ref's
    intermediates: all seven gradients equal the float64 oracle's adjoint and torch autograd through
    selective_scan_ref (rather than the reference loop's decayed-adjoint formulas)."""
    import numpy as np

    from mamba_windows_cuda.mamba_cuda import selective_scan_backward, selective_scan_ref
    from oracle import oracle as orc

    g = torch.Generator().manual_seed(12)
    B, L, D, N = 2, 13, 5, 16
    u = torch.randn(B, L, D, generator=g, dtype=torch.float64)
    delta = 0.05 + 0.5 * torch.rand(B, L, D, generator=g, dtype=torch.float64)
    A = -torch.rand(D, N, generator=g, dtype=torch.float64)
    Bs = torch.randn(B, L, N, generator=g, dtype=torch.float64)
    Cs = torch.randn(B, L, N, generator=g, dtype=torch.float64)
    Dv = torch.randn(D, generator=g, dtype=torch.float64)
    hp = torch.randn(B, D, N, generator=g, dtype=torch.float64)
    dout = torch.randn(B, L, D, generator=g, dtype=torch.float64)
    dhl = torch.randn(B, D, N, generator=g, dtype=torch.float64)
    out, hl, inter = selective_scan_ref(u, delta, A, Bs, Cs, Dv, hp, return_intermediates=True)
    got = selective_scan_backward(dout, dhl, inter, Dv)
    ref = orc.ssm_bwd(u, delta, A, Bs, Cs, Dv, dout, hp, dhl)
    names = ("du", "ddelta", "dA", "dB", "dC", "dD", "dh_prev")
    for name, t in zip(names, got):
        np.testing.assert_allclose(t.numpy(), ref[name], rtol=1e-10, atol=1e-12, err_msg=name)
    leaves = [x.clone().requires_grad_(True) for x in (u, delta, A, Bs, Cs, Dv, hp)]
    o2, h2 = selective_scan_ref(*leaves)
    torch.autograd.backward([o2, h2], [dout, dhl])
    for name, t, leaf in zip(names, got, leaves):
        torch.testing.assert_close(t, leaf.grad, rtol=1e-10, atol=1e-12, msg=name)
    # dh_last=None means zeros
    got0 = selective_scan_backward(dout, None, inter, Dv)
    ref0 = orc.ssm_bwd(u, delta, A, Bs, Cs, Dv, dout, hp, None)
    np.testing.assert_allclose(got0[6].numpy(), ref0["dh_prev"], rtol=1e-10, atol=1e-12)
    # the reference's own 8-key dict (mamba_cuda.py:934-944, no 'A'): A recovered from dA and delta_t,
    # or passed as a keyword
    inter.pop("A")
    assert sorted(inter) == sorted(["h_states", "dA", "dBu", "u_t", "delta_t", "B_t", "C_t", "h_prev"])
    for got in (selective_scan_backward(dout, dhl, inter, Dv), selective_scan_backward(dout, dhl, inter, Dv, A=A)):
        for name, t in zip(names, got):
            np.testing.assert_allclose(t.numpy(), ref[name], rtol=1e-10, atol=1e-12, err_msg=name)
    # a channel whose delta is 0 at every step: its decay factors are 1 whatever A is
    inter["delta_t"] = inter["delta_t"].clone()
    inter["delta_t"][:, 2] = 0.0
    with pytest.raises(RuntimeError, match="pass A="):
        selective_scan_backward(dout, dhl, inter, Dv)


def test_selective_scan_backward_reference_dict_fp32():
    """The reference's fp32 intermediates (config-0 distributions, delta ~ U(1e-3, 1e-1)) without 'A':
    the recovered A (absolute error ~eps/max delta) keeps every gradient within the fp32 bound of the
    float64 oracle."""
    import numpy as np

    from mamba_windows_cuda import workloads
    from mamba_windows_cuda.mamba_cuda import recover_A, selective_scan_backward, selective_scan_ref
    from oracle import oracle as orc

    x = workloads.ssm_inputs(2, 64, 24, dtype=torch.float32, a_lo=0.0, a_hi=0.1, d_mode="ones", h_prev=True,
                             seed=5)
    dhl = torch.randn(2, 24, 16, generator=torch.Generator().manual_seed(6))
    _, _, inter = selective_scan_ref(x["u"], x["delta"], x["A"], x["B"], x["C"], x["D"], x["h_prev"],
                                     return_intermediates=True)
    inter.pop("A")
    Ar = recover_A(inter["dA"], inter["delta_t"])
    # log(dA) carries about one ulp of 1: an absolute error in A of ~eps32/max(delta) = 7e-7
    np.testing.assert_allclose(Ar.numpy(), x["A"].numpy(), rtol=0, atol=2e-6)
    got = selective_scan_backward(x["dout"], dhl, inter, x["D"])
    ref = orc.ssm_bwd(x["u"], x["delta"], x["A"], x["B"], x["C"], x["D"], x["dout"], x["h_prev"], dhl)
    for name, t in zip(("du", "ddelta", "dA", "dB", "dC", "dD", "dh_prev"), got):
        np.testing.assert_allclose(t.numpy(), ref[name], rtol=1e-3, atol=1e-4, err_msg=name)


def test_scan_status_queue_reports_finished_failures():
    """The non-waiting scan status: words whose events have completed are retired in order, a non-zero
    word raises MWC_ERR_INCOMPLETE, unfinished ones stay queued until pscan_check() waits for them."""
    import torch

    from mamba_windows_cuda import ops

    class Ev:
        def __init__(self, done):
            self.done, self.waited = done, False

        def query(self):
            return self.done

        def synchronize(self):
            self.waited = True
            self.done = True

    q = ops._pending_status
    saved = list(q)
    q.clear()
    try:
        ok, bad, later = Ev(True), Ev(True), Ev(False)
        q.extend([(ok, torch.zeros(1, dtype=torch.int32), "a"), (bad, torch.ones(1, dtype=torch.int32), "b"),
                  (later, torch.zeros(1, dtype=torch.int32), "c")])
        with pytest.raises(RuntimeError, match="b failed: MWC_ERR_INCOMPLETE"):
            ops._drain_status()
        assert [w for _, _, w in q] == ["c"] and not later.waited  # the unfinished one stays, not waited for
        ops._drain_status()  # nothing finished: no error, still queued
        assert len(q) == 1
        ops.pscan_check()  # waits for it; its word is 0
        assert later.waited and len(q) == 0
        fail = Ev(False)
        q.append((fail, torch.full((1,), 5, dtype=torch.int32), "d"))
        with pytest.raises(RuntimeError, match="d failed"):
            ops.pscan_check()
        assert fail.waited and len(q) == 0
    finally:
        q.clear()
        q.extend(saved)
