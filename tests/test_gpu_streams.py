"""Work enqueued on several HIP streams at once: every scan call takes its scratch from its own
workspace (the caching allocator, per stream), and the kernels keep no state between calls, so
training steps and parallel scans running concurrently on different streams give exactly the results
they give one after the other on the default stream."""
import pytest
import torch

from mamba_windows_cuda import SelectiveScanCuda, parallel_scan_fn, workloads
from mamba_windows_cuda.pscan import pscan_check

pytestmark = pytest.mark.gpu

NAMES = ("u", "delta", "A", "B", "C", "D", "h_prev")


def _ssm_step(x, dout, lvl):
    leaves = {k: v.detach().clone().requires_grad_(True) for k, v in x.items()}
    out, h_last = SelectiveScanCuda(checkpoint_lvl=lvl).forward_with_state(*(leaves[k] for k in NAMES))
    out.backward(dout)
    return [out.detach(), h_last.detach()] + [leaves[k].grad for k in NAMES]


def _scan(a, b, dh):
    A, X = a.detach().clone().requires_grad_(True), b.detach().clone().requires_grad_(True)
    H = parallel_scan_fn(A, X)
    H.backward(dh)
    return [H.detach(), A.grad, X.grad]


def test_concurrent_streams_match_serial_results(dev):
    print("case concurrent streams", flush=True)
    cases = []
    for i, (B, L, D, dtype) in enumerate(((2, 700, 384, torch.float16), (1, 1500, 256, torch.float32),
                                          (4, 300, 1024, torch.bfloat16))):
        x = {k: v.to(dev) for k, v in workloads.ssm_inputs(B, L, D, dtype=dtype, h_prev=True, seed=50 + i).items()}
        cases.append(("ssm", ({k: x[k] for k in NAMES}, x["dout"], i % 2)))
    for i, shape in enumerate(((2, 5000, 96), (3, 40, 700, 8))):
        a, b = workloads.pscan_inputs(shape, seed=70 + i, device=dev)
        cases.append(("scan", (a, b, torch.randn(shape, device=dev))))
    run = {"ssm": lambda args: _ssm_step(*args), "scan": lambda args: _scan(*args)}

    serial = [run[kind](args) for kind, args in cases]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream() for _ in cases]
    for s in streams:
        s.wait_stream(torch.cuda.current_stream())
    results = [None] * len(cases)
    for rep in range(3):  # several rounds, each case on its own stream, all in flight together
        for i, ((kind, args), s) in enumerate(zip(cases, streams)):
            with torch.cuda.stream(s):
                results[i] = run[kind](args)
        for s in streams:
            torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        pscan_check()
        for (kind, _), got, ref in zip(cases, results, serial):
            for g, r in zip(got, ref):
                if kind == "ssm":  # deterministic kernels and plans: bitwise
                    assert torch.equal(g, r), f"round {rep}"
                else:  # the scan's look-back order varies: rounding-level agreement
                    torch.testing.assert_close(g, r, rtol=1e-5, atol=1e-5)
