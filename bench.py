#!/usr/bin/env python3
"""Benchmark of the fused selective-scan training step on one MI355X.

Default workload (the Mamba-130M layer shape): fp16
storage / fp32 compute, B=8, L=2048, D=1536, N=16; one step = fused forward
(checkpoint level 0) + fused backward through the drop-in autograd API, with
all inputs resident in HBM. Prints ONE JSON line.

  python bench.py [--steps K] [--warmup W] [--config cfg2|cfg3|cfg4a|cfg4b]
                  [--level 0|1] [--skip-cpu] [--transforms] [--decode [BATCH]] [--shard K]
                  [--nstate 8|16|32|64] [--dtype f16|bf16|f32]
  python bench.py --profile-recipe DIR   # the rocprofv3 commands behind profiles/*.txt
  python bench.py --summarize DIR        # their CSV output -> profiles/*.txt (no GPU needed)

`value` = B*L*D / ms_per_step (elements/s). `roofline` covers the dominant
kernel (the fused backward call), timed live with HIP events on the stream
the kernels run on; its algorithmic bytes are s*(5BLD + 4BLN + 2DN + 2D).
`cpu_baseline` times the plain-PyTorch sequential restatement of the
reference's CPU path (selective_scan_ref forward + autograd backward) on a
bounded sample of the same workload on this host's cores.
"""
from __future__ import annotations

import argparse
import json
import os
import re
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "mamba-windows-cuda_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0  # MI355X published HBM3E peak
# non-packed fp32 VALU issue: 256 CUs x 64 lanes x 2.4 GHz, in 1e12 lane-operations per second
VALU_PEAK_TOPS = 256 * 64 * 2.4e9 / 1e12
# algorithmic VALU issue slots per state and step (v_exp_f32 counted as two): forward = mul
# (delta*A), exp, mul (delta*u*B), fma (state), fma (C-contraction); backward = the recompute
# (mul, exp, mul, fma) + the reverse sweep (fma, fma, mul, mul, fma, fma) + the dB/dC fold (2 fma)
VALU_SLOTS_FWD, VALU_SLOTS_BWD = 6, 13
METRIC = "fwd+bwd elements/sec (B·L·D) and achieved HBM GB/s vs peak, 1×MI355X"


def _traffic_from_profiles(name):
    """HBM bytes per launch measured with rocprofv3 --pmc (FETCH_SIZE + WRITE_SIZE,
    copy-kernel calibrated), read from the committed summary if present."""
    path = os.path.join(ROOT, "profiles", f"{name}_pmc.txt")
    if not os.path.exists(path):
        return None
    m = re.search(r"^traffic_bytes_per_launch:\s*([0-9.eE+]+)", open(path).read(), re.M)
    return float(m.group(1)) if m else None


# The GPU's clocks ramp over the first ~0.1 s of sustained load (measured at cfg2: 20 timed steps right
# after 5 warm-up steps read 0.495 ms per step, 400 read 0.413 ms, the sum of the two calls' times), and a
# training loop runs at the ramped clock: the warm-up runs its W steps and, past them, until this much
# wall time of back-to-back steps has passed.
MIN_WARMUP_S = 0.3


def _warmup(fn, n):
    """Runs `fn` untimed at least `n` times and at least MIN_WARMUP_S of wall time (synchronizing every 16
    calls, so the time counts work done, not work queued); returns the number of calls run."""
    import torch

    t0 = time.perf_counter()
    done = 0
    while done < n or time.perf_counter() - t0 < MIN_WARMUP_S:
        fn()
        done += 1
        if done % 16 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    return done


def _events_ms(fn, n):
    import torch

    st = torch.cuda.current_stream()
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    a.record(st)
    for _ in range(n):
        fn()
    b.record(st)
    b.synchronize()
    return a.elapsed_time(b) / n


DTYPES = {"f16": "float16", "bf16": "bfloat16", "f32": "float32"}


def _pmc_field(name, key):
    """A figure from a committed rocprofv3 --pmc summary (profiles/<name>_pmc.txt), or None."""
    path = os.path.join(ROOT, "profiles", f"{name}_pmc.txt")
    if not os.path.exists(path):
        return None
    m = re.search(rf"^{key}:\s*([0-9.eE+-]+)", open(path).read(), re.M)
    return float(m.group(1)) if m else None


def _capture_step(step):
    """The step captured once in a HIP graph (after eager warm-up steps on a side stream)."""
    import torch

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):
            step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    return graph.replay


def bench_ssm(cfg, steps, warmup, level, shard=1, nstate=16, dtype_name=None, graph=False):
    import torch

    from mamba_windows_cuda import SelectiveScanCuda, ops, workloads

    c = workloads.CONFIGS[cfg]
    B, L, D = c["B"], c["L"], c["D"] // shard
    dtype = getattr(torch, DTYPES[dtype_name]) if dtype_name else c["dtype"]
    if shard == 1 and nstate == 16 and dtype == c["dtype"]:
        x = workloads.config_inputs(cfg, device="cuda", gen_device="cuda")
    else:  # one GPU's channels when D is split over `shard` GPUs, or another state count / dtype
        kw = {k: v for k, v in c.items() if k not in ("B", "L", "D", "dtype")}
        x = workloads.ssm_inputs(B, L, D, device="cuda", gen_device="cuda", dtype=dtype, nstate=nstate, **kw)
    leaves = {k: x[k].requires_grad_(True) for k in ("u", "delta", "A", "B", "C", "D")}
    dout = x["dout"]
    m = SelectiveScanCuda(checkpoint_lvl=level)

    def step():
        for t in leaves.values():
            t.grad = None
        out = m(leaves["u"], leaves["delta"], leaves["A"], leaves["B"], leaves["C"], leaves["D"])
        torch.autograd.backward(out, dout)

    # activation memory a forward keeps for its backward at this checkpoint level (probed before the
    # warm-up, so the timed steps follow it with the allocator settled and the clocks ramped)
    step()
    torch.cuda.synchronize()
    base = torch.cuda.memory_allocated()
    out_keep = m(leaves["u"], leaves["delta"], leaves["A"], leaves["B"], leaves["C"], leaves["D"])
    torch.cuda.synchronize()
    kept = torch.cuda.memory_allocated() - base - out_keep.numel() * out_keep.element_size()
    del out_keep
    torch.cuda.reset_peak_memory_stats()
    run = _capture_step(step) if graph else step
    warm_run = _warmup(run, warmup)
    t0 = time.perf_counter()
    ms_events = _events_ms(run, steps)
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / steps
    ms = max(ms_events, 0.0)

    # live per-call timing of the fused kernels on the same stream
    with torch.no_grad():
        xs = {k: v.detach() for k, v in x.items()}
        _, _, ckpt = ops.ssm_forward(xs["u"], xs["delta"], xs["A"], xs["B"], xs["C"], xs["D"], want_ckpt=True)
        fwd = lambda: ops.ssm_forward(xs["u"], xs["delta"], xs["A"], xs["B"], xs["C"], xs["D"], want_ckpt=True,
                                      want_h_last=False)
        bwd = lambda: ops.ssm_backward(xs["u"], xs["delta"], xs["A"], xs["B"], xs["C"], xs["D"], dout, ckpt)
        for _ in range(3):
            fwd()
            bwd()
        n_k = max(steps, 100)
        fwd_ms = _events_ms(fwd, n_k)
        bwd_ms = _events_ms(bwd, n_k)

    s = torch.tensor([], dtype=dtype).element_size()
    bytes_fwd = workloads.algorithmic_bytes(B, L, D, s, fwd=True, bwd=False, nstate=nstate)
    bytes_bwd = workloads.algorithmic_bytes(B, L, D, s, fwd=False, bwd=True, nstate=nstate)
    elems = B * L * D
    states = elems * nstate
    gbs_bwd = bytes_bwd / (bwd_ms * 1e-3) / 1e9
    gbs_step = (bytes_fwd + bytes_bwd) / (ms * 1e-3) / 1e9
    default_case = shard == 1 and nstate == 16 and dtype == c["dtype"]
    # HBM bytes the counters measured for one backward call (committed rocprofv3 --pmc summary), and the
    # VALU instructions its main kernel issued per state and step (SQ_INSTS_VALU x 64 lanes / states)
    traffic = _traffic_from_profiles(f"ssm_bwd_{cfg}") if default_case else None
    key = "main_kernel_valu_instructions_per_state_step"
    valu_instr = _pmc_field(f"ssm_bwd_{cfg}", key) if default_case else None
    valu_instr_fwd = _pmc_field(f"ssm_fwd_{cfg}", key) if default_case else None
    sdt = {torch.float16: "f16", torch.bfloat16: "bf16"}.get(dtype, "f32")
    res = {
        "metric": METRIC,
        "value": elems / (ms * 1e-3),
        "unit": "elements/s",
        "ms_per_step": ms,
        "dtype": "f32",
        "storage_dtype": sdt,
        "config": {"workload": f"{cfg}: selective scan fwd+bwd (fused), B={B} L={L} D={D} N={nstate}, "
                               f"checkpoint_lvl={level}"
                               + (f", {sdt} storage" if dtype != c["dtype"] else "")
                               + (f"; one GPU's share of D={c['D']} split over {shard} GPUs" if shard > 1 else "")
                               + ("; the step replayed from a HIP graph" if graph else ""),
                   "B": B, "L": L, "D": D, "N": nstate, "checkpoint_lvl": level, "graph": graph},
        # achieved = algorithmic (useful) bytes / call time; traffic = what the counters measured moving
        "roofline": {"bound": "hbm", "kernel": "ssm_bwd (fused backward call)",
                     "achieved": gbs_bwd, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": gbs_bwd / HBM_PEAK_GBS, "traffic": traffic,
                     "algorithmic_bytes_per_launch": bytes_bwd, "avg_launch_ms": bwd_ms,
                     "achieved_counts": "useful (algorithmic) bytes",
                     "traffic_GBps": traffic / (bwd_ms * 1e-3) / 1e9 if traffic else None,
                     "traffic_frac": traffic / (bwd_ms * 1e-3) / 1e9 / HBM_PEAK_GBS if traffic else None,
                     "limiter": "VALU issue (SQ counters: the SIMDs are VALU-busy most of the waves' lifetime; "
                                "HBM and LDS are not saturated)"},
        "valu_roofline": {"bound": "valu", "kernel": "ssm_bwd (fused backward call)",
                          "achieved": states * VALU_SLOTS_BWD / (bwd_ms * 1e-3) / 1e12,
                          "peak": VALU_PEAK_TOPS, "unit": "T lane-op/s",
                          "frac": states * VALU_SLOTS_BWD / (bwd_ms * 1e-3) / 1e12 / VALU_PEAK_TOPS,
                          "slots_per_state": VALU_SLOTS_BWD,
                          "fwd_frac": states * VALU_SLOTS_FWD / (fwd_ms * 1e-3) / 1e12 / VALU_PEAK_TOPS,
                          "measured_valu_instr_per_state_step_bwd_main": valu_instr,
                          "measured_valu_instr_per_state_step_fwd_main": valu_instr_fwd},
        "kernels": {"ssm_fwd_ms": fwd_ms, "ssm_bwd_ms": bwd_ms,
                    "fwd_algorithmic_GBps": bytes_fwd / (fwd_ms * 1e-3) / 1e9},
        "step_hbm": {"algorithmic_bytes": bytes_fwd + bytes_bwd, "achieved_GBps": gbs_step,
                     "frac_of_peak": gbs_step / HBM_PEAK_GBS},
        "wall_ms_per_step": wall_ms,
        "warmup_steps_run": warm_run,
        "retained_after_forward_GB": kept / 1e9,
    }
    if shard > 1:  # what the shards would exchange: one all-reduce of the dB/dC partials (fp32)
        res["shard"] = {"gpus": shard, "split": "D", "allreduce_bytes": 2 * B * L * nstate * 4}
    return res


def bench_transforms(cfg, steps, warmup):
    """A Mamba block's scan call: delta' = softplus(delta + delta_bias) and out * silu(z) fused into the
    kernels, against the same step with the transforms as separate torch elementwise passes around
    the plain fused scan. Both are fwd + bwd through autograd with all six gradients plus
    d(delta_bias) and dz."""
    import torch

    from mamba_windows_cuda import SelectiveScanCuda, workloads

    c = workloads.CONFIGS[cfg]
    B, L, D = c["B"], c["L"], c["D"]
    x = workloads.config_inputs(cfg, device="cuda", gen_device="cuda")
    g = torch.Generator(device="cuda").manual_seed(1)
    x["delta"] = (-4.0 + torch.randn(B, L, D, generator=g, device="cuda")).to(c["dtype"])
    x["delta_bias"] = (0.5 * torch.randn(D, generator=g, device="cuda")).to(c["dtype"])
    x["z"] = torch.randn(B, L, D, generator=g, device="cuda").to(c["dtype"])
    names = ("u", "delta", "A", "B", "C", "D", "delta_bias", "z")
    leaves = {k: x[k].requires_grad_(True) for k in names}
    dout = x["dout"]
    m = SelectiveScanCuda()

    def fused():
        for t in leaves.values():
            t.grad = None
        out = m(leaves["u"], leaves["delta"], leaves["A"], leaves["B"], leaves["C"], leaves["D"],
                z=leaves["z"], delta_bias=leaves["delta_bias"], delta_softplus=True)
        torch.autograd.backward(out, dout)

    def unfused():
        for t in leaves.values():
            t.grad = None
        dl = torch.nn.functional.softplus(leaves["delta"] + leaves["delta_bias"])
        y = m(leaves["u"], dl, leaves["A"], leaves["B"], leaves["C"], leaves["D"])
        torch.autograd.backward(y * torch.nn.functional.silu(leaves["z"]), dout)

    res = {"metric": "fwd+bwd elements/sec (B·L·D), Mamba-block scan call with delta_bias + softplus + z gating",
           "unit": "elements/s", "dtype": "f32", "storage_dtype": "f16" if c["dtype"] == torch.float16 else "f32",
           "config": {"workload": f"{cfg} + fused transforms, B={B} L={L} D={D} N=16", "B": B, "L": L, "D": D}}
    for name, fn in (("fused", fused), ("unfused_torch_elementwise", unfused)):
        _warmup(fn, warmup)
        ms = _events_ms(fn, steps)
        res[name] = {"ms_per_step": ms, "elements_per_s": B * L * D / (ms * 1e-3)}
    res["value"] = res["fused"]["elements_per_s"]
    res["ms_per_step"] = res["fused"]["ms_per_step"]
    return res


def bench_decode(cfg, steps, warmup, batch=None):
    """Decode steps (L = 1, state carried in place) at the config's D and dtype. Bytes per step:
    the state read and written (2*B*D*16*s) plus u, delta, out (3*B*D*s), B, C (2*B*16*s), A, D."""
    import torch

    from mamba_windows_cuda import SelectiveScanCuda, workloads

    c = workloads.CONFIGS[cfg]
    B, D = batch or c["B"], c["D"]
    x = workloads.ssm_inputs(B, 1, D, dtype=c["dtype"], h_prev=True, dout=False, device="cuda", gen_device="cuda")
    s = 2 if c["dtype"] == torch.float16 else 4
    m = SelectiveScanCuda()
    h = x["h_prev"].clone()
    args = (x["u"][:, 0].contiguous(), x["delta"][:, 0].contiguous(), x["A"], x["B"][:, 0].contiguous(),
            x["C"][:, 0].contiguous(), x["D"])

    def step():
        m.step(*args, h, out_state=h)

    with torch.no_grad():
        _warmup(step, warmup)
        ms_eager = _events_ms(step, max(steps, 100))
        # a decode loop as a serving engine runs it: 32 steps captured once in a HIP graph, replayed
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for _ in range(32):
                step()
        graph.replay()
        torch.cuda.synchronize()
        ms = _events_ms(graph.replay, max(steps // 32, 10)) / 32
    nbytes = s * (2 * B * D * 16 + 3 * B * D + 2 * B * 16 + D * 16 + D)
    gbs = nbytes / (ms * 1e-3) / 1e9
    return {"metric": "decode steps/s (L=1, state in place, HIP-graph replay)", "value": 1e3 / ms,
            "unit": "steps/s", "us_per_step": ms * 1e3, "us_per_step_eager": ms_eager * 1e3, "dtype": "f32",
            "storage_dtype": "f16" if s == 2 else "f32",
            "config": {"workload": f"{cfg} decode step, B={B} D={D} N=16", "B": B, "D": D, "N": 16},
            "roofline": {"bound": "hbm", "kernel": "ssm_step_kernel", "achieved": gbs, "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": gbs / HBM_PEAK_GBS, "algorithmic_bytes_per_launch": nbytes}}


def bench_pscan(steps, warmup):
    """cfg4b through parallel_scan_fn (value: the API call, including the non-waiting read of the
    scan's status word) and through the C ABI alone (the roofline: the clear and scan kernels)."""
    import torch

    from mamba_windows_cuda import _lib, ops, parallel_scan_fn, workloads

    a, b = workloads.pscan_inputs(device="cuda", gen_device="cuda")
    _warmup(lambda: parallel_scan_fn(a, b), warmup)
    ms = _events_ms(lambda: parallel_scan_fn(a, b), steps)
    L_ = _lib.lib()
    nseq, L, nc = a.shape
    nbytes = L_.mwc_pscan_workspace_size(nseq, L, nc)
    ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    H = torch.empty_like(b)
    stream = ops._stream(a.device)

    def kernels():
        _lib.check(L_.mwc_pscan_fwd(_lib.MWC_DTYPE_F32, a.data_ptr(), b.data_ptr(), H.data_ptr(), nseq, L, nc,
                                    ws.data_ptr(), nbytes, stream), "mwc_pscan_fwd")

    _warmup(kernels, warmup)
    kms = _events_ms(kernels, steps)
    _lib.check(L_.mwc_pscan_status(ws.data_ptr(), nbytes, nseq, L, nc, stream), "mwc_pscan_status")
    nbytes_alg = 3 * 4 * a.numel()
    gbs = nbytes_alg / (kms * 1e-3) / 1e9
    return {
        "metric": "parallel_scan_fn elements/s and achieved HBM GB/s vs peak, 1×MI355X",
        "value": a.numel() / (ms * 1e-3), "unit": "elements/s", "ms_per_step": ms, "dtype": "f32",
        "config": {"workload": "cfg4b: parallel_scan_fn over (4, 65536, 1024) fp32", "shape": list(a.shape)},
        "kernel_ms": kms,
        "roofline": {"bound": "hbm", "kernel": "pscan (decoupled look-back; clear + scan kernels)", "achieved": gbs,
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": gbs / HBM_PEAK_GBS,
                     "traffic": _traffic_from_profiles("pscan_cfg4b"), "algorithmic_bytes_per_launch": nbytes_alg,
                     "avg_launch_ms": kms},
    }


def bench_stream(steps, warmup):
    """cfg4a: L=131072 fp32 fed as 32 chunks of 4096 through forward_with_state (no grad)."""
    import torch

    from mamba_windows_cuda import SelectiveScanCuda, workloads

    x = workloads.config_inputs("cfg4a", device="cuda", gen_device="cuda", dout=False)
    m = SelectiveScanCuda()

    def run():
        h = None
        with torch.no_grad():
            for s0 in range(0, 131072, 4096):
                sl = slice(s0, s0 + 4096)
                _, h = m.forward_with_state(x["u"][:, sl], x["delta"][:, sl], x["A"], x["B"][:, sl],
                                            x["C"][:, sl], x["D"], h)
        return h

    _warmup(run, warmup)
    ms = _events_ms(run, steps)
    from mamba_windows_cuda.workloads import algorithmic_bytes

    nbytes = algorithmic_bytes(1, 131072, 2048, 4, fwd=True, bwd=False) + 32 * 4 * 2 * 2048 * 16
    gbs = nbytes / (ms * 1e-3) / 1e9
    return {
        "metric": "streaming forward elements/s and achieved HBM GB/s vs peak, 1×MI355X",
        "value": 131072 * 2048 / (ms * 1e-3), "unit": "elements/s", "ms_per_step": ms, "dtype": "f32",
        "config": {"workload": "cfg4a: fp32 B=1 L=131072 D=2048 as 32 x 4096 chunks via forward_with_state"},
        "roofline": {"bound": "hbm", "kernel": "ssm_fwd", "achieved": gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": gbs / HBM_PEAK_GBS, "traffic": None, "algorithmic_bytes_per_launch": nbytes / 32,
                     "avg_launch_ms": ms / 32},
    }


def cpu_baseline(cfg, d_frac=2, runs=3):
    """Plain-PyTorch restatement of the reference's CPU path, structured like
    selective_scan_ref (mamba_cuda.py:875-946: (B,D,N,L) dA/dBu then a loop
    over L) with torch autograd for the backward, in the config's dtype (torch's
    CPU kernels run fp16 elementwise work natively), timed on a bounded sample of
    the workload: batch row 0, full L, the first D/d_frac channels; the median of
    `runs` timed runs after one warm-up call."""
    import torch

    from mamba_windows_cuda import workloads
    from oracle import torch_ref

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    c = workloads.CONFIGS[cfg]
    L, D = c["L"], c["D"] // d_frac
    x = workloads.ssm_inputs(1, L, D, dtype=c["dtype"], a_lo=c["a_lo"], a_hi=c["a_hi"], d_mode=c["d_mode"])

    def once(n):
        leaves = [x[k][:, :n].clone().requires_grad_(True) if x[k].dim() == 3 else x[k].clone().requires_grad_(True)
                  for k in ("u", "delta", "A", "B", "C", "D")]
        out, _ = torch_ref.selective_scan_vectorized(*leaves)
        out.backward(x["dout"][:, :n])

    once(16)  # load the CPU kernels
    times = []
    for _ in range(runs):
        t = time.perf_counter()
        once(L)
        times.append(time.perf_counter() - t)
    per = sorted(times)[len(times) // 2]
    sdt = "fp16" if c["dtype"] == torch.float16 else "fp32"
    return {"value": L * D / per, "unit": "elements/s", "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"{cfg} batch row 0, L={L}, first {D} of {c['D']} channels, {sdt}, forward + autograd "
                      f"backward of the selective_scan_ref-structured restatement; median of {runs} runs "
                      f"({', '.join(f'{t:.1f}' for t in times)} s); os.cpu_count()={os.cpu_count()}, "
                      f"affinity={cores}"}


def cpu_baseline_pscan(runs=3):
    """The reference's CPU path for cfg4b: parallel_scan_ref (pscan.py:153-171, the package's
    restatement: one torch elementwise update per step over L), on the whole cfg4b workload in fp32;
    the median of `runs` timed runs."""
    import torch

    from mamba_windows_cuda import parallel_scan_ref, workloads

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    a, b = workloads.pscan_inputs()
    times = []
    for _ in range(runs):
        t = time.perf_counter()
        parallel_scan_ref(a, b)
        times.append(time.perf_counter() - t)
    per = sorted(times)[len(times) // 2]
    return {"value": a.numel() / per, "unit": "elements/s", "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"cfg4b in full: parallel_scan_ref over {tuple(a.shape)} fp32 on the host; median of {runs} "
                      f"runs ({', '.join(f'{t:.2f}' for t in times)} s); os.cpu_count()={os.cpu_count()}, "
                      f"affinity={cores}"}


def kernels_only(cfg):
    """Profiling driver: three fused forward/backward calls at `cfg`, three cfg4b scans and a
    1 GiB device copy (the copy calibrates rocprofv3's FETCH_SIZE/WRITE_SIZE counters)."""
    import torch

    from mamba_windows_cuda import ops, parallel_scan_fn, workloads

    x = workloads.config_inputs(cfg, device="cuda", gen_device="cuda")
    for _ in range(3):
        _, _, ck = ops.ssm_forward(x["u"], x["delta"], x["A"], x["B"], x["C"], x["D"], want_ckpt=True,
                                   want_h_last=False)
        ops.ssm_backward(x["u"], x["delta"], x["A"], x["B"], x["C"], x["D"], x["dout"], ck)
    del x
    a, b = workloads.pscan_inputs(device="cuda", gen_device="cuda")
    for _ in range(3):
        parallel_scan_fn(a, b)
    del a, b
    src = torch.ones(1 << 28, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    return {"mode": "kernels-only", "config": cfg, "calibration_copy_bytes": src.numel() * 4}


# rocprofv3 runs behind the committed summaries in profiles/ (bench.py arguments per kernel-trace run;
# counter passes over `bench.py --kernels-only`). `--profile-recipe DIR` prints the commands, `--summarize
# DIR` turns their CSV output into profiles/*.txt.
TRACE_RUNS = {
    "cfg2_fwd_bwd": ["--skip-cpu"],
    "cfg3_level0": ["--config", "cfg3", "--level", "0", "--skip-cpu", "--steps", "30"],
    "cfg3_level1": ["--config", "cfg3", "--level", "1", "--skip-cpu", "--steps", "30"],
    "cfg4a_stream": ["--config", "cfg4a", "--steps", "10"],
    "cfg4b_pscan": ["--config", "cfg4b", "--steps", "50", "--skip-cpu"],
    "decode_b1024": ["--decode", "1024", "--steps", "320"],
    "shard8_eager": ["--shard", "8", "--steps", "400"],
}
PMC_PASSES = {
    "fetch": "FETCH_SIZE",
    "write": "WRITE_SIZE",
    "sq1": "SQ_WAVE_CYCLES SQ_INSTS_VALU SQ_INSTS_LDS SQ_ACTIVE_INST_VALU SQ_ACTIVE_INST_LDS SQ_WAIT_INST_LDS "
           "SQ_LDS_BANK_CONFLICT SQ_LDS_IDX_ACTIVE",
    "sq2": "SQ_WAIT_INST_ANY SQ_WAIT_ANY SQ_ACTIVE_INST_ANY SQ_INSTS_SALU SQ_BUSY_CYCLES SQ_WAVES SQ_INSTS_VMEM "
           "SQ_INSTS_SMEM",
}
# one call of each fused operation in the --kernels-only run: (summary name, kernels of the call, the main
# kernel whose SQ counters are listed, algorithmic bytes, state-steps for the VALU count, description)
PMC_CALLS = (
    ("ssm_bwd_cfg2", r"ssm_bwd_carry_kernel|ssm_bwd_kernel|bwd_finish_kernel", r"ssm_bwd_kernelI",
     2 * (5 * 8 * 2048 * 1536 + 4 * 8 * 2048 * 16 + 2 * 1536 * 16 + 2 * 1536), 8 * 2048 * 1536 * 16,
     "fused backward call at cfg2 (carry, main and finish kernels)"),
    ("ssm_fwd_cfg2", r"ssm_fwd_kernel", r"ssm_fwd_kernelIDF16_Li16ELi2ELi0E",
     2 * (3 * 8 * 2048 * 1536 + 2 * 8 * 2048 * 16 + 1536 * 16 + 1536), 8 * 2048 * 1536 * 16,
     "fused forward call with checkpoints at cfg2 (carry and main kernels)"),
    ("pscan_cfg4b", r"pscan_kernel|pscan_clear_kernel", r"pscan_kernel", 3 * 4 * 4 * 65536 * 1024, None,
     "parallel_scan_fn at cfg4b (clear and scan kernels)"),
)


def _profile_cmd(out, run, args):
    return (f"rocprofv3 --kernel-trace --stats -f csv -d {out}/trace_{run} -o run -- python3 {ROOT}/bench.py "
            + " ".join(args) + f" > {out}/trace_{run}.json")


def profile_recipe(out):
    """The shell commands behind profiles/*.txt (run from /tmp with TMPDIR=/tmp, one GPU)."""
    lines = ["cd /tmp && export TMPDIR=/tmp"]
    lines += [_profile_cmd(out, run, args) for run, args in TRACE_RUNS.items()]
    lines += [f"timeout -s KILL 120 rocprofv3 --pmc {c} -f csv -d {out}/pmc_{n} -o run -- python3 {ROOT}/bench.py "
              f"--kernels-only" for n, c in PMC_PASSES.items()]
    lines.append(f"python3 {ROOT}/bench.py --summarize {out}")
    return lines


def _short(k):
    m = re.search(r"(ssm_fwd_kernel|ssm_bwd_carry_kernel|ssm_bwd_kernel|bwd_finish_kernel|ssm_step_kernel|"
                  r"pscan_kernel|pscan_clear_kernel|copyBuffer)", k)
    name = m.group(1) if m else k[:48]
    if name == "ssm_fwd_kernel":
        mode = re.search(r"Li\d+ELi\d+ELi(\d)E", k)
        name += {"0": " (main)", "1": " (state-only)", "2": " (carry)"}.get(mode.group(1) if mode else "", "")
    return name


def _csv_rows(d, suffix):
    import csv
    import glob

    rows = []
    for f in sorted(glob.glob(os.path.join(d, "**", f"*{suffix}"), recursive=True)):
        rows += list(csv.DictReader(open(f)))
    return rows


def summarize(out, dest=None):
    """Writes profiles/*.txt from the rocprofv3 CSV output of the profile_recipe() commands in `out`."""
    import statistics

    dest = dest or os.path.join(ROOT, "profiles")
    written = []
    for run, args in TRACE_RUNS.items():
        d = os.path.join(out, f"trace_{run}")
        stats = _csv_rows(d, "kernel_stats.csv")
        if not stats:
            continue
        L = ["# rocprofv3 kernel statistics (MI355X, gfx950)",
             f"command: cd /tmp && export TMPDIR=/tmp && {_profile_cmd('<out>', run, args)}; "
             f"python3 bench.py --summarize <out>",
             "kernel | calls | avg_us | min_us | max_us | pct"]
        avg = {}
        for r in stats:
            k = r["Name"]
            avg[k] = float(r["AverageNs"]) / 1e3
            L.append(f"{_short(k)} [{k[:60]}] | {r['Calls']} | {avg[k]:.1f} | {float(r['MinNs']) / 1e3:.1f} | "
                     f"{float(r['MaxNs']) / 1e3:.1f} | {float(r['Percentage']):.2f}")
        fwd = sum(v for k, v in avg.items() if "ssm_fwd_kernel" in k and re.search(r"ELi[02]ELi\d+EEEv", k))
        bwd = sum(v for k, v in avg.items() if re.search(r"ssm_bwd_carry_kernel|ssm_bwd_kernel|bwd_finish_kernel", k))
        if fwd or bwd:
            L.append(f"fused forward call (carry + main kernels): {fwd:.1f} us; fused backward call (carry + main + "
                     f"finish kernels): {bwd:.1f} us")
        bj = os.path.join(out, f"trace_{run}.json")
        if os.path.exists(bj):
            try:
                line = json.loads([x for x in open(bj).read().splitlines() if x.startswith("{")][-1])
                keep = {k: line[k] for k in ("metric", "value", "unit", "ms_per_step", "us_per_step", "storage_dtype",
                                             "retained_after_forward_GB", "peak_hbm_allocated_GB", "kernels")
                        if k in line}
                if "roofline" in line:
                    keep["roofline"] = {k: line["roofline"][k] for k in ("achieved", "frac", "avg_launch_ms")
                                        if k in line["roofline"]}
                keep["workload"] = line.get("config", {}).get("workload")
                L.append("bench line under the profiler: " + json.dumps(keep))
            except (ValueError, IndexError):
                pass
        name = f"kernel_trace_{run}.txt"
        open(os.path.join(dest, name), "w").write("\n".join(L) + "\n")
        written.append(name)

    # counter passes: per kernel name, the median over its dispatches of each counter (for the copy
    # kernel, the largest dispatch: the 1 GiB calibration copy, not the small copies of status reads)
    def pmc(n):
        per = {}
        for r in _csv_rows(os.path.join(out, f"pmc_{n}"), "counter_collection.csv"):
            key = (r["Kernel_Name"], r["Dispatch_Id"])
            per.setdefault(key, {}).setdefault(r["Counter_Name"], 0.0)
            per[key][r["Counter_Name"]] += float(r["Counter_Value"])
        agg = {}
        for (k, _), cs in per.items():
            for c, v in cs.items():
                agg.setdefault(k, {}).setdefault(c, []).append(v)
        return {k: {c: (max(v) if "copyBuffer" in k else statistics.median(v)) for c, v in cs.items()}
                for k, cs in agg.items()}

    F, W, S1, S2 = pmc("fetch"), pmc("write"), pmc("sq1"), pmc("sq2")
    copies = [k for k in F if "copyBuffer" in k]
    if F and W and copies:
        copy = copies[0]
        gib = float(1 << 30)
        fcal = gib / (F[copy]["FETCH_SIZE"] * 1024)
        wcal = gib / (W[[k for k in W if "copyBuffer" in k][0]]["WRITE_SIZE"] * 1024)
        for name, pat, main_pat, alg, nstate_steps, what in PMC_CALLS:
            ks = [k for k in F if re.search(pat, k)]
            if not ks:
                continue
            fb = sum(F[k]["FETCH_SIZE"] for k in ks) * 1024 * fcal
            wb = sum(W[k]["WRITE_SIZE"] for k in W if re.search(pat, k)) * 1024 * wcal
            L = [f"# rocprofv3 --pmc summary (MI355X, gfx950), one {what}",
                 "command: cd /tmp && export TMPDIR=/tmp && for each pass: timeout -s KILL 120 rocprofv3 --pmc "
                 "<counters> -f csv -d <out>/pmc_<pass> -o run -- python3 bench.py --kernels-only; then "
                 "python3 bench.py --summarize <out>. Passes: "
                 + "; ".join(f"{n}: {c}" for n, c in PMC_PASSES.items()),
                 f"calibration: a 1 GiB device copy reads FETCH_SIZE={F[copy]['FETCH_SIZE']:.4g} KiB and "
                 f"WRITE_SIZE={W[[k for k in W if 'copyBuffer' in k][0]]['WRITE_SIZE']:.4g} KiB -> scale FETCH by "
                 f"{fcal:.3f}, WRITE by {wcal:.3f} (bytes moved = counter KiB x 1024 x scale)",
                 "kernels: " + ", ".join(sorted({_short(k) for k in ks})),
                 f"fetch_bytes_per_launch: {fb:.4g}", f"write_bytes_per_launch: {wb:.4g}",
                 f"traffic_bytes_per_launch: {fb + wb:.6g}", f"algorithmic_bytes_per_launch: {alg}",
                 f"traffic_over_algorithmic: {(fb + wb) / alg:.3f}"]
            mains = [k for k in S1 if re.search(main_pat, k)]
            if mains:
                m = mains[0]
                sq = dict(S1[m])
                sq.update(S2.get([k for k in S2 if re.search(main_pat, k)][0], {}) if S2 else {})
                L.append(f"SQ counters of {_short(m)}: " + ", ".join(f"{c}={v:.4g}" for c, v in sorted(sq.items())))
                wc = sq.get("SQ_WAVE_CYCLES")
                if wc:
                    L.append(f"per wave-cycle: VALU busy {sq['SQ_ACTIVE_INST_VALU'] / wc:.3f}, LDS busy "
                             f"{sq['SQ_ACTIVE_INST_LDS'] / wc:.3f}, waiting on LDS {sq['SQ_WAIT_INST_LDS'] / wc:.3f}, "
                             f"waiting on anything {sq.get('SQ_WAIT_ANY', 0) / wc:.3f}")
                if nstate_steps:
                    L.append(f"main_kernel_valu_instructions_per_state_step: "
                             f"{sq['SQ_INSTS_VALU'] * 64 / nstate_steps:.3f}")
            # the call's other kernels: issue use of the carry passes (at cfg2 they scan half of L) and the
            # finishing kernel's bytes against its traced duration
            durs = {r["Name"]: float(r["AverageNs"]) for r in _csv_rows(os.path.join(out, "trace_cfg2_fwd_bwd"),
                                                                      "kernel_stats.csv")}
            for k in sorted(set(ks) - set(mains[:1])):
                sq = dict(S1.get(k, {}))
                sq.update(S2.get(k, {}))
                kb = F[k]["FETCH_SIZE"] * 1024 * fcal + W.get(k, {}).get("WRITE_SIZE", 0.0) * 1024 * wcal
                parts = [f"{_short(k)}: {kb:.4g} bytes moved"]
                if k in durs and durs[k] > 0:
                    parts.append(f"{kb / durs[k]:.4g} GB/s over its traced {durs[k] / 1e3:.1f} us")
                wc = sq.get("SQ_WAVE_CYCLES")
                if wc:
                    parts.append(f"VALU busy {sq['SQ_ACTIVE_INST_VALU'] / wc:.3f} and LDS busy "
                                 f"{sq['SQ_ACTIVE_INST_LDS'] / wc:.3f} per wave-cycle")
                if nstate_steps and "carry" in _short(k) and "SQ_INSTS_VALU" in sq:
                    parts.append(f"{sq['SQ_INSTS_VALU'] * 64 / (nstate_steps / 2):.3f} VALU instructions per "
                                 f"state-step of the half of L it scans")
                L.append("; ".join(parts))
            fname = f"{name}_pmc.txt"
            open(os.path.join(dest, fname), "w").write("\n".join(L) + "\n")
            written.append(fname)
    return written


# The reference's own benchmark procedures (benchmark.py:26-253): the same shapes, input distributions,
# warm-up and iteration counts and wall-clock timing around torch.cuda.synchronize(). Its published
# figures (NVIDIA RTX 5070 Laptop GPU, BENCHMARK_RESULTS.md:12-34) are printed beside these for
# context only: other hardware, and its "Fused" columns come from an extension that does not build.
REF_FWD_MS = {(1, 512, 256): (2.50, 1.80), (1, 1024, 256): (5.10, 3.40), (1, 2048, 512): (15.20, 9.80),
              (1, 4096, 768): (45.30, 28.50), (1, 8192, 1024): (120.50, 72.30), (1, 16384, 2048): (350.20, 195.80)}
REF_TRAIN_MS = {(1, 512, 256): (8.50, 5.20, 6.10), (1, 1024, 256): (18.20, 10.50, 12.80),
                (1, 2048, 512): (55.80, 30.20, 38.50), (1, 4096, 768): (165.50, 85.20, 110.50)}
REF_MEM_MB = {"Original": (245.3, 892.1), "Fused(ckpt0)": (198.5, 756.2), "Fused(ckpt1)": (152.8, 523.4)}


def reference_suite():
    """benchmark_forward_only / benchmark_forward_backward / benchmark_memory of the reference, run
    through this package: "Original" is SelectiveScanCuda, "Fused(ckpt0/1)" FusedSelectiveScan."""
    import torch

    from mamba_windows_cuda import FusedSelectiveScan, SelectiveScanCuda

    dev, N = "cuda", 16
    torch.manual_seed(0)
    orig, fused0, fused1 = SelectiveScanCuda(), FusedSelectiveScan(0), FusedSelectiveScan(1)

    def wall_ms(fn, n):
        torch.cuda.synchronize()
        t = time.time()
        for _ in range(n):
            fn()
        torch.cuda.synchronize()
        return (time.time() - t) / n * 1e3

    res = {"suite": "the reference's benchmark.py procedures (wall clock, synchronize)", "forward_fp16": [],
           "train_fp32": [], "memory_fp32_B1_L4096_D768": []}
    _ref_forward(res, orig, fused0, wall_ms, dev, N)
    _ref_train(res, orig, fused0, fused1, wall_ms, dev, N)
    _ref_memory(res, orig, fused0, fused1, dev, N)
    return res


def _ref_train_inputs(B, L, D, dev, N):
    import torch

    return [torch.randn(B, L, D, device=dev), torch.ones(B, L, D, device=dev) * 0.01,
            -torch.rand(D, N, device=dev) * 0.1, torch.randn(B, L, N, device=dev) * 0.1,
            torch.randn(B, L, N, device=dev) * 0.1, torch.ones(D, device=dev) * 0.1]


# (each section in a function of its own, so that its tensors are freed before the next one runs)
def _ref_forward(res, orig, fused0, wall_ms, dev, N):
    import torch

    for (B, L, D), ref in REF_FWD_MS.items():
        x = (torch.randn(B, L, D, device=dev).half(), torch.ones(B, L, D, device=dev).half(),
             (-torch.rand(D, N, device=dev) * 0.1).half(), torch.randn(B, L, N, device=dev).half(),
             torch.randn(B, L, N, device=dev).half(), torch.ones(D, device=dev).half())
        for _ in range(5):
            orig(*x)
            fused0(*x)
        t_o, t_f = wall_ms(lambda: orig(*x), 50), wall_ms(lambda: fused0(*x), 50)
        res["forward_fp16"].append({"B": B, "L": L, "D": D, "original_ms": t_o, "fused_ms": t_f,
                                    "reference_rtx5070_original_fused_ms": ref})


def _ref_train(res, orig, fused0, fused1, wall_ms, dev, N):
    for (B, L, D), ref in REF_TRAIN_MS.items():
        base = _ref_train_inputs(B, L, D, dev, N)
        row = {"B": B, "L": L, "D": D}
        for name, k in (("original_ms", orig), ("fused_ckpt0_ms", fused0), ("fused_ckpt1_ms", fused1)):
            leaves = [t.clone().requires_grad_(True) for t in base]

            def step():
                for t in leaves:
                    t.grad = None
                out, h = k.forward_with_state(*leaves)
                (out.sum() + h.sum()).backward()

            for _ in range(3):
                step()
            row[name] = wall_ms(step, 20)
        row["reference_rtx5070_original_ckpt0_ckpt1_ms"] = ref
        res["train_fp32"].append(row)


def _ref_memory(res, orig, fused0, fused1, dev, N):
    import torch

    for name, k in (("Original", orig), ("Fused(ckpt0)", fused0), ("Fused(ckpt1)", fused1)):
        torch.cuda.reset_peak_memory_stats()
        torch.cuda.empty_cache()
        x = _ref_train_inputs(1, 4096, 768, dev, N)
        leaves = [x[0].requires_grad_(True), torch.ones(1, 4096, 768, device=dev, requires_grad=True) * 0.01] + \
                 [t.requires_grad_(True) for t in x[2:]]  # delta as the reference builds it (not a leaf)
        out, h = k.forward_with_state(*leaves)
        fwd_mb = torch.cuda.max_memory_allocated() / 2**20
        (out.sum() + h.sum()).backward()
        res["memory_fp32_B1_L4096_D768"].append({"name": name, "forward_mb": fwd_mb,
                                                  "total_mb": torch.cuda.max_memory_allocated() / 2**20,
                                                  "reference_rtx5070_forward_total_mb": REF_MEM_MB[name]})
        del x, leaves, out, h


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default="cfg2", choices=["cfg2", "cfg3", "cfg4a", "cfg4b"])
    ap.add_argument("--level", type=int, default=0, choices=[0, 1])
    ap.add_argument("--skip-cpu", action="store_true")
    ap.add_argument("--decode", type=int, nargs="?", const=0, default=None, metavar="BATCH",
                    help="time the L=1 decode step at the config's D (batch defaults to the config's)")
    ap.add_argument("--transforms", action="store_true",
                    help="time the scan call with delta_bias/softplus/z gating fused vs. as torch passes")
    ap.add_argument("--shard", type=int, default=1, choices=[1, 2, 4, 8],
                    help="time one GPU's share of the config when D is split over this many GPUs")
    ap.add_argument("--graph", action="store_true",
                    help="replay the fwd+bwd step from a HIP graph (no host path per step)")
    ap.add_argument("--kernels-only", action="store_true",
                    help="profiling driver: fused calls, cfg4b scan and a 1 GiB copy; no timing")
    ap.add_argument("--nstate", type=int, default=16, choices=[8, 16, 32, 64],
                    help="state count N of the fwd+bwd step (the reference builds N=16 only)")
    ap.add_argument("--dtype", default=None, choices=sorted(DTYPES),
                    help="storage dtype of the fwd+bwd step (default: the config's)")
    ap.add_argument("--profile-recipe", metavar="DIR", default=None,
                    help="print the rocprofv3 commands whose output --summarize turns into profiles/*.txt")
    ap.add_argument("--reference-suite", action="store_true",
                    help="run the reference's benchmark.py procedures (forward fp16, fwd+bwd fp32, memory)")
    ap.add_argument("--summarize", metavar="DIR", default=None,
                    help="write profiles/*.txt from the rocprofv3 CSV output in DIR (no GPU needed)")
    args = ap.parse_args()
    if args.profile_recipe:
        print("\n".join(profile_recipe(args.profile_recipe)))
        return
    if args.summarize:
        print(json.dumps({"written": summarize(args.summarize)}))
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(json.dumps({"error": "this build measures one GPU only (sharding over GPUs is designed, not "
                                   "built); run with --gpus 1"}))
        sys.exit(2)
    import torch

    if not torch.cuda.is_available():
        print(json.dumps({"error": "no HIP device visible"}))
        sys.exit(1)
    if args.kernels_only:
        print(json.dumps(kernels_only(args.config if args.config in ("cfg2", "cfg3") else "cfg2")))
        return
    if args.reference_suite:
        print(json.dumps(reference_suite()))
        return
    if args.decode is not None:
        res = bench_decode(args.config if args.config in ("cfg2", "cfg3") else "cfg2", args.steps, args.warmup,
                           args.decode or None)
        args.skip_cpu = True
    elif args.transforms:
        res = bench_transforms(args.config if args.config in ("cfg2", "cfg3") else "cfg2", args.steps, args.warmup)
        args.skip_cpu = True
    elif args.config == "cfg4b":
        res = bench_pscan(args.steps, args.warmup)
    elif args.config == "cfg4a":
        res = bench_stream(args.steps, args.warmup)
    else:
        res = bench_ssm(args.config, args.steps, args.warmup, args.level, args.shard, args.nstate, args.dtype,
                        args.graph)
        res["peak_hbm_allocated_GB"] = torch.cuda.max_memory_allocated() / 1e9
        if args.shard > 1 or args.nstate != 16 or args.dtype is not None or args.graph:
            args.skip_cpu = True
    res.update({"n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "higher_is_better": True,
                "scaling": "weak", "vs_baseline": None, "data": "synthetic (seeded; BASELINE.json distributions)",
                "device": torch.cuda.get_device_name(0)})
    if not args.skip_cpu and args.config in ("cfg2", "cfg3"):
        res["cpu_baseline"] = cpu_baseline(args.config)
    elif not args.skip_cpu and args.config == "cfg4b":
        res["cpu_baseline"] = cpu_baseline_pscan()
    print(json.dumps(res))


if __name__ == "__main__":
    main()
