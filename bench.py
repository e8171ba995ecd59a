"""Benchmark of the Mira mixer hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-stack] [--no-traffic]
                    [--only LEG ...]

Headline (BASELINE.json `metric`, `configs[1]`): bf16 prefill of the depthwise causal conv
(width 4) + diagonal decay scan at B=8, T=4096, D=2048 with a carried-in fp32 state, inputs
resident in HBM. A step is one mira_diag_conv_scan launch over the whole batch; `value` is
tokens/s over exactly K timed steps. Beside it: the decode leg (`configs[3]`, batch 256,
128 steps of conv+diag and GLA matrix-state updates), the roofline of the dominant kernel from
HIP events on the launch stream, and the CPU oracle timed on the host's cores on a bounded
sample of the same workload. Also reported, not headline: the GLA chunked prefill (`configs[2]`,
% HBM and % MFMA), the reference operator matrix_lattice_iir at the cfg5 mixer geometry
(K=2, M=64), matrix_lattice_iir_control (coefficients formed inside the scan) at the
reference's own mixer geometry against its materialised path, and the 24-layer MiraLLM forward
of `configs[4]` with the mixer's and the scan's share of its time (skip it with --no-stack), and a
training step of the scan (forward + backward) at the reference's mira-s and the cfg5 geometry,
and the MiraMixer module at the shapes the reference quotes its own mixer numbers for.
The headline kernel's HBM traffic is measured in the same run by two rocprofv3 --pmc child runs
(FETCH_SIZE, WRITE_SIZE) started before this process initialises the GPU (skip with
--no-traffic). `--only LEG` runs the headline plus the named legs (`--only prefill`: the headline
alone), which is how each kernel is profiled on its own. Prints one JSON line.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "official-mira-llm_amd"))

HBM_PEAK_GBS = 8000.0
LEGS = ("decode", "gla", "lattice", "control", "backward", "mixer", "stack")
ONLY = ("prefill",) + LEGS
CALIBRATION_KERNEL = "neg_kernel"                 # torch.neg over 64 Mi bf16 elements:
CALIBRATION_KIB = 131072.0                         # it reads 128 MiB and writes 128 MiB
METRIC = "prefill scan tokens/s + % HBM roofline; decode steps/s at batch 256"
PROFILES = os.path.join(ROOT, "profiles")


def parse():
    parser = argparse.ArgumentParser()
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=50)
    parser.add_argument("--warmup", type=int, default=5)
    parser.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    parser.add_argument("--no-stack", action="store_true",
                        help="skip the 24-layer MiraLLM forward (BASELINE configs[4])")
    parser.add_argument("--decode-steps", type=int, default=128)
    parser.add_argument("--calibrate", action="store_true",
                        help="also run an elementwise kernel of known traffic (torch.neg: reads "
                             "and writes 128 MiB each) five times, to scale rocprofv3 FETCH_SIZE / "
                             "WRITE_SIZE")
    parser.add_argument("--only", action="append", choices=ONLY, default=None,
                        help="run only these legs (repeatable), e.g. to profile one kernel; the "
                             "headline prefill leg always runs")
    parser.add_argument("--no-traffic", action="store_true",
                        help="skip the live rocprofv3 FETCH_SIZE / WRITE_SIZE runs of the headline "
                             "kernel")
    parser.add_argument("--traffic-child", action="store_true", help=argparse.SUPPRESS)
    return parser.parse_args()


def _prefill_inputs(torch):
    B, T, D = 8, 4096, 2048
    g = torch.Generator(device="cuda").manual_seed(0)
    x = torch.randn(B, T, D, device="cuda", generator=g).to(torch.bfloat16)
    a = torch.sigmoid(torch.rand(B, T, D, device="cuda", generator=g) * 4 + 2).to(torch.bfloat16)
    w = torch.randn(D, 4, device="cuda", generator=g) * 0.5
    bias = torch.zeros(D, device="cuda")
    h0 = torch.randn(B, D, device="cuda", generator=g) * 0.1
    return (B, T, D), (x, a, w, bias, h0)


def traffic_child():
    """What the traffic measurement profiles: the calibration copy (torch.neg over 64 Mi bf16
    elements: 128 MiB read, 128 MiB written; no other kernel of this process is a neg) and the
    headline prefill kernel, three times each."""
    import torch

    from mira_amd import mira

    _, (x, a, w, bias, h0) = _prefill_inputs(torch)
    calibrate(torch, 3)
    for _ in range(3):
        mira.diag_conv_scan(x, a, w, bias, h0=h0, return_state=True)
    torch.cuda.synchronize()


def calibrate(torch, times):
    """The copy of known traffic that scales rocprofv3's FETCH_SIZE and WRITE_SIZE readings."""
    source = torch.ones(64 << 20, device="cuda", dtype=torch.bfloat16)
    target = torch.empty_like(source)
    for _ in range(times):
        torch.neg(source, out=target)
    torch.cuda.synchronize()


def measure_traffic(kernel="diag_column_kernel"):
    """HBM bytes per launch of the headline kernel in this run: two rocprofv3 --pmc child runs of
    `bench.py --traffic-child` (FETCH_SIZE, then WRITE_SIZE: one TCC counter set per run), each
    counter scaled by what it reads for the calibration copy of known size. Run before this
    process touches the GPU. Returns (dict or None, reason)."""
    import csv
    import glob
    import shutil
    import subprocess
    import tempfile

    profiler = shutil.which("rocprofv3") or "/opt/rocm/bin/rocprofv3"
    if not os.path.exists(profiler):
        return None, "rocprofv3 not found"
    measured = {}
    for counter in ("FETCH_SIZE", "WRITE_SIZE"):
        out = tempfile.mkdtemp(prefix=f"mira_{counter.lower()}_", dir="/tmp")
        command = [profiler, "--pmc", counter, "--output-format", "csv", "-d", out, "-o", "t",
                   "--", sys.executable, os.path.abspath(__file__), "--traffic-child"]
        try:
            subprocess.run(command, cwd="/tmp", env=dict(os.environ, TMPDIR="/tmp"),
                           stdout=subprocess.DEVNULL, stderr=subprocess.DEVNULL, timeout=150,
                           check=False)
        except subprocess.TimeoutExpired:
            return None, f"rocprofv3 --pmc {counter} did not finish in 150 s"
        rows = []
        for path in glob.glob(os.path.join(out, "**", "*counter_collection.csv"), recursive=True):
            with open(path) as handle:
                rows += list(csv.DictReader(handle))
        shutil.rmtree(out, ignore_errors=True)
        values = {"kernel": [], "calibration": []}
        for row in rows:
            name = row.get("Kernel_Name", "")
            if kernel in name:
                values["kernel"].append(float(row["Counter_Value"]))
            elif CALIBRATION_KERNEL in name:
                values["calibration"].append(float(row["Counter_Value"]))
        if not values["kernel"] or not values["calibration"]:
            return None, f"rocprofv3 --pmc {counter} returned no rows for the kernel or the copy"
        scale = CALIBRATION_KIB / (sum(values["calibration"]) / len(values["calibration"]))
        measured[counter] = (sum(values["kernel"]) / len(values["kernel"]) * scale * 1024, scale)
    fetch, write = measured["FETCH_SIZE"], measured["WRITE_SIZE"]
    return {"bytes": round(fetch[0] + write[0]), "fetch_bytes": round(fetch[0]),
            "write_bytes": round(write[0]), "fetch_scale": round(fetch[1], 4),
            "write_scale": round(write[1], 4)}, ""


def prefill_leg(torch, mira, steps, warmup):
    (B, T, D), (x, a, w, bias, h0) = _prefill_inputs(torch)
    for _ in range(warmup):
        mira.diag_conv_scan(x, a, w, bias, h0=h0, return_state=True)
    # one launch per step, back to back on the launch stream; HIP events around the timed
    # region give the average launch duration (the host enqueues faster than the GPU runs them)
    stream = torch.cuda.current_stream()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start.record(stream)
    for _ in range(steps):
        mira.diag_conv_scan(x, a, w, bias, h0=h0, return_state=True)
    end.record(stream)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    kernel_s = start.elapsed_time(end) * 1e-3 / steps
    algorithmic = B * T * D * 6 + B * D * 4 * 2 + D * 4 * 4 + D * 4
    watchdog = mira.diag_workspace_error()
    return {
        "tokens": B * T, "elapsed": elapsed, "kernel_s": kernel_s, "algorithmic": algorithmic,
        "watchdog": watchdog,
    }


def decode_leg(torch, mira, steps):
    """256 sequences, one token each per step; per step the conv ring, the
    diagonal state and the GLA matrix state [256,16,128,128] are read and written in HBM."""
    B, D, H, d = 256, 2048, 16, 128
    g = torch.Generator(device="cuda").manual_seed(1)
    h = torch.randn(B, D, device="cuda", generator=g) * 0.1
    ring = (torch.randn(B, D, 3, device="cuda", generator=g) * 0.1).to(torch.bfloat16)
    S = torch.randn(B, H, d, d, device="cuda", generator=g) * 0.1
    xs = torch.randn(steps, B, D, device="cuda", generator=g).to(torch.bfloat16)
    as_ = torch.sigmoid(torch.rand(steps, B, D, device="cuda", generator=g) * 4 + 2).to(torch.bfloat16)
    w = torch.randn(D, 4, device="cuda", generator=g) * 0.5
    qs = torch.nn.functional.normalize(torch.randn(steps, B, H, d, device="cuda", generator=g), dim=-1).bfloat16()
    ks = torch.nn.functional.normalize(torch.randn(steps, B, H, d, device="cuda", generator=g), dim=-1).bfloat16()
    vs = torch.randn(steps, B, H, d, device="cuda", generator=g).bfloat16()
    gs = torch.rand(steps, B, H, device="cuda", generator=g) * -0.099 - 0.001
    y = torch.empty(B, D, device="cuda", dtype=torch.bfloat16)
    o = torch.empty(B, H, d, device="cuda", dtype=torch.bfloat16)

    def run(n):
        for t in range(n):
            mira.diag_conv_step(xs[t], as_[t], w, None, h, ring, pos=t, out=y)
            mira.gla_step(qs[t], ks[t], vs[t], gs[t], S, out=o)

    run(4)
    stream = torch.cuda.current_stream()
    gla_start = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    gla_end = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for t in range(steps):
        mira.diag_conv_step(xs[t], as_[t], w, None, h, ring, pos=t, out=y)
        gla_start[t].record(stream)
        mira.gla_step(qs[t], ks[t], vs[t], gs[t], S, out=o)
        gla_end[t].record(stream)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    gla_s = sum(s.elapsed_time(e) for s, e in zip(gla_start, gla_end)) * 1e-3 / steps
    # the same steps as a serving loop runs them: the 2 x `steps` launches captured once as a HIP
    # graph (the step kernels take no workspace and record no memset) and replayed
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run(steps)
    graph.replay()
    torch.cuda.synchronize()
    replays = 3
    t0 = time.perf_counter()
    for _ in range(replays):
        graph.replay()
    torch.cuda.synchronize()
    serial_elapsed = (time.perf_counter() - t0) / replays
    # the two ops of a step are independent: each step forks the conv + diagonal step onto a side
    # stream beside the GLA step and joins before the next step (steps stay in order), so the
    # latency-bound diagonal step hides under the HBM-bound GLA step
    main, side = torch.cuda.current_stream(), torch.cuda.Stream()
    overlapped = torch.cuda.CUDAGraph()
    with torch.cuda.graph(overlapped):
        for t in range(steps):
            side.wait_stream(main)
            with torch.cuda.stream(side):
                mira.diag_conv_step(xs[t], as_[t], w, None, h, ring, pos=t, out=y)
            mira.gla_step(qs[t], ks[t], vs[t], gs[t], S, out=o)
            main.wait_stream(side)
    overlapped.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(replays):
        overlapped.replay()
    torch.cuda.synchronize()
    graph_elapsed = (time.perf_counter() - t0) / replays
    per_step = (B * H * d * d * 4 * 2 + B * H * d * 2 * 4 + B * H * 4      # GLA state, q k v o, g
                + B * D * 4 * 2 + B * D * 2 * 3 + B * D * 2 * 3 + B * D * 2)  # h, x a y, ring r+w
    gla_bytes = B * H * d * d * 4 * 2 + B * H * d * 2 * 4 + B * H * 4
    return {"steps": steps, "elapsed": elapsed, "graph_elapsed": graph_elapsed,
            "serial_elapsed": serial_elapsed, "per_step_bytes": per_step, "gla_kernel_s": gla_s,
            "gla_bytes": gla_bytes}


def gla_prefill_leg(torch, mira, steps, warmup):
    """the matrix-state chunked scan (GLA), bf16 q/k/v, fp32 state, chunk 64,
    B=4 T=8192 H=16 d=128, carried-in and returned state. One step = one mira_gla_chunked launch."""
    B, T, H, d = 4, 8192, 16, 128
    g = torch.Generator(device="cuda").manual_seed(2)
    q = torch.nn.functional.normalize(torch.randn(B, T, H, d, device="cuda", generator=g), dim=-1).bfloat16()
    k = torch.nn.functional.normalize(torch.randn(B, T, H, d, device="cuda", generator=g), dim=-1).bfloat16()
    v = torch.randn(B, T, H, d, device="cuda", generator=g).bfloat16()
    gd = torch.rand(B, T, H, device="cuda", generator=g) * -0.099 - 0.001
    S0 = torch.randn(B, H, d, d, device="cuda", generator=g) * 0.1
    for _ in range(warmup):
        mira.gla_chunked(q, k, v, gd, state=S0, return_state=True)
    stream = torch.cuda.current_stream()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start.record(stream)
    for _ in range(steps):
        mira.gla_chunked(q, k, v, gd, state=S0, return_state=True)
    end.record(stream)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    kernel_s = start.elapsed_time(end) * 1e-3 / steps
    algorithmic = B * T * H * d * 2 * 4 + B * T * H * 4 + B * H * d * d * 4 * 2
    flops = B * T * H * 6 * d * d      # per (token, head): 2d^2 state update, 2d^2 readout, 2d^2 intra
    return {"tokens": B * T, "steps": steps, "elapsed": elapsed, "kernel_s": kernel_s,
            "algorithmic": algorithmic, "flops": flops}


def lattice_leg(torch, mira, steps, warmup):
    """The reference operator itself, matrix_lattice_iir (model/mira_mixer.py:246-387), at the
    cfg5 mixer geometry (lattice_d_e 2048, order 2, memory 64; B=4 T=2048), bf16 in/out, fp32
    state in and out, arch cauchy_x_hyperbolic. Bytes per call (reference-native):
    B*T*C*2*(3K+4) + B*T*2*M*(K+2) + 2*B*K*C*M*4; fp32 flops B*T*C*M*(9K+4)."""
    B, T, C, K, M = 4, 2048, 2048, 2, 64
    g = torch.Generator(device="cuda").manual_seed(3)
    bf = torch.bfloat16
    x = (torch.randn(B, T, C, device="cuda", generator=g) * 0.15).to(bf)
    alpha = (torch.randn(B, T, C, K, device="cuda", generator=g) * 0.12).to(bf)
    beta = (torch.randn(B, T, C, K, device="cuda", generator=g) * 0.12).to(bf)
    rho = (torch.randn(B, T, C, K + 1, device="cuda", generator=g) * 0.12).to(bf)
    gamma = torch.randn(B, T, C, device="cuda", generator=g).to(bf)
    write = torch.nn.functional.silu(torch.randn(B, T, M, device="cuda", generator=g)).to(bf)
    read = (torch.randn(B, T, K + 1, M, device="cuda", generator=g) * 0.12).to(bf)
    state = torch.randn(B, K, C, M, device="cuda", generator=g) * 0.1

    def call():
        return mira.matrix_lattice_iir(x, alpha, rho, gamma, write, read, raw_beta=beta,
                                       state=state, return_state=True)

    for _ in range(warmup):
        call()
    stream = torch.cuda.current_stream()
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    torch.cuda.synchronize()
    for i in range(steps):
        starts[i].record(stream)
        call()
        ends[i].record(stream)
    torch.cuda.synchronize()
    call_s = sum(s.elapsed_time(e) for s, e in zip(starts, ends)) * 1e-3 / steps
    nbytes = B * T * C * 2 * (3 * K + 4) + B * T * 2 * M * (K + 2) + 2 * B * K * C * M * 4
    flops = B * T * C * M * (9 * K + 4)

    # the operator's decode: one token for 256 sequences with the state updated in place
    # (matrix_lattice_step, the prefix-cache step of a served MIRA layer)
    SB = 256
    step_in = [(torch.randn(SB, 1, *shape, device="cuda", generator=g) * 0.12).to(bf)
               for shape in ((C,), (C, K), (C, K + 1), (C,), (M,), (K + 1, M), (C, K))]
    step_in[4] = torch.nn.functional.silu(step_in[4])
    step_state = torch.randn(SB, K, C, M, device="cuda", generator=g) * 0.1
    step_out = torch.empty(SB, 1, C, device="cuda", dtype=bf)

    def step():
        mira.matrix_lattice_step(*step_in, step_state, out=step_out, inplace=True)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    starts[0].record(stream)
    for _ in range(steps * 4):
        step()
    ends[0].record(stream)
    torch.cuda.synchronize()
    step_s = starts[0].elapsed_time(ends[0]) * 1e-3 / (steps * 4)
    step_bytes = 2 * SB * K * C * M * 4 + SB * C * 2 * (3 * K + 4) + SB * 2 * M * (K + 2)
    return {"tokens": B * T, "call_s": call_s, "bytes": nbytes, "flops": flops,
            "shape": f"B={B} T={T} C={C} K={K} M={M}", "step_s": step_s,
            "step_bytes": step_bytes, "step_shape": f"B={SB} T=1 C={C} K={K} M={M}"}


def control_leg(torch, mira, steps, warmup):
    """matrix_lattice_iir_control (mira.py:1840-1894) at the reference's own mixer geometry
    (K=2, d_e 1536, d_m 16, d_r 48, cauchy_x_hyperbolic) at a batch that fills the GPU in one
    token chunk, B=256 T=512: the scan forms alpha, beta and rho from the control on the matrix
    cores, against the materialised path (the coefficient GEMM, then matrix_lattice_iir) on the
    same inputs. The kernel alone is also timed through the C-ABI, with memory_read projected
    beforehand. Algorithmic bytes of the kernel: x, gamma, y 6 B per (t,c) + control 2 d_r + s,
    nu 2 (K+2) M per token; fp32 VALU flops B*T*C*M*(9K+4)."""
    import torch.nn.functional as F

    from mira_amd import _lib

    B, T, C, K, M, R = 256, 512, 1536, 2, 16, 48
    arch = "cauchy_x_hyperbolic"
    g = torch.Generator(device="cuda").manual_seed(8)
    bf = torch.bfloat16
    total = C * (3 * K + 1) + (K + 1) * M
    spans = ((0, C * K), (C * K, 2 * C * K), (2 * C * K, C * (3 * K + 1)), (C * (3 * K + 1), total))
    weight = (torch.randn(total, R, device="cuda", generator=g) / R ** 0.5).to(bf)
    bias = (0.3 * torch.randn(total, device="cuda", generator=g)).to(bf)
    control = F.silu(torch.randn(B, T, R, device="cuda", generator=g)).to(bf)
    packed = torch.randn(B, T, 2 * C, device="cuda", generator=g).to(bf)
    x, gamma = packed[..., :C], packed[..., C:]
    write = (torch.randn(B, T, M, device="cuda", generator=g) / 4).to(bf)
    read = F.linear(control, weight[spans[3][0]:], bias[spans[3][0]:]).contiguous()
    plan = mira._control_plan(x, control, weight, bias, gamma, write, K, M)
    assert plan is not None, "the control scan does not serve the bench shape"
    lib = _lib.require()
    out = torch.empty(B, T, C, device="cuda", dtype=bf)
    stream = torch.cuda.current_stream()

    def fused():
        return mira.matrix_lattice_iir_control(x, control, weight, bias, spans, gamma, write,
                                               arch=arch)

    def kernel():
        lib.mira_lattice_control_forward(
            x.data_ptr(), plan[0], control.data_ptr(), weight.data_ptr(), R, total,
            bias.data_ptr(), spans[0][0], spans[1][0], spans[2][0], gamma.data_ptr(), plan[1],
            write.data_ptr(), read.data_ptr(), (K + 1) * M, None, None, None, out.data_ptr(),
            B, T, C, K, M, R, _lib.BF16, mira.ARCH_STAGE[arch], stream.cuda_stream)

    def materialised():
        coefficients = F.linear(control, weight, bias)
        alpha, beta, rho, nu = coefficients.split(tuple(hi - lo for lo, hi in spans), dim=-1)
        return mira.matrix_lattice_iir(
            x, alpha.view(B, T, C, K), rho.view(B, T, C, K + 1), gamma, write,
            nu.view(B, T, K + 1, M), raw_beta=beta.view(B, T, C, K), arch=arch)

    def timed(fn):
        with torch.no_grad():
            start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            start.record(stream)
            for _ in range(steps):
                fn()
            end.record(stream)
            torch.cuda.synchronize()
        return start.elapsed_time(end) * 1e-3 / steps

    with torch.no_grad():
        for _ in range(warmup):
            fused(), kernel(), materialised()
    call_s, kernel_s, materialised_s = timed(fused), timed(kernel), timed(materialised)
    with torch.no_grad():
        same = float((fused() == materialised()).float().mean())
    nbytes = B * T * C * 6 + B * T * (2 * R + 2 * (K + 2) * M)
    return {"tokens": B * T, "call_s": call_s, "kernel_s": kernel_s,
            "materialised_s": materialised_s, "bytes": nbytes, "flops": B * T * C * M * (9 * K + 4),
            "identical": same, "shape": f"B={B} T={T} C={C} K={K} M={M} d_r={R}"}


def backward_leg(torch, mira, steps, warmup):
    """A training step of the scan: matrix_lattice_iir under autograd (the forward at the
    backward's chunk length, keeping every chunk's entering state) and its backward (all seven
    gradients: mira_lattice_backward), bf16 in/out, fp32 arithmetic, zero initial state, at the
    reference's mira-s mixer geometry (d_e 1536, K 2, d_m 16) over B=8 T=2048 and at the cfg5
    geometry (d_e 2048, K 2, d_m 64, B=4 T=2048). Times the forward alone and forward + backward
    with HIP events on the launch stream."""
    results = {}
    bf = torch.bfloat16
    for label, (B, T, C, K, M) in (("mira_s", (8, 2048, 1536, 2, 16)),
                                   ("cfg5", (4, 2048, 2048, 2, 64))):
        g = torch.Generator(device="cuda").manual_seed(11)
        shapes = ((B, T, C), (B, T, C, K), (B, T, C, K + 1), (B, T, C), (B, T, M),
                  (B, T, K + 1, M), (B, T, C, K))
        tensors = [(torch.randn(*shape, device="cuda", generator=g) * 0.15).to(bf).requires_grad_()
                   for shape in shapes]
        dy = torch.randn(B, T, C, device="cuda", generator=g).to(bf)
        stream = torch.cuda.current_stream()

        def forward():
            x, alpha, rho, gamma, write, read, beta = tensors
            return mira.matrix_lattice_iir(x, alpha, rho, gamma, write, read, raw_beta=beta)

        def step():
            forward().backward(dy)

        for _ in range(warmup):
            step()
        times = {}
        for name, fn in (("forward", forward), ("step", step)):
            start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            start.record(stream)
            for _ in range(steps):
                fn()
            end.record(stream)
            torch.cuda.synchronize()
            times[name] = start.elapsed_time(end) * 1e-3 / steps
        for t in tensors:
            t.grad = None
        backward_s = times["step"] - times["forward"]
        results[label] = {
            "shape": f"B={B} T={T} C={C} K={K} M={M}", "tokens": B * T,
            "forward_us": round(times["forward"] * 1e6, 1),
            "backward_us": round(backward_s * 1e6, 1),
            "step_us": round(times["step"] * 1e6, 1),
            "tokens_per_s": round(B * T / times["step"], 1),
            "backward_over_forward": round(backward_s / times["forward"], 3)}
    return results


def mixer_leg(torch, mira, steps, warmup):
    """The MiraMixer module (projections, control SiLU, the scan, gate, out_proj) at the reference's
    mira-s mixer geometry (width 768, d_e 1536, K 2, d_m 16, d_r 48, bf16, eval, no cache) and the
    shapes its own numbers are quoted at: one 32,768-token sequence (forward latency), and the
    profiler's maximum-batch calls of ~1.18 M tokens at T = 2,048 (B = 574) and T = 32,768
    (B = 36) (kernel/cuda/mira_dspv2/README.md:41-49). The reference's figures are RTX A6000 /
    RTX 6000 Ada measurements and simulations: context, not a target."""
    from mira_amd.mixer import MiraMixer

    d, C, K, M, R = 768, 1536, 2, 16, 48
    torch.manual_seed(9)
    mixer = MiraMixer(d, K, C, R, M).to("cuda", torch.bfloat16).eval()
    stream = torch.cuda.current_stream()
    results = {}
    for B, T in ((1, 32768), (574, 2048), (36, 32768)):
        x = torch.randn(B, T, d, device="cuda", dtype=torch.bfloat16)
        with torch.no_grad():
            for _ in range(warmup):
                mixer(x)
            before = dict(mira.usage())
            start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            start.record(stream)
            for _ in range(steps):
                mixer(x)
            end.record(stream)
            torch.cuda.synchronize()
        seconds = start.elapsed_time(end) * 1e-3 / steps
        fused = mira.usage()["control"] > before["control"]
        results[f"B{B}_T{T}"] = {"tokens": B * T, "ms": round(seconds * 1e3, 3),
                                 "tokens_per_s": round(B * T / seconds, 1),
                                 "scan": "coefficients formed in the scan" if fused
                                 else "coefficient GEMM + chunked scan"}
        del x
    del mixer
    torch.cuda.empty_cache()
    return results


def stack_leg(torch, steps, warmup):
    """24 random-init MiraBlocks (d_model 2048, lattice_d_e 2048, K=2,
    d_m 64, d_r 128, FFN 8192 SiLU-MLP), vocab 32000 with the tied head, weights N(0, 0.02^2),
    bf16, forward prefill of B=4 T=2048 uniform token ids with no cache. A step is one whole
    forward including the logits. One further forward carries HIP events around every mixer and
    every scan launch (matrix_lattice_iir) for the time shares."""
    from mira_amd import mixer as mixer_module
    from mira_amd.llm import MiraLLM

    B, T, V, L, d, C, M, R, H = 4, 2048, 32000, 24, 2048, 2048, 64, 128, 8192
    with torch.device("cuda"):
        torch.manual_seed(5)
        model = MiraLLM(vocab_size=V, n_layer=L, n_embd=d, lattice_d_e=C, lattice_order=2,
                        memory_dimension=M, coefficient_bottleneck=R, ffn_hidden=H)
    model = model.to(torch.bfloat16).eval()
    g = torch.Generator(device="cuda").manual_seed(6)
    ids = torch.randint(0, V, (B, T), device="cuda", generator=g)
    stream = torch.cuda.current_stream()
    with torch.no_grad():
        for _ in range(warmup):
            model(ids)
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        start.record(stream)
        for _ in range(steps):
            model(ids)
        end.record(stream)
        torch.cuda.synchronize()
        forward_s = start.elapsed_time(end) * 1e-3 / steps

        spans = {"mixer": [], "scan": []}

        def opener(kind):
            def hook(*_):
                event = torch.cuda.Event(enable_timing=True)
                event.record(stream)
                spans[kind].append([event])
            return hook

        def closer(kind):
            def hook(*_):
                event = torch.cuda.Event(enable_timing=True)
                event.record(stream)
                spans[kind][-1].append(event)
            return hook

        scan = mixer_module.plugin.matrix_lattice_iir

        def timed_scan(*args, **kwargs):
            opener("scan")()
            result = scan(*args, **kwargs)
            closer("scan")()
            return result

        handles = []
        for block in model.blocks:
            handles.append(block.mixer.register_forward_pre_hook(opener("mixer")))
            handles.append(block.mixer.register_forward_hook(closer("mixer")))
        mixer_module.plugin.matrix_lattice_iir = timed_scan
        try:
            start.record(stream)
            model(ids)
            end.record(stream)
            torch.cuda.synchronize()
        finally:
            mixer_module.plugin.matrix_lattice_iir = scan
            for handle in handles:
                handle.remove()
        whole = start.elapsed_time(end)
        share = {k: sum(a.elapsed_time(b) for a, b in v) / whole for k, v in spans.items()}
    gemm_per_token = 2 * L * (d * (C + M) + d * C + d * R + R * (7 * C + 3 * M) + C * d + 2 * d * H)
    gemm_per_token += 2 * d * V
    scan_per_token = L * C * M * (9 * 2 + 4)
    decode = decode_through_cache(torch, model, V)
    del model
    torch.cuda.empty_cache()
    return {"tokens": B * T, "forward_s": forward_s, "mixer_share": share["mixer"],
            "scan_share": share["scan"], "flops": (gemm_per_token + scan_per_token) * B * T,
            "shape": f"{L} layers, d_model {d}, d_e {C}, K 2, d_m {M}, d_r {R}, FFN {H}, "
                     f"vocab {V}; B={B} T={T}", "decode": decode}


def decode_through_cache(torch, model, vocab, prompt=64, new=24):
    """Greedy decoding with mira_amd.generate (the reference's mirachat.generate loop, batched):
    a 64-token prompt, then single-token steps through the prefix cache, eager and with the step
    replayed from a HIP graph, at batch 1 and 64. HIP events recorded as each token is accepted
    time the steps after the first (which holds the graph capture)."""
    from mira_amd.generate import generate

    results = {}
    g = torch.Generator(device="cuda").manual_seed(7)
    for batch in (1, 64):
        ids = torch.randint(0, vocab, (batch, prompt), device="cuda", generator=g)
        for graph in (False, True):
            marks = []

            def mark(_tokens):
                event = torch.cuda.Event(enable_timing=True)
                event.record()
                marks.append(event)

            generate(model, ids, 4, graph=graph)                       # warm-up
            torch.cuda.synchronize()
            generate(model, ids, new, graph=graph, on_token=mark)
            torch.cuda.synchronize()
            step_s = marks[1].elapsed_time(marks[-1]) * 1e-3 / (len(marks) - 2)
            results[f"b{batch}_{'graph' if graph else 'eager'}"] = {
                "tokens_per_s": round(batch / step_s, 1), "ms_per_step": round(step_s * 1e3, 3)}
    return results


def _cpu_sample(channels, tokens, seed, block=2048):
    """The oracle's restatement of the reference CPU mixer (the batched per-token formulation
    of model/mira_mixer.py:319-387, numpy float32) on `channels` channels of one cfg2 sequence
    of `tokens` tokens, realised as the K=1 lattice with the conv in front, in blocks that carry
    the scan state and the conv ring. Inputs are drawn first; returns the compute seconds."""
    import numpy as np

    from oracle import baseline as Bl
    from oracle import lattice as L

    rng = np.random.default_rng(seed)
    _, _, w, bias, h0 = Bl.diag_inputs(rng, 1, 1, channels, h0_scale=0.1)
    blocks = [Bl.diag_inputs(rng, 1, min(block, tokens - first), channels)[:2]
              for first in range(0, tokens, block)]
    state = h0.reshape(1, 1, channels, 1).astype(np.float32)
    ring = np.zeros((1, channels, 3), np.float32)
    seconds, position = 0.0, 0
    for x, a in blocks:
        t0 = time.perf_counter()
        u = Bl.causal_conv(x, w, bias, ring=ring, pos=position, dtype=np.float32).astype(np.float32)
        inputs = Bl.diag_as_lattice(u, a)
        _, state = L.lattice_scan_batched(*inputs[:7], state=state)
        seconds += time.perf_counter() - t0
        ring = Bl.ring_after(x.astype(np.float32), ring, position)
        position += x.shape[1]
    return seconds


def _cpu_worker(job):
    from threadpoolctl import threadpool_limits

    with threadpool_limits(limits=1):
        return _cpu_sample(*job)


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as handle:
            for line in handle:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_leg(tokens=8192, channels=2048, runs=3):
    """The CPU baseline: the oracle restatement of the reference CPU
    mixer on one cfg2 sequence of `tokens` tokens x `channels` channels, one warm-up and then
    the median of `runs` runs, once on one thread and once on all the host cores this job may
    use (the scan is independent per channel, so each worker process takes an equal channel
    slice; a run lasts as long as its slowest worker). Worker processes are started fresh (spawn)
    and touch no GPU."""
    import multiprocessing
    import statistics

    import numpy as np
    import torch

    from threadpoolctl import threadpool_limits

    cores = max(1, min(16, os.cpu_count() or 1))
    with threadpool_limits(limits=1):
        _cpu_sample(channels, 512, 99)                                   # warm-up
        single = statistics.median(_cpu_sample(channels, tokens, seed) for seed in range(runs))
    width = channels // cores
    with multiprocessing.get_context("spawn").Pool(cores) as pool:
        pool.map(_cpu_worker, [(width, 512, 99)] * cores)                # warm-up
        walls = []
        for seed in range(runs):
            walls.append(max(pool.map(_cpu_worker, [(width, tokens, seed * 100 + i)
                                                    for i in range(cores)])))
    parallel = statistics.median(walls)
    covered = width * cores
    return {"value": tokens * covered / channels / parallel, "unit": "tokens/s", "cores": cores,
            "kind": "port",
            "sample": f"1 sequence x {tokens} tokens x {channels} channels of the cfg2 workload "
                      f"(fp32; the oracle's batched restatement of the reference CPU mixer on the "
                      f"K=1 lattice realisation, conv in front, blocks of 2048 tokens carrying "
                      f"state and ring): {cores} worker processes of {width} channels each, one "
                      f"warm-up, median of {runs} runs ({parallel:.2f} s)",
            "single_thread": {"value": tokens / single, "unit": "tokens/s", "cores": 1,
                              "seconds": round(single, 2)},
            "method": f"one warm-up, median of {runs}", "cpu_model": _cpu_model(),
            "host_cpus": os.cpu_count(), "numpy": np.__version__, "torch": torch.__version__}


def _cpu_gla_sample(streams, tokens, seed):
    """The reference CPU mixer's per-token loop in its GLA realisation (the K = 1 lattice with
    C = d_v = M = d_k = 128 per (b, head) stream; the oracle's restatement, numpy float32) on
    `streams` streams of the cfg3 inputs for `tokens` tokens. Inputs are drawn first; returns
    the compute seconds."""
    import numpy as np

    from oracle import baseline as Bl

    rng = np.random.default_rng(seed)
    q, k, v, g = Bl.gla_inputs(rng, 1, tokens, streams, 128, 128)
    S0 = (rng.standard_normal((1, streams, 128, 128)) * 0.1).astype(np.float32)
    t0 = time.perf_counter()
    Bl.gla_recurrent(q, k, v, g, S0, dtype=np.float32)
    return time.perf_counter() - t0


def _cpu_decode_sample(heads, channels, steps, seed):
    """`steps` cfg4 decode steps on the CPU (the oracle's restatement, numpy float32): the GLA
    state update and readout of `heads` (b, head) streams and the conv + diagonal step of
    `channels` (b, d) channels, each step from the previous one's states. Returns seconds."""
    import numpy as np

    from oracle import baseline as Bl

    rng = np.random.default_rng(seed)
    q, k, v, g = Bl.gla_inputs(rng, 1, steps, heads, 128, 128)
    S = (rng.standard_normal((1, heads, 128, 128)) * 0.1).astype(np.float32)
    x, a, w, bias, h = Bl.diag_inputs(rng, 1, steps, channels, h0_scale=0.1)
    ring = (rng.standard_normal((1, channels, 3)) * 0.1).astype(np.float32)
    t0 = time.perf_counter()
    for t in range(steps):
        _, S = Bl.gla_recurrent(q[:, t:t + 1], k[:, t:t + 1], v[:, t:t + 1], g[:, t:t + 1], S,
                                dtype=np.float32)
        _, h, ring = Bl.diag_conv_scan(x[:, t:t + 1], a[:, t:t + 1], w, bias, h, ring, pos=3 + t,
                                       dtype=np.float32)
    return time.perf_counter() - t0


def _cpu_job(job):
    from threadpoolctl import threadpool_limits

    kind, rest = job
    with threadpool_limits(limits=1):
        return (_cpu_gla_sample if kind == "gla" else _cpu_decode_sample)(*rest)


def _cpu_split(kind, jobs, runs):
    """Median over `runs` of the slowest worker's seconds, one fresh spawned worker per job."""
    import multiprocessing
    import statistics

    with multiprocessing.get_context("spawn").Pool(len(jobs)) as pool:
        pool.map(_cpu_job, [(kind, jobs[0][:-1] + (99,))] * len(jobs))     # warm-up
        return statistics.median(max(pool.map(_cpu_job, [(kind, j[:-1] + (j[-1] + 100 * r,))
                                                          for j in jobs]))
                                 for r in range(runs))


def cpu_gla_leg(tokens=2048, runs=3):
    """cfg3's CPU baseline on a fixed prefix (the cost per token of the recurrence is constant,
    so the rate extrapolates to the whole sequence): all 64 (b, head) streams for `tokens` tokens,
    one warm-up, median of `runs`, on one thread and on all the job's cores (4 streams each)."""
    import statistics

    from threadpoolctl import threadpool_limits

    cores = max(1, min(16, os.cpu_count() or 1))
    with threadpool_limits(limits=1):
        _cpu_gla_sample(64, 16, 99)
        single = statistics.median(_cpu_gla_sample(64, tokens, seed) for seed in range(runs))
    per = 64 // cores
    parallel = _cpu_split("gla", [(per, tokens, i) for i in range(cores)], runs)
    # the GPU rate counts (b, t) tokens of all 16 heads: 4 sequences of `tokens` tokens
    return {"value": 4 * tokens / parallel, "unit": "tokens/s", "cores": cores, "kind": "port",
            "sample": f"the first {tokens} of 8192 tokens of cfg3 (B 4 x H 16 = 64 streams, "
                      f"d_k = d_v = 128), the reference CPU per-token loop in its GLA "
                      f"realisation (oracle gla_recurrent, numpy float32): {cores} worker "
                      f"processes of {per} streams, one warm-up, median of {runs} "
                      f"({parallel:.2f} s)",
            "single_thread": {"value": 4 * tokens / single, "unit": "tokens/s", "cores": 1,
                              "seconds": round(single, 2)}}


def cpu_decode_leg(steps=4, runs=3):
    """cfg4's CPU baseline on a fixed number of steps: the batch-256 decode step (GLA over
    256 x 16 streams, conv + diagonal over 256 x 2048 channels), one warm-up, median of `runs`,
    on one thread and on all the job's cores (an equal share of streams and channels each)."""
    import statistics

    from threadpoolctl import threadpool_limits

    cores = max(1, min(16, os.cpu_count() or 1))
    heads, channels = 256 * 16, 256 * 2048
    with threadpool_limits(limits=1):
        _cpu_decode_sample(64, 1024, 1, 99)
        single = statistics.median(_cpu_decode_sample(heads, channels, steps, seed)
                                   for seed in range(runs))
    parallel = _cpu_split("decode", [(heads // cores, channels // cores, steps, i)
                                     for i in range(cores)], runs)
    return {"value": steps / parallel, "unit": "steps/s", "cores": cores, "kind": "port",
            "sample": f"{steps} cfg4 decode steps at batch 256 (GLA state [256,16,128,128] and "
                      f"conv + diagonal over [256,2048], oracle restatement, numpy float32): "
                      f"{cores} worker processes of {heads // cores} streams and "
                      f"{channels // cores} channels, one warm-up, median of {runs} "
                      f"({parallel:.2f} s)",
            "single_thread": {"value": steps / single, "unit": "steps/s", "cores": 1,
                              "seconds": round(single, 2)}}


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only: the Mira scan shards over "
                                   "batch and channels with no exchange, and no multi-GPU leg "
                                   "is built or measured", "n_gpus": args.gpus}))
        sys.exit(2)
    if args.traffic_child:
        traffic_child()
        return
    # the headline kernel's HBM traffic, from child rocprofv3 runs started before this process
    # initialises the GPU
    traffic, traffic_note = (None, "skipped (--no-traffic)") if args.no_traffic else measure_traffic()
    import torch

    from mira_amd import _lib, mira

    if not torch.cuda.is_available() or _lib.library() is None:
        print(json.dumps({"error": f"needs a HIP device and the built library: {_lib.why()}"}))
        sys.exit(1)
    legs = (set(args.only) & set(LEGS)) if args.only else set(LEGS)
    if args.no_stack:
        legs.discard("stack")
    prefill = prefill_leg(torch, mira, args.steps, args.warmup)
    decode = decode_leg(torch, mira, args.decode_steps) if "decode" in legs else None
    # every leg warms up for at least ~5 ms of its own calls first: with two warm-up calls the
    # lattice operator's first timed calls still ran ~20 % slower than its steady state
    gla = gla_prefill_leg(torch, mira, max(5, args.steps // 2), 10) if "gla" in legs else None
    lat = lattice_leg(torch, mira, max(10, args.steps // 2), 10) if "lattice" in legs else None
    ctl = control_leg(torch, mira, max(5, args.steps // 10), 5) if "control" in legs else None
    back = backward_leg(torch, mira, max(3, args.steps // 10), 3) if "backward" in legs else None
    mix = mixer_leg(torch, mira, 3, 3) if "mixer" in legs else None
    stack = stack_leg(torch, 3, 2) if "stack" in legs else None
    achieved = prefill["algorithmic"] / prefill["kernel_s"] / 1e9
    line = {
        "metric": METRIC,
        "value": prefill["tokens"] * args.steps / prefill["elapsed"],
        "unit": "tokens/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": prefill["elapsed"] / args.steps * 1e3,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic",
        "config": {"workload": "cfg2: conv(width 4) + diagonal decay scan prefill, bf16 in/out, "
                               "fp32 state, B=8 T=4096 D=2048, h0 ~ N(0, 0.1^2)",
                   "global_batch": 8, "seq_len": 4096, "channels": 2048, "parallelism": "none"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": None if traffic is None else traffic["bytes"],
                     "kernel": "diag_column_kernel",
                     "kernel_us": round(prefill["kernel_s"] * 1e6, 2),
                     "algorithmic_bytes": prefill["algorithmic"],
                     "traffic_source": ("measured in this run: rocprofv3 --pmc FETCH_SIZE, then "
                                        "WRITE_SIZE, over `bench.py --traffic-child`, each scaled "
                                        "by its reading for a 128 MiB + 128 MiB copy")
                     if traffic is not None else f"not measured: {traffic_note}",
                     "traffic_detail": traffic},
        "watchdog": prefill["watchdog"],
    }
    if decode is not None:
        gla_achieved = decode["gla_bytes"] / decode["gla_kernel_s"] / 1e9
        line["decode"] = {"metric": "decode steps/s at batch 256", "unit": "steps/s",
                   "value": decode["steps"] / decode["graph_elapsed"], "steps": decode["steps"],
                   "launch": "the steps' launches replayed as one HIP graph, each step's "
                             "conv+diag launch on a side stream beside its GLA launch",
                   "serial_graph_value": decode["steps"] / decode["serial_elapsed"],
                   "eager_value": decode["steps"] / decode["elapsed"],
                   "bytes_per_step": decode["per_step_bytes"],
                   "step_GBps": round(decode["per_step_bytes"] * decode["steps"]
                                      / decode["graph_elapsed"] / 1e9, 1),
                   "frac_of_hbm": round(decode["per_step_bytes"] * decode["steps"]
                                        / decode["graph_elapsed"] / 1e9 / HBM_PEAK_GBS, 4),
                   "eager_frac_of_hbm": round(decode["per_step_bytes"] * decode["steps"]
                                              / decode["elapsed"] / 1e9 / HBM_PEAK_GBS, 4),
                   "roofline": {"bound": "hbm", "kernel": "gla_step_kernel",
                                "achieved": round(gla_achieved, 1), "peak": HBM_PEAK_GBS,
                                "unit": "GB/s", "frac": round(gla_achieved / HBM_PEAK_GBS, 4),
                                "kernel_us": round(decode["gla_kernel_s"] * 1e6, 2),
                                "algorithmic_bytes": decode["gla_bytes"]}}
    if gla is not None:
        gla_hbm = gla["algorithmic"] / gla["kernel_s"] / 1e9
        line["matrix_state_prefill"] = {
            "metric": "GLA chunked prefill tokens/s (cfg3: B=4 T=8192 H=16 d=128 bf16, chunk 64)",
            "unit": "tokens/s", "value": gla["tokens"] * gla["steps"] / gla["elapsed"],
            "roofline": {"bound": "hbm", "kernel": "gla_chunk_kernel",
                         "achieved": round(gla_hbm, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(gla_hbm / HBM_PEAK_GBS, 4),
                         "kernel_us": round(gla["kernel_s"] * 1e6, 2),
                         "algorithmic_bytes": gla["algorithmic"]},
            "mfma": {"achieved": round(gla["flops"] / gla["kernel_s"] / 1e12, 1),
                     "peak": 2500.0, "unit": "TFLOP/s",
                     "frac": round(gla["flops"] / gla["kernel_s"] / 1e12 / 2500.0, 4),
                     "flops": gla["flops"]}}
    if lat is not None:
        line["lattice_operator"] = {
            "metric": "matrix_lattice_iir tokens/s at the cfg5 mixer geometry, bf16",
            "shape": lat["shape"], "unit": "tokens/s", "value": lat["tokens"] / lat["call_s"],
            "call_us": round(lat["call_s"] * 1e6, 1),
            "hbm": {"achieved": round(lat["bytes"] / lat["call_s"] / 1e9, 1),
                    "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": round(lat["bytes"] / lat["call_s"] / 1e9 / HBM_PEAK_GBS, 4),
                    "algorithmic_bytes": lat["bytes"]},
            "valu": {"achieved": round(lat["flops"] / lat["call_s"] / 1e12, 1),
                     "peak": 157.3, "unit": "TFLOP/s",
                     "frac": round(lat["flops"] / lat["call_s"] / 1e12 / 157.3, 4),
                     "flops": lat["flops"]},
            "decode_step": {
                "shape": lat["step_shape"], "unit": "steps/s", "value": 1.0 / lat["step_s"],
                "step_us": round(lat["step_s"] * 1e6, 1),
                "roofline": {"bound": "hbm", "kernel": "lattice_step_kernel",
                             "achieved": round(lat["step_bytes"] / lat["step_s"] / 1e9, 1),
                             "peak": HBM_PEAK_GBS, "unit": "GB/s",
                             "frac": round(lat["step_bytes"] / lat["step_s"] / 1e9 / HBM_PEAK_GBS, 4),
                             "algorithmic_bytes": lat["step_bytes"]}}}
    if ctl is not None:
        line["control_scan"] = {
            "metric": "matrix_lattice_iir_control tokens/s at the reference mixer geometry, bf16, "
                      "coefficients formed inside the scan",
            "shape": ctl["shape"], "unit": "tokens/s", "value": ctl["tokens"] / ctl["call_s"],
            "call_us": round(ctl["call_s"] * 1e6, 1),
            "kernel": "lattice_control_kernel", "kernel_us": round(ctl["kernel_s"] * 1e6, 1),
            "materialised_value": ctl["tokens"] / ctl["materialised_s"],
            "materialised_us": round(ctl["materialised_s"] * 1e6, 1),
            "speedup": round(ctl["materialised_s"] / ctl["call_s"], 3),
            "outputs_identical_to_materialised": round(ctl["identical"], 6),
            "hbm": {"achieved": round(ctl["bytes"] / ctl["kernel_s"] / 1e9, 1),
                    "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": round(ctl["bytes"] / ctl["kernel_s"] / 1e9 / HBM_PEAK_GBS, 4),
                    "algorithmic_bytes": ctl["bytes"]},
            "valu": {"achieved": round(ctl["flops"] / ctl["kernel_s"] / 1e12, 1),
                     "peak": 157.3, "unit": "TFLOP/s",
                     "frac": round(ctl["flops"] / ctl["kernel_s"] / 1e12 / 157.3, 4),
                     "flops": ctl["flops"]}}
    if back is not None:
        line["training_scan"] = dict(
            back, metric="matrix_lattice_iir forward + backward (all seven gradients) tokens/s, "
                         "bf16, zero initial state")
    if mix is not None:
        line["mixer_module"] = dict(
            mix, metric="MiraMixer forward tokens/s at the reference's mira-s geometry (d 768, "
                        "d_e 1536, K 2, d_m 16, d_r 48), bf16, eval",
            reference_context="published for the mixer module on an RTX A6000 at 32,768 tokens: "
                              "11.37 ms forward, 8.36 M tokens/s at maximum batch "
                              "(doc/html/pages/results.html); simulated RTX 6000 Ada max-batch "
                              "8.70-11.03 M tokens/s (kernel/cuda/mira_dspv2/README.md:41-49)")
    if stack is not None:
        line["stack"] = {
            "metric": "cfg5 forward prefill tokens/s (24 MiraBlocks, bf16, no cache)",
            "shape": stack["shape"], "unit": "tokens/s",
            "value": stack["tokens"] / stack["forward_s"],
            "ms_per_forward": round(stack["forward_s"] * 1e3, 2),
            "mixer_share": round(stack["mixer_share"], 4),
            "scan_share": round(stack["scan_share"], 4),
            "tflops": round(stack["flops"] / stack["forward_s"] / 1e12, 1),
            "flops_per_forward": stack["flops"],
            "decode": dict(stack["decode"], metric="greedy decode through the prefix cache, "
                                                   "64-token prompt, tokens/s per batch size")}
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_leg()
        if "matrix_state_prefill" in line:
            line["matrix_state_prefill"]["cpu_baseline"] = cpu_gla_leg()
        if "decode" in line:
            line["decode"]["cpu_baseline"] = cpu_decode_leg()
    if args.calibrate:
        calibrate(torch, 5)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
