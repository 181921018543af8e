"""Headline benchmark: ALIF forward + fast_sigmoid surrogate backward on one MI355X,
plus the path's other synthetic workloads, in one JSON line.

Headline workload: input currents [T=256, B=128, N=4096] fp32 ~ N(0.25, 0.6),
ALIFParams(tau_mem=20 (decay 0.95), tau_adaptation=50 (rho 0.98),
threshold=1, reset=0 (hard reset), beta=1.8), fast_sigmoid slope 10, upstream
dL/ds ~ N(0, 1).  One step = the public-API forward
(``surrogate_alif_forward``) plus ``spikes.backward(dL/ds)``, inputs resident
in HBM.

    python bench.py [--steps K] [--warmup W] [--no-cpu-baseline] [--workload NAME]

By default the line also carries, under "workloads", one entry per other
workload, each with its own throughput, dominant-kernel roofline (HIP events
around C-ABI launches of that kernel on the launch stream) and a bounded
CPU baseline (the oracle's restatement of myelin's torch path on the host
cores):
  lif_fwd         LIF forward [100, 64, 1024], tau 10, hard reset (20 input
                  buffers of 26.2 MB rotated, 524 MB, twice the 256 MB
                  Infinity Cache, so each launch reads x from HBM)
  linear_bf16     one training step: LinearSurrogateLIF(784 -> 2048,
                  stream_synapse, atan, bf16 GEMM) + LinearSurrogateLIFRate
                  (2048 -> 10, atan, C=25), CE on spike counts, [50, 256, 784]
  long_rate       one training step: LinearSurrogateLIF(1024 -> 4096,
                  checkpoint "memory", superspike, fp32) + rate readout
                  (4096 -> 20), CE, [2000, 32, 1024]; reports peak HBM bytes
  long_rate_packed  the same network and step through
                  two_layer_surrogate_lif_rate_packed_hidden_forward (the two
                  layers interleaved per checkpoint chunk, hidden spikes kept
                  bitpacked); reports peak HBM bytes.  checkpoint_size=
                  "memory" is the memory-lean policy (buffers of one
                  checkpoint chunk)
  long_rate_fast, long_rate_packed_fast  the same two steps with
                  checkpoint_size=45: the same chunk length, buffers of 2**25
                  floats
  bitpack         pack [512, 64, 8192] spikes, unpack, per-neuron counts over
                  T, per-sample rates (the 33.5 MB packed input of the counts
                  and rates rotated over 12 copies, 403 MB)
``--workload NAME`` prints only that workload's line (``alif_headline``: only
the headline).
"""

from __future__ import annotations

import argparse
import json
import math
import os
import pathlib
import sys
import time

ROOT = pathlib.Path(__file__).resolve().parent
METRIC = "neuron-steps/sec (T·B·N) LIF fwd+bwd at 1 GPU; % of HBM roofline"
T, B, N = 256, 128, 4096
HBM_PEAK_GBPS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
FP32_PEAK_TFLOPS = 157.3
# algorithmic bytes per neuron-step: forward reads x and writes spikes;
# backward re-reads x, reads dL/ds, writes dL/dx
FWD_BYTES, BWD_BYTES = 8, 12
PROFILES = ROOT / "profiles"
TRAFFIC_FILE = PROFILES / "traffic_alif_fast_sigmoid_T256_B128_N4096.json"
WORKLOADS = ("lif_fwd", "linear_bf16", "long_rate", "long_rate_fast", "long_rate_packed", "long_rate_packed_fast",
             "bitpack")


def _args():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    # 100 steps: the fixed cost of starting and ending the timed region (the
    # first launch after a synchronize, the last synchronize) stays under 1 %
    # of a step
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true", help="skip the CPU oracle timings")
    ap.add_argument("--workload", default="all", choices=["all", "alif_headline", *WORKLOADS])
    ap.add_argument("--cpu-sample-batch", type=int, default=128)
    ap.add_argument("--cpu-min-seconds", type=float, default=10.0,
                    help="CPU baseline sampling time of the headline (the other workloads take a third)")
    ap.add_argument(
        "--calibration-copy",
        action="store_true",
        help="also run one 1 GiB device-to-device copy (the known-size kernel that scales PMC byte counters)",
    )
    return ap.parse_args()


# ---------------------------------------------------------------- helpers
def _host_threads(torch) -> dict:
    """Use every core this process may run on; report what that was."""

    avail = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    torch.set_num_threads(avail)
    return {"cores": torch.get_num_threads(), "os_cpu_count": os.cpu_count(), "affinity_cpus": avail}


def _cpu_mean(run, min_seconds: float, max_runs: int = 50) -> tuple[float, int, float]:
    """Mean duration of `run()` (which returns its own duration), repeated
    until `min_seconds` have been spent; returns (mean, runs, total)."""

    times = []
    while sum(times) < min_seconds and len(times) < max_runs:
        times.append(run())
    return sum(times) / len(times), len(times), sum(times)


def _launch_ms(torch, launch, reps: int) -> float:
    """Average duration of `launch()` over back-to-back launches bracketed by
    one HIP event pair on the current stream (the launch stream): a pair
    around each launch would also time the host's launch latency.  The
    launches queue up behind a GPU-side spin of about 30 us per launch, so
    that a short kernel runs back to back even where the host issues
    launches more slowly than the GPU runs them (under a kernel tracer)."""

    launch()
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda._sleep(int(reps * 30e-6 * 2.5e9))  # spin cycles: ~30 us per launch at 2.5 GHz
    ev0.record()
    for _ in range(reps):
        launch()
    ev1.record()
    torch.cuda.synchronize()
    return ev0.elapsed_time(ev1) / reps


def _launch_ms_median(torch, launch, reps: int, warmup: int = 10) -> float:
    """Median duration of `launch()` from one HIP event pair per launch on
    the current stream (the launch stream), after `warmup` untimed launches:
    the figure a kernel trace's per-dispatch durations give, insensitive to
    the few launches a clock change catches."""

    for _ in range(warmup):
        launch()
    torch.cuda.synchronize()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(2 * reps)]
    for i in range(reps):
        ev[2 * i].record()
        launch()
        ev[2 * i + 1].record()
    torch.cuda.synchronize()
    d = sorted(ev[2 * i].elapsed_time(ev[2 * i + 1]) for i in range(reps))
    return d[reps // 2] if reps % 2 else 0.5 * (d[reps // 2 - 1] + d[reps // 2])


def _traffic(name: str, kernel: str):
    """HBM bytes per launch of `kernel` from profiles/traffic_<name>.json
    (rocprofv3 FETCH_SIZE / WRITE_SIZE, calibrated on a copy), or None."""

    f = PROFILES / f"traffic_{name}.json"
    if not f.exists():
        return None
    return json.loads(f.read_text()).get("hbm_bytes_per_launch", {}).get(kernel)


def _timed(torch, step, steps, warmup):
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) * 1e3 / steps


# eager steps timed beside a graph replay: at least this many, so that the
# first step's wait for the host's first launches (the timed region starts
# from an idle GPU) does not stand for the steady state of a training loop
EAGER_MIN_STEPS = 100


def _graph_timed(torch, body, params, steps, warmup):
    """ms per step of `body()` (forward + backward of a training step,
    gradients set to None first) replayed from one captured HIP graph: the
    same kernels in the same order as an eager step, launched without the
    host's per-op work.  The capture follows torch's whole-network recipe:
    warm up on a side stream, drop the gradients, capture.  Returns
    (ms, eager ms over max(steps, EAGER_MIN_STEPS) steps, the same eager
    timing with torch's autograd engine running the backward on the calling
    thread instead of its device thread)."""

    eager = _timed(torch, lambda: (_none(params), body()), max(steps, EAGER_MIN_STEPS), warmup)
    with torch.autograd.set_multithreading_enabled(False):
        eager_one_thread = _timed(torch, lambda: (_none(params), body()), max(steps, EAGER_MIN_STEPS), warmup)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):
            _none(params)
            body()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    _none(params)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        body()
    ms = _timed(torch, graph.replay, steps, warmup)
    return ms, eager, eager_one_thread


def _none(params):
    for q in params:
        q.grad = None


def _line(metric, value, unit, ms, args, config, steps=None, warmup=None, **extra):
    out = {
        "metric": metric, "value": value, "unit": unit, "n_gpus": 1,
        "steps": args.steps if steps is None else steps, "warmup": args.warmup if warmup is None else warmup,
        "ms_per_step": ms, "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic", "config": config,
    }
    out.update(extra)
    return out


def _oracle():
    sys.path.insert(0, str(ROOT))
    from oracle import torch_ref as R

    return R


# ---------------------------------------------------------------- headline
def _kernel_times(torch, myelin, x, gs, reps: int):
    """Average duration (ms) of the forward and backward kernels, launched
    through the C ABI on the current stream and timed with HIP events on
    that stream."""

    from myelin_amd import _lib
    from myelin_amd.autograd import BWD_CHUNK

    p = myelin.ALIFParams(20.0, 50.0, 1.0, 0.0, 1.8)
    dev = x.device
    z = torch.zeros((B, N), device=dev)
    K = math.ceil(T / BWD_CHUNK)
    mT, aT = torch.empty_like(z), torch.empty_like(z)
    spikes = torch.empty_like(x)
    ck_m = torch.empty((K, B, N), device=dev)
    ck_a = torch.empty_like(ck_m)
    gx = torch.empty_like(x)
    gm0, ga0 = torch.empty_like(z), torch.empty_like(z)
    stream = _lib.stream(dev)
    # the arithmetic surrogate_alif_forward runs by default: straight-through
    # spike values and the adjoint in torch autograd's operation order
    from myelin_amd.surrogates import surrogate_id

    rule = _lib.RULE_STRAIGHT_THROUGH + surrogate_id("fast_sigmoid")
    code = _lib.SG_AUTOGRAD + surrogate_id("fast_sigmoid")

    def fwd():
        _lib.call("myelin_alif_fwd_f32", x.data_ptr(), z.data_ptr(), z.data_ptr(), mT.data_ptr(), aT.data_ptr(),
                  spikes.data_ptr(), None, ck_m.data_ptr(), ck_a.data_ptr(), T, B, N, p.decay,
                  p.adaptation_decay, p.threshold, p.beta, p.reset, 10.0, rule, BWD_CHUNK, stream)

    def bwd():
        _lib.call("myelin_alif_bwd_f32", x.data_ptr(), ck_m.data_ptr(), ck_a.data_ptr(), gs.data_ptr(), None, None,
                  gx.data_ptr(), gm0.data_ptr(), ga0.data_ptr(), T, B * N, p.decay, p.adaptation_decay,
                  p.threshold, p.beta, p.reset, 10.0, code, BWD_CHUNK, stream)

    out = {}
    for name, fn in (("fwd", fwd), ("bwd", bwd)):
        fn()
        torch.cuda.synchronize()
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(2 * reps)]
        for i in range(reps):
            ev[2 * i].record()
            fn()
            ev[2 * i + 1].record()
        torch.cuda.synchronize()
        out[name] = sum(ev[2 * i].elapsed_time(ev[2 * i + 1]) for i in range(reps)) / reps
    return out


def _cpu_baseline_headline(torch, sample_b: int, min_seconds: float, threads: dict):
    """myelin's torch path (restated in the oracle) on the host cores, on a
    bounded sample: the same T and N, the first `sample_b` batch rows."""

    R = _oracle()
    g = torch.Generator().manual_seed(2)

    def run(b):
        x = (0.25 + 0.6 * torch.randn(T, b, N, generator=g)).requires_grad_()
        gs = torch.randn(T, b, N, generator=g)
        z = torch.zeros(b, N)
        t0 = time.perf_counter()
        _, _, s = R.surrogate_alif_unroll(x, z, z, 20.0, 50.0, 1.0, 0.0, 1.8, "fast_sigmoid", 10.0)
        s.backward(gs)
        return time.perf_counter() - t0

    run(2)  # warmup, excluded
    dt, n, tot = _cpu_mean(lambda: run(sample_b), min_seconds)
    return {
        "value": T * sample_b * N / dt, "unit": "neuron-steps/s", **threads, "kind": "port",
        "sample": f"oracle torch_ref.surrogate_alif_unroll fwd + autograd bwd, T={T}, B={sample_b} of {B}, "
        f"N={N}, fp32, mean of {n} runs ({tot:.1f} s total) after a B=2 warmup",
    }


def _headline(torch, myelin, args, threads):
    dev = torch.device("cuda:0")
    from myelin_amd.autograd import BWD_CHUNK

    g = torch.Generator().manual_seed(2)
    x = (0.25 + 0.6 * torch.randn(T, B, N, generator=g)).to(dev)
    gs = torch.randn(T, B, N, generator=g).to(dev)
    z = torch.zeros((B, N), device=dev)
    p = myelin.ALIFParams(20.0, 50.0, 1.0, 0.0, 1.8)
    xd = x.clone().requires_grad_()

    def step():
        xd.grad = None
        _, s = myelin.surrogate_alif_forward(xd, myelin.ALIFState(z, z), p, surrogate="fast_sigmoid",
                                             surrogate_slope=10.0)
        s.backward(gs)

    # the per-kernel HIP-event times first: they launch the same two kernels
    # back to back, so the timed steps below start on a GPU already running
    # at its working clocks rather than from idle
    kt = _kernel_times(torch, myelin, x, gs, reps=max(20, args.steps))
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / args.steps
    E = T * B * N
    value = E / (ms * 1e-3)

    fwd_gbps = FWD_BYTES * E / (kt["fwd"] * 1e-3) / 1e9
    bwd_gbps = BWD_BYTES * E / (kt["bwd"] * 1e-3) / 1e9
    traffic = None
    if TRAFFIC_FILE.exists():
        traffic = json.loads(TRAFFIC_FILE.read_text()).get("bwd_hbm_bytes_per_launch")
    line = {
        "metric": METRIC, "value": value, "unit": "neuron-steps/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": ms, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {
            "workload": "ALIF forward + fast_sigmoid surrogate backward (surrogate_alif_forward + backward)",
            "T": T, "B": B, "N": N, "tau_mem": 20.0, "tau_adaptation": 50.0, "beta": 1.8, "threshold": 1.0,
            "reset": 0.0, "surrogate_slope": 10.0, "x": "N(0.25, 0.6)", "grad_spikes": "N(0, 1)",
        },
        "roofline": {
            "bound": "hbm", "kernel": f"bwd_chunked<ALIF, C={BWD_CHUNK}, fast_sigmoid, V=2, autograd order>",
            "achieved": bwd_gbps, "peak": HBM_PEAK_GBPS, "unit": "GB/s", "frac": bwd_gbps / HBM_PEAK_GBPS,
            "traffic": traffic,
        },
        "kernels": {
            "fwd_ms": kt["fwd"], "bwd_ms": kt["bwd"], "fwd_GBps_algorithmic": fwd_gbps,
            "bwd_GBps_algorithmic": bwd_gbps,
            "step_GBps_algorithmic": (FWD_BYTES + BWD_BYTES) * E / (ms * 1e-3) / 1e9,
            "step_hbm_frac": (FWD_BYTES + BWD_BYTES) * E / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS,
        },
    }
    del x, gs, xd
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = _cpu_baseline_headline(torch, args.cpu_sample_batch, args.cpu_min_seconds, threads)
    return line


# ---------------------------------------------------------------- config: LIF forward
def _workload_lif_fwd(torch, myelin, args, threads):
    Tl, Bl, Nl = 100, 64, 1024
    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(1)
    # 20 inputs of 26.2 MB (524 MB) rotated, and as many outputs for the
    # kernel timing: twice the 256 MB Infinity Cache, so each launch's x
    # comes from HBM, not from the cache the previous launches filled
    nrot = 20
    x0_cpu = 0.3 + 0.5 * torch.randn(Tl, Bl, Nl, generator=g)
    xs = [x0_cpu.to(dev)]
    for r in range(1, nrot):
        xs.append(0.3 + 0.5 * torch.randn(Tl, Bl, Nl, generator=g).to(dev))
    m0 = myelin.LIFState(torch.zeros(Bl, Nl, device=dev))
    p = myelin.LIFParams(10.0, 1.0, 0.0)
    it = [0]

    def step():
        myelin.lif_forward(xs[it[0] % nrot], m0, p)
        it[0] += 1

    ms = _timed(torch, step, args.steps, args.warmup)
    E = Tl * Bl * Nl
    from myelin_amd import _lib

    stream = _lib.stream(dev)
    m_final = torch.empty(Bl, Nl, device=dev)
    spikes = [torch.empty(Tl, Bl, Nl, device=dev) for _ in range(nrot)]
    i = [0]

    def launch():
        k = i[0] % nrot
        _lib.call("myelin_lif_fwd_f32", xs[k].data_ptr(), m0.membrane.data_ptr(), m_final.data_ptr(),
                  spikes[k].data_ptr(), None, None, Tl, Bl, Nl, p.decay, p.threshold, p.reset, 0.0,
                  _lib.RULE_THRESHOLD, 1, stream)
        i[0] += 1

    # back-to-back launches under one event pair: per launch within 4 % of
    # the per-dispatch duration a kernel trace reports (a per-launch event
    # pair adds ~2 us of event processing to this 13 us kernel; its median
    # is reported beside)
    kern_ms = _launch_ms(torch, launch, max(args.steps, nrot) * 4)
    kern_pair = _launch_ms_median(torch, launch, max(args.steps, nrot) * 2 + 1)
    # algorithmic bytes: read x, write spikes (8 B per neuron-step) + m0 in, m_final out
    nbytes = 8 * E + 8 * Bl * Nl
    gbps = nbytes / (kern_ms * 1e-3) / 1e9
    kernel = "fwd_dense<LIF, threshold, V=1, U=32>"
    line = _line("neuron-steps/sec LIF forward", E / (ms * 1e-3), "neuron-steps/s", ms, args,
                 {"workload": "lif_forward, hard reset", "T": Tl, "B": Bl, "N": Nl, "tau_mem": 10.0,
                  "x": "N(0.3, 0.5)", "rotated_input_buffers": nrot},
                 roofline={"bound": "hbm", "kernel": kernel, "achieved": gbps, "peak": HBM_PEAK_GBPS,
                           "unit": "GB/s", "frac": gbps / HBM_PEAK_GBPS,
                           "traffic": _traffic("lif_fwd_T100_B64_N1024", "fwd_dense"),
                           "bytes_per_launch": nbytes, "kernel_ms": kern_ms,
                           "kernel_ms_event_pair_median": kern_pair},
                 kernels={"fwd_ms": kern_ms, "step_ms": ms})
    if not args.no_cpu_baseline:
        R = _oracle()
        z = torch.zeros(Bl, Nl)

        def run():
            t0 = time.perf_counter()
            R.lif_unroll(x0_cpu, z, 10.0, 1.0, 0.0)
            return time.perf_counter() - t0

        run()
        dt, n, tot = _cpu_mean(run, args.cpu_min_seconds / 3)
        line["cpu_baseline"] = {"value": E / dt, "unit": "neuron-steps/s", **threads, "kind": "port",
                                "sample": f"oracle torch_ref.lif_unroll, the whole [100, 64, 1024] workload, mean "
                                          f"of {n} runs ({tot:.1f} s total) after one warmup run"}
    return line


# ---------------------------------------------------------------- config: streamed synapse, bf16
def _kaiming_(torch, w, fan_in, g=None):
    bound = math.sqrt(6.0 / fan_in)
    with torch.no_grad():
        w.uniform_(-bound, bound, generator=g)
    return w


def _workload_linear_bf16(torch, myelin, args, threads):
    Tl, Bl, F, H, O = 50, 256, 784, 2048, 10
    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(3)
    rate_f = torch.rand(F, generator=g) * 0.2
    x_cpu = (torch.rand(Tl, Bl, F, generator=g) < rate_f).float()
    labels_cpu = torch.randint(0, O, (Bl,), generator=g)
    x, labels = x_cpu.to(dev), labels_cpu.to(dev)
    torch.manual_seed(3)
    hidden = myelin.LinearSurrogateLIF(F, H, surrogate=myelin.atan_surrogate, stream_synapse=True,
                                       synapse_precision="bf16")
    readout = myelin.LinearSurrogateLIFRate(H, O, surrogate=myelin.atan_surrogate, checkpoint_size=25,
                                            synapse_precision="bf16")
    for mod, fan in ((hidden, F), (readout, H)):
        wt = torch.empty(mod.synapse.weight.shape[1], fan)
        torch.nn.init.kaiming_uniform_(wt)  # a=0: bound sqrt(6 / fan_in)
        with torch.no_grad():
            mod.synapse.weight.copy_(wt.t())
    w1_cpu, w2_cpu = hidden.synapse.weight.detach().clone(), readout.synapse.weight.detach().clone()
    hidden.to(dev)
    readout.to(dev)
    params = list(hidden.parameters()) + list(readout.parameters())

    def body():
        rates = readout(hidden(x))
        loss = torch.nn.functional.cross_entropy(rates * Tl, labels)
        loss.backward()

    # the step as a captured HIP graph (about 30 launches whose host-side
    # work, ~0.3-0.45 ms by box, would otherwise exceed the GPU's ~0.37 ms)
    ms, eager_ms, eager_1t_ms = _graph_timed(torch, body, params, args.steps, args.warmup)
    flops = 2 * Tl * Bl * F * H * 2 + 4 * 2 * Tl * Bl * H * O
    tflops = flops / (ms * 1e-3) / 1e12
    E = Tl * Bl * H
    # the dominant kernel: the fused forward (current tiles on the bf16 MFMA,
    # recurrence in the same workgroup), as the hidden layer launches it
    from myelin_amd import _lib

    stream = _lib.stream(dev)
    xb = x.to(torch.bfloat16)
    wt = hidden.synapse.weight.detach().t().contiguous().to(torch.bfloat16)
    bias = hidden.synapse.bias.detach()
    m_final = torch.empty(Bl, H, device=dev)
    spikes = torch.empty(Tl, Bl, H, device=dev)
    pre = torch.empty(Tl, Bl, H, device=dev)
    words = torch.empty(Tl, Bl, H // 32, dtype=torch.int32, device=dev)
    P = myelin.LIFParams()

    def launch():
        # the training step's outputs: trace, spikes and their packed twin
        _lib.call("myelin_linear_lif_fwd_bf16", xb.data_ptr(), wt.data_ptr(), bias.data_ptr(), None,
                  m_final.data_ptr(), spikes.data_ptr(), pre.data_ptr(), words.data_ptr(), None, None, Tl, Bl, F, H,
                  0, Tl, 1, P.decay, P.threshold, P.reset, 10.0, _lib.RULE_THRESHOLD, stream)

    # median of per-launch event pairs: the per-dispatch duration a kernel
    # trace reports (back-to-back launches of this one-round grid also count
    # the gap before each launch's workgroups start; reported beside)
    kern_b2b = _launch_ms(torch, launch, max(args.steps, 10))
    kern_ms = _launch_ms_median(torch, launch, 2 * max(args.steps, 10) + 1)
    fwd_flops = 2 * Tl * Bl * F * H
    k_tflops = fwd_flops / (kern_ms * 1e-3) / 1e12
    line = _line("neuron-steps/sec, streamed-synapse training step", E / (ms * 1e-3), "neuron-steps/s", ms, args,
                 {"workload": "LinearSurrogateLIF(784->2048, stream_synapse, atan, bf16) + "
                              "LinearSurrogateLIFRate(2048->10, atan, C=25) + CE, fwd+bwd",
                  "T": Tl, "B": Bl, "F": F, "N": H, "readout": O, "gflop_per_step": flops / 1e9},
                 roofline={"bound": "mfma",
                           "kernel": "linear_lif_fwd_pipe<trace + spikes + packed> (fused forward: each time "
                                     "chunk's recurrence under the next chunk's GEMM)",
                           "achieved": k_tflops, "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                           "frac": k_tflops / BF16_PEAK_TFLOPS,
                           "traffic": _traffic("linear_bf16_T50_B256_F784_N2048", "linear_lif_fwd_pipe"),
                           "flops_per_launch": fwd_flops, "kernel_ms": kern_ms,
                           "kernel_ms_back_to_back": kern_b2b},
                 step_tflops=tflops, step_frac_of_bf16_peak=tflops / BF16_PEAK_TFLOPS, dtype="bf16",
                 timing="HIP graph replay of the whole step (forward, loss, backward)", eager_ms_per_step=eager_ms,
                 eager_steps=max(args.steps, EAGER_MIN_STEPS), eager_over_graph=eager_ms / ms,
                 eager_caller_thread_backward_ms_per_step=eager_1t_ms,
                 eager_caller_thread_backward_over_graph=eager_1t_ms / ms)
    if not args.no_cpu_baseline:
        R = _oracle()
        sb = 32
        w1r, w2r = w1_cpu.bfloat16().float(), w2_cpu.bfloat16().float()

        def run():
            a = w1r.clone().requires_grad_()
            c = w2r.clone().requires_grad_()
            t0 = time.perf_counter()
            _, hs = R.linear_surrogate_lif_stream(x_cpu[:, :sb], a, torch.zeros(H), 20.0, 1.0, 0.0, "atan", 10.0)
            _, r = R.linear_surrogate_lif_rate(hs, c, torch.zeros(O), 20.0, 1.0, 0.0, "atan", 10.0, 25,
                                               reduction="none")
            torch.nn.functional.cross_entropy(r * Tl, labels_cpu[:sb]).backward()
            return time.perf_counter() - t0

        run()
        dt, n, tot = _cpu_mean(run, args.cpu_min_seconds / 3)
        line["cpu_baseline"] = {
            "value": Tl * sb * H / dt, "unit": "neuron-steps/s", **threads, "kind": "port",
            "sample": f"oracle torch_ref stream + checkpoint-rate Functions (fp32 on bf16-rounded weights), one "
                      f"training step on B={sb} of {Bl} rows at full T/F/N, mean of {n} runs ({tot:.1f} s total) "
                      f"after one warmup run"}
    return line


# ---------------------------------------------------------------- config: long-horizon rate network
def _workload_long_rate(torch, myelin, args, threads, packed_hidden=False, checkpoint_size="memory"):
    from myelin_amd import _lib
    from myelin_amd import linear as lin

    Tl, Bl, F, H, O = 2000, 32, 1024, 4096, 20
    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(4)
    x_cpu = (torch.rand(Tl, Bl, F, generator=g) < 0.05).float()
    labels_cpu = torch.randint(0, O, (Bl,), generator=g)
    x, labels = x_cpu.to(dev), labels_cpu.to(dev)
    torch.manual_seed(4)
    hidden = myelin.LinearSurrogateLIF(F, H, surrogate=myelin.superspike_surrogate, stream_synapse=True,
                                       checkpoint_size=checkpoint_size).to(dev)
    readout = myelin.LinearSurrogateLIFRate(H, O, surrogate=myelin.superspike_surrogate,
                                            checkpoint_size=checkpoint_size).to(dev)
    params = list(hidden.parameters()) + list(readout.parameters())
    wh, bh, wo, bo = hidden.synapse.weight, hidden.synapse.bias, readout.synapse.weight, readout.synapse.bias

    def step():
        for q in params:
            q.grad = None
        if packed_hidden:
            rates = myelin.two_layer_surrogate_lif_rate_packed_hidden_forward(
                x, wh, bh, wo, bo, myelin.LIFParams(), surrogate="superspike", surrogate_slope=10.0,
                checkpoint_size=checkpoint_size)
        else:
            rates = readout(hidden(x))
        torch.nn.functional.cross_entropy(rates * Tl, labels).backward()

    # the dominant kernel: one forward chunk of the split synapse, 256 steps
    # x 32 rows = 8192 x 4096 currents over 3 x 1024 bf16 k (the forward's
    # 2**25-current chunk; the backward's span recomputes run the same kernel)
    stream = _lib.stream(dev)
    rows = (lin._CURRENT_CHUNK_ELEMS // (Bl * H)) * Bl
    xb = x.reshape(Tl * Bl, F)[:rows].to(torch.bfloat16)
    w3 = torch.empty((3, H, F), dtype=torch.bfloat16, device=dev)
    _lib.call("myelin_split_bf16x3", wh.data_ptr(), w3.data_ptr(), F, H, 1, stream)
    cur = torch.empty(rows, H, device=dev)

    def launch():
        _lib.call("myelin_gemm_parts", xb.data_ptr(), w3.data_ptr(), 3, H * F, bh.data_ptr(), cur.data_ptr(), rows,
                  H, F, F, F, H, 0, 1, 0, None, 0, stream)

    # 41 back-to-back launches under one HIP event pair after 10 warmup
    # launches (the per-dispatch durations a kernel trace averages, without
    # an event pair's overhead per launch), timed before any training step
    # in both config-4 workloads (the same memory state in each; afterwards
    # the caching allocator's placement differs); the per-launch event-pair
    # median beside it
    for _ in range(10):
        launch()
    kern_ms = _launch_ms(torch, launch, 41)
    kern_pair = _launch_ms_median(torch, launch, 41, warmup=0)
    del xb, w3, cur
    step()
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats(dev)
    base = torch.cuda.memory_allocated(dev)
    # a step takes ~7 ms: a fifth of the requested steps (at least 4) after
    # one more warmup step; the line reports the counts actually timed
    n_steps, n_warm = max(4, args.steps // 5), 1
    ms = _timed(torch, step, n_steps, n_warm)
    peak_bytes = torch.cuda.max_memory_allocated(dev) - base
    flops = 3 * 2 * Tl * Bl * F * H + 4 * 2 * Tl * Bl * H * O
    tflops = flops / (ms * 1e-3) / 1e12
    E = Tl * Bl * H
    # the input is spikes, so the hidden synapse GEMMs (forward, recompute,
    # dW) run as the exact three-part bf16 split: 3x their flops on the bf16
    # MFMA; the readout GEMMs stay fp32
    split = lin._split_eligible(_lib.PREC["fp32"], Tl, Bl, F, H) and bool(torch.equal(x, x.bfloat16().float()))
    hidden_flops = 3 * 2 * Tl * Bl * F * H
    executed = (3 * hidden_flops if split else hidden_flops) + (flops - hidden_flops)
    mfma_tflops = executed / (ms * 1e-3) / 1e12
    k_flops = 3 * 2 * rows * H * F
    k_tflops = k_flops / (kern_ms * 1e-3) / 1e12
    ck = ("'memory'=45 (lean: chunk and span buffers of one checkpoint chunk)" if checkpoint_size == "memory"
          else f"{checkpoint_size} (buffers of 2**25 floats)")
    name = (f"two_layer_surrogate_lif_rate_packed_hidden_forward(1024->4096->20, checkpoint {ck}, "
            "superspike, fp32) + CE, fwd+bwd" if packed_hidden else
            f"LinearSurrogateLIF(1024->4096, stream_synapse, checkpoint {ck}, superspike, "
            f"fp32) + LinearSurrogateLIFRate(4096->20, {checkpoint_size!r}) + CE, fwd+bwd")
    line = _line("neuron-steps/sec, long-horizon checkpointed rate training step", E / (ms * 1e-3),
                 "neuron-steps/s", ms, args,
                 {"workload": name, "T": Tl, "B": Bl, "F": F, "N": H, "readout": O, "gflop_per_step": flops / 1e9},
                 steps=n_steps, warmup=n_warm + 1,
                 roofline={"bound": "mfma",
                           "kernel": "gemm_dma<256 x 256 tiles, 3 bf16 parts> (one forward chunk of the exact "
                                     "bf16 split of the fp32 synapse, 8192 x 4096 x 3*1024)",
                           "achieved": k_tflops, "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                           "frac": k_tflops / BF16_PEAK_TFLOPS,
                           "traffic": _traffic("long_rate_T2000_B32_F1024_N4096", "gemm_dma_256x256"),
                           "flops_per_launch": k_flops, "kernel_ms": kern_ms,
                           "kernel_ms_event_pair_median": kern_pair},
                 step_mfma_tflops_executed=mfma_tflops, step_mfma_frac_executed=mfma_tflops / BF16_PEAK_TFLOPS,
                 fp32_equivalent_tflops=tflops, fp32_equivalent_frac_of_fp32_peak=tflops / FP32_PEAK_TFLOPS,
                 hidden_synapse="exact bf16 split (3 parts)" if split else "fp32",
                 peak_step_bytes=peak_bytes, dense_hidden_spike_bytes=Tl * Bl * H * 4)
    if not args.no_cpu_baseline and not packed_hidden and checkpoint_size == "memory":
        R = _oracle()
        sb = 1
        C = R.resolve_checkpoint_size(Tl, "memory")
        wh_c, bh_c, wo_c, bo_c = (t.detach().cpu() for t in (wh, bh, wo, bo))

        def run():
            a, b_, c, d = (t.clone().requires_grad_() for t in (wh_c, bh_c, wo_c, bo_c))
            t0 = time.perf_counter()
            _, hs = R.linear_surrogate_lif_checkpoint(x_cpu[:, :sb], a, b_, 20.0, 1.0, 0.0, "superspike", 10.0, C)
            _, r = R.linear_surrogate_lif_rate(hs, c, d, 20.0, 1.0, 0.0, "superspike", 10.0, C, reduction="none")
            torch.nn.functional.cross_entropy(r * Tl, labels_cpu[:sb]).backward()
            return time.perf_counter() - t0

        run()  # warmup, excluded (baselines.py:72-100 times after warmup runs)
        dt, n, tot = _cpu_mean(run, args.cpu_min_seconds / 3, max_runs=5)
        line["cpu_baseline"] = {
            "value": Tl * sb * H / dt, "unit": "neuron-steps/s", **threads, "kind": "port",
            "sample": f"oracle torch_ref checkpoint + checkpoint-rate Functions (C={C}), one training step on B={sb} "
                      f"of {Bl} rows at full T/F/N/readout, mean of {n} runs ({tot:.1f} s total) after one warmup "
                      f"run"}
    return line


# ---------------------------------------------------------------- config: bitpacking
def _workload_bitpack(torch, myelin, args, threads):
    Tl, Bl, Nl = 512, 64, 8192
    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(5)
    rate = torch.exp(-3.0 + torch.randn(Nl, generator=g)).clamp(0.0, 1.0)
    s_cpu = (torch.rand((Tl, Bl, Nl), generator=g) < rate).float()
    s = s_cpu.to(dev)
    pk = myelin.pack_spikes(s)
    E = Tl * Bl * Nl
    # the counts and rates read only the 33.5 MB of words: 12 copies (403 MB)
    # rotated, so each call reads them from HBM rather than from the 256 MB
    # Infinity Cache (pack and unpack move 1.1 GB per call, beyond it)
    nrot = 12
    pks = [pk] + [myelin.PackedSpikes(pk.data.clone(), pk.original_shape) for _ in range(nrot - 1)]
    it = [0]

    def rotated(fn):
        def call():
            fn(pks[it[0] % nrot])
            it[0] += 1

        return call

    times = {}
    for name, fn in (("pack", lambda: myelin.pack_spikes(s)), ("unpack", lambda: myelin.unpack_spikes(pk)),
                     ("count_dim0", rotated(lambda q: myelin.packed_spike_count(q, dim=0))),
                     ("rate_dim0_last", rotated(lambda q: myelin.packed_spike_rate(q, dim=(0, -1))))):
        times[name] = _timed(torch, fn, args.steps, args.warmup)
    ms = sum(times.values())
    from myelin_amd import _lib

    stream = _lib.stream(dev)
    words = torch.empty_like(pk.data)
    dense = torch.empty_like(s)
    k_pack = _launch_ms(torch, lambda: _lib.call("myelin_pack", s.data_ptr(), _lib.DT[torch.float32],
                                                 words.data_ptr(), Tl * Bl, Nl, stream), max(args.steps, 10))
    k_unpack = _launch_ms(torch, lambda: _lib.call("myelin_unpack", pk.data.data_ptr(), dense.data_ptr(),
                                                   _lib.DT[torch.float32], Tl * Bl, Nl, stream), max(args.steps, 10))
    byte_model = {"pack": 4.125 * E, "unpack": 4.125 * E, "count_dim0": E / 8 + Bl * Nl * 8,
                  "rate_dim0_last": E / 8}
    gbps = {k: byte_model[k] / (times[k] * 1e-3) / 1e9 for k in times}
    pack_gbps = byte_model["pack"] / (k_pack * 1e-3) / 1e9
    line = _line("spikes/sec, pack + unpack + counts + rates", E / (ms * 1e-3), "spikes/s", ms, args,
                 {"workload": "bitpack [512, 64, 8192], Bernoulli(LogNormal(-3, 1) clipped)", "T": Tl, "B": Bl,
                  "N": Nl},
                 roofline={"bound": "hbm", "kernel": "pack_kernel<f32>", "achieved": pack_gbps,
                           "peak": HBM_PEAK_GBPS, "unit": "GB/s", "frac": pack_gbps / HBM_PEAK_GBPS,
                           "traffic": _traffic("bitpack_T512_B64_N8192", "pack_kernel"),
                           "bytes_per_launch": byte_model["pack"], "kernel_ms": k_pack},
                 kernels={**{f"{k}_ms": v for k, v in times.items()}, **{f"{k}_GBps": v for k, v in gbps.items()},
                          "pack_kernel_ms": k_pack, "unpack_kernel_ms": k_unpack,
                          "unpack_kernel_GBps": byte_model["unpack"] / (k_unpack * 1e-3) / 1e9},
                 dtype="i32", dtypes={"spikes": "f32", "words": "i32", "counts": "i64", "rates": "f32"},
                 rotated_word_buffers=nrot)
    if not args.no_cpu_baseline:
        R = _oracle()
        ts = 64
        sample = s_cpu[:ts].contiguous()

        def run():
            t0 = time.perf_counter()
            w, shape = R.pack_spikes(sample)
            R.unpack_spikes(w, shape)
            R.packed_spike_count(w, shape, 0)
            R.packed_spike_rate(w, shape, (0, -1))
            return time.perf_counter() - t0

        run()
        dt, n, tot = _cpu_mean(run, args.cpu_min_seconds / 3)
        line["cpu_baseline"] = {
            "value": ts * Bl * Nl / dt, "unit": "spikes/s", **threads, "kind": "port",
            "sample": f"oracle torch_ref pack + unpack + count(dim=0) + rate(dim=(0,-1)) on T={ts} of {Tl} steps "
                      f"(all B, N), mean of {n} runs ({tot:.1f} s total) after one warmup run"}
    return line


def main() -> int:
    args = _args()
    if args.gpus != 1:
        print(
            f"bench.py measures one GPU; --gpus {args.gpus} is not supported (the recurrence shards over B*N with "
            "no exchange; multi-GPU runs are not part of this build)",
            file=sys.stderr,
        )
        return 2
    import torch

    import myelin_amd as myelin

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    threads = _host_threads(torch)
    if args.calibration_copy:
        src = torch.empty(1 << 28, device=dev)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    others = {"lif_fwd": _workload_lif_fwd, "linear_bf16": _workload_linear_bf16, "long_rate": _workload_long_rate,
              "long_rate_packed": lambda t, m, a, th: _workload_long_rate(t, m, a, th, packed_hidden=True),
              "long_rate_fast": lambda t, m, a, th: _workload_long_rate(t, m, a, th, checkpoint_size=45),
              "long_rate_packed_fast": lambda t, m, a, th: _workload_long_rate(t, m, a, th, packed_hidden=True,
                                                                                checkpoint_size=45),
              "bitpack": _workload_bitpack}
    if args.workload in others:
        print(json.dumps(others[args.workload](torch, myelin, args, threads)), flush=True)
        return 0
    line = _headline(torch, myelin, args, threads)
    if args.workload == "all":
        line["workloads"] = {}
        for name in WORKLOADS:
            torch.cuda.empty_cache()
            line["workloads"][name] = others[name](torch, myelin, args, threads)
            print(f"# {name} done", file=sys.stderr, flush=True)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
