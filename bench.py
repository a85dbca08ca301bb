"""Benchmark of the MGN MLP hot path on one MI355X.

A step is one call of the fused edge MLP (384->128->128->128 + LayerNorm,
fp16 I/O, fp32 accumulate) over the full headline batch M = 1,048,576 with
all inputs already resident in HBM.  Prints ONE JSON line: rows/s, the
HBM-roofline fraction of the kernel measured with HIP events on the launch
stream, the HBM traffic per launch measured with rocprofv3 counters
(profiles/traffic.json), and the CPU oracle timed on a bounded sample on the
host cores.

  python bench.py [--gpus 1] [--steps 200] [--warmup 20] [--settle-ms 1000]
                  [--workload edge|node|edge_gather|bert|dlrm|nerf|bert_addln|bert_app|nerf_a|queue|mfma_peak|gemm]
                  [--impl fused|pipelined|pipelined_split_ln] [--no-cpu]

Every line carries "spread": the per-launch HIP-event times of the timed
region in launch order (min, median, max, and the means of the first and last
five launches), so a clock ramp or a slow box shows in the line itself.
--settle-ms runs untimed launches for that long between the warm-up and the
timed region, with no synchronisation between them, so the timed region starts
while the GPU is busy; the line states it in "settle".  ms_per_step is the
HIP-event time between the first and the last timed step divided by K.  For
the MGN workloads, "repeats" also gives the ms per step of --repeats blocks of
K steps per submission (the timed block and the blocks that follow it back to
back) and their median; value comes from the first block.

--workload bert times the BERT-large FFN block of configs[2] instead
(LayerNorm(GELU(x W1 + b1) W2 + b2 + x), M = 65,536, H 1024, FF 4096): a step is
one gp_bert_ffn_out call, bound by MFMA, so its roofline is TFLOP/s against the
dense fp16 peak.  --workload dlrm (configs[3]: the bottom and top MLPs over
M = 262,144) and --workload nerf (configs[4]: the NeRF MLP over M = 1,048,576
samples) are measured the same way.
"""
import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "gpu-pipes_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "rows/sec + % fp16 MFMA peak, MGN edge MLP M=1M (1×MI355X)"
HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, GB/s
MFMA_F16_PEAK_TFLOPS = 2500.0  # MI355X dense fp16 MFMA, TFLOP/s

WORKLOADS = {
    # name: (M, K, layernorm)
    "edge": (1048576, 384, True),
    "node": (262144, 256, True),
    # edge MLP with the gather front end: M edges over GATHER_NODES nodes,
    # X rows gathered as [nf[src] | ef | nf[dst]] (int64 indices)
    "edge_gather": (1048576, 384, True),
}
GATHER_NODES = 262144
WORKLOAD_METRIC = {
    "node": "rows/sec + % HBM roofline, MGN node MLP M=262144 (1×MI355X)",
    "edge_gather": "rows/sec + % HBM roofline, MGN edge MLP with gather front end M=1M (1×MI355X)",
}
BERT = {"M": 65536, "H": 1024, "FF": 4096, "eps": 1e-12}
BERT_METRIC = "rows/sec + % fp16 MFMA peak, BERT-large FFN+residual+LN M=65536 (1×MI355X)"


def algorithmic(M, K, ln, gather_nodes=0, idx_bytes=8):
    """Bytes that must cross HBM per call and MFMA FLOPs per call.  With the
    gather front end the input is the edge features (256 B/row), two indices
    per row and the node table (read at least once), not the [M, K] matrix."""
    params = (K * 128 + 2 * 128 * 128) * 2 + 3 * 128 * 2 + (2 * 128 * 2 if ln else 0)
    if gather_nodes:
        bytes_ = M * (128 * 2 + 2 * idx_bytes + 128 * 2) + gather_nodes * 128 * 2 + params
    else:
        bytes_ = M * (K + 128) * 2 + params
    flops = 2 * M * (K * 128 + 128 * 128 + 128 * 128)
    return bytes_, flops


def host_cores():
    """(threads to use, description): the cores of this process's affinity set,
    capped by a cgroup CPU quota when one is set (threads beyond the quota only
    time-slice)."""
    n = len(os.sched_getaffinity(0))
    quota = None
    try:
        with open("/sys/fs/cgroup/cpu.max") as fh:
            q, period = fh.read().split()[:2]
            if q != "max":
                quota = max(1, int(int(q) // int(period)))
    except (OSError, ValueError):
        pass
    use = min(n, quota) if quota else n
    how = f"{n} cores in the affinity set" + (f", cgroup quota {quota} cores" if quota else ", no cgroup quota")
    return use, how


def _median_runs(run, budget_s, min_runs=10, warmups=3):
    """3 warm-ups, then runs until budget_s has passed and at least min_runs
    were timed; returns (median seconds, runs, total seconds)."""
    import numpy as np

    for _ in range(warmups):
        run()
    times = []
    t_end = time.perf_counter() + budget_s
    while time.perf_counter() < t_end or len(times) < min_runs:
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    return float(np.median(times)), len(times), sum(times)


def cpu_baseline_torch_mgn(K, ln, budget_s=8.0):
    """MgnMlp (common/mlps.py:3-20) restated as torch.nn modules in fp32 on the
    host cores, under inference_mode, on the config-0 shape X[16384, K]."""
    import torch

    threads, how = host_cores()
    torch.set_num_threads(threads)
    Ms = 16384
    with torch.random.fork_rng(devices=[]):
        torch.manual_seed(0)
        layers = [torch.nn.Linear(K, 128), torch.nn.ReLU(), torch.nn.Linear(128, 128), torch.nn.ReLU(),
                  torch.nn.Linear(128, 128)]
        if ln:
            layers.append(torch.nn.LayerNorm(128))
        model = torch.nn.Sequential(*layers).eval()
        x = torch.randn(Ms, K)
    with torch.inference_mode():
        med, n, tot = _median_runs(lambda: model(x), budget_s)
    return {
        "value": Ms / med, "unit": "rows/s", "cores": threads, "kind": "port",
        "sample": f"torch.nn MgnMlp({K},[128,128,128]) fp32 on X[{Ms},{K}] (config-0 shape), torch "
                  f"{torch.__version__}, {threads} threads ({how}), 3 warm-ups, median of {n} runs "
                  f"({tot:.1f} s): {med * 1e3:.2f} ms/call",
    }


def cpu_baseline(K, ln, budget_s=8.0):
    """The CPU oracle (oracle/oracle.c, OpenMP over rows) on the config-0 shape."""
    import oracle
    from gpipes.synth import mgn_params, normal_fp16

    threads, how = host_cores()
    oracle.set_num_threads(threads)
    Ms = 16384
    p = mgn_params(K, seed=0, layernorm=ln)
    f = lambda t: None if t is None else t.float().numpy()  # noqa: E731
    x = f(normal_fp16(Ms, K, seed=0))
    args = [f(p[k]) for k in ("w1", "b1", "w2", "b2", "w3", "b3", "gamma", "beta")]
    med, n, tot = _median_runs(lambda: oracle.mgn_mlp(x, *args), budget_s)
    return {
        "value": Ms / med, "unit": "rows/s", "cores": threads, "kind": "port",
        "sample": f"oracle/oracle.c MgnMlp fp32 on X[{Ms},{K}] (config-0 shape), {threads} OpenMP threads "
                  f"({how}), 3 warm-ups, median of {n} calls ({tot:.1f} s): {med * 1e3:.2f} ms/call",
    }


def cpu_baseline_bert(budget_s=10.0):
    """The CPU oracle's BERT FFN (oracle_bert_ffn, OpenMP over rows) on a row sample."""
    import oracle
    from gpipes.synth import bert_params, normal_fp16

    threads, how = host_cores()
    oracle.set_num_threads(threads)
    Ms, H, FF = 256, BERT["H"], BERT["FF"]
    p = {k: v.float().numpy() for k, v in bert_params(H, FF, seed=0).items()}
    x = normal_fp16(Ms, H, seed=0).float().numpy()
    run = lambda: oracle.bert_ffn(x, p["w1"], p["b1"], p["w2"], p["b2"], p["gamma"], p["beta"],  # noqa: E731
                                  act=oracle.ACT_GELU_TANH, eps=BERT["eps"])
    med, n, tot = _median_runs(run, budget_s, min_runs=3, warmups=1)
    return {
        "value": Ms / med, "unit": "rows/s", "cores": threads, "kind": "port",
        "sample": f"oracle/oracle.c BertFfn fp32 on X[{Ms},{H}] (H {H}, FF {FF}, GELU tanh), {threads} threads "
                  f"({how}), median of {n} calls ({tot:.1f} s): {med * 1e3:.1f} ms/call",
    }


def spread(ms):
    """Per-launch times (ms) in launch order -> min / median / max and the
    means of the first and last five launches."""
    s = sorted(ms)
    k = min(5, len(ms))
    return {"min": s[0], "median": s[len(s) // 2], "max": s[-1],
            "first5_mean": sum(ms[:k]) / k, "last5_mean": sum(ms[-k:]) / k}


class _Pacer:
    """Keeps the launch queue busy but bounded: after every 16 enqueued steps
    an event is recorded, and the host waits for the event recorded `depth`
    steps earlier, so the GPU never drains and the host never runs more than
    about `depth` steps ahead."""

    def __init__(self, stream, depth=64):
        self.stream, self.depth, self.marks, self.n = stream, depth, [], 0

    def tick(self):
        import torch

        self.n += 1
        if self.n % 16 == 0:
            e = torch.cuda.Event()
            e.record(self.stream)
            self.marks.append(e)
            if len(self.marks) > self.depth // 16:
                self.marks.pop(0).synchronize()


def _settle(run_one, stream, settle_ms, bracket=None):
    """Untimed submissions for settle_ms, paced by _Pacer (no synchronisation,
    so the timed region that follows starts while the GPU is still busy).
    bracket: a pair of timing events recorded around every launch, as the
    timed region records its per-step events, so that the submission pattern
    does not change where the timed region starts."""
    pacer = _Pacer(stream)
    t0 = time.perf_counter()
    n = 0
    while (time.perf_counter() - t0) * 1e3 < settle_ms:
        if bracket is not None:
            bracket[0].record(stream)
        run_one(n)
        if bracket is not None:
            bracket[1].record(stream)
        pacer.tick()
        n += 1
    return {"ms": (time.perf_counter() - t0) * 1e3, "launches": n}


def start_telemetry(delay_s=1.0):
    """Start a child process that reads the board's telemetry (rocm-smi
    --showmetrics: socket power, per-XCD engine clocks, activity; rocm-smi -M:
    the power cap) delay_s from now, while the settle launches run."""
    import subprocess

    smi = "/opt/rocm/bin/rocm-smi"
    cmd = f"sleep {delay_s}; {smi} --showmetrics; {smi} -M"
    return subprocess.Popen(["bash", "-c", cmd], stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)


def finish_telemetry(child):
    """Parse the telemetry child's output into a small record."""
    import re

    out, _ = child.communicate(timeout=120)

    def field(name):
        m = re.search(re.escape(name) + r"[^:]*:\s*(\[[^\]]*\]|[0-9.]+)", out)
        if not m:
            return None
        v = m.group(1)
        return [float(t) for t in v.strip("[]").split(",") if t.strip()] if v.startswith("[") else float(v)

    return {"source": "rocm-smi --showmetrics and -M, read about 1 s into the settle phase",
            "socket_power_w": field("current_socket_power"), "power_cap_w": field("Max Graphics Package Power"),
            "gfxclk_mhz_per_xcd": field("current_gfxclks"), "gfx_activity_pct": field("average_gfx_activity"),
            "umc_activity_pct": field("average_umc_activity")}


def timed_steps(step, args, dev, with_repeats=False):
    """Warm-up and synchronise, then a settle phase and the timed region back
    to back: the settle launches keep the GPU busy up to the first timed step,
    so the timed region starts in the steady state with no idle gap (after an
    idle gap the engine clock overshoots and the first launches run up to 1.5x
    slower).  step(i) enqueues step i on torch's current stream, the stream
    every entry point launches on.  The K timed steps are bracketed by HIP
    events on that stream (outer events around all K, and a pair around each
    step); the host synchronises after the last one.  Returns (per-step ms in
    launch order, ms per step between the outer events, settle record); with
    with_repeats, also the ms per step of args.repeats blocks of K steps: the
    timed block, then the further blocks right behind it (each step bracketed
    by events like the others, outer events per block)."""
    import torch

    stream = torch.cuda.current_stream(dev)
    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
    outer = (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
    settle = {"ms": 0.0, "launches": 0}
    settle_ms, tel = args.settle_ms, None
    if getattr(args, "telemetry", False):
        settle_ms, tel = max(settle_ms, 3000.0), start_telemetry()
    if settle_ms > 0:
        bracket = (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
        settle = _settle(lambda n: step(args.warmup + n), stream, settle_ms, bracket)
    outer[0].record(stream)
    for i in range(args.steps):
        ev[i][0].record(stream)
        step(i)
        ev[i][1].record(stream)
    outer[1].record(stream)
    blocks = []
    if with_repeats:
        bracket = (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
        for _ in range(args.repeats - 1):
            o = (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
            o[0].record(stream)
            for i in range(args.steps):
                bracket[0].record(stream)
                step(i)
                bracket[1].record(stream)
            o[1].record(stream)
            blocks.append(o)
    torch.cuda.synchronize()
    if tel is not None:
        settle["telemetry"] = finish_telemetry(tel)
    ms_per_step = outer[0].elapsed_time(outer[1]) / args.steps
    res = ([a.elapsed_time(b) for a, b in ev], ms_per_step, settle)
    if with_repeats:
        return res + ([ms_per_step] + [a.elapsed_time(b) / args.steps for a, b in blocks],)
    return res


def graph_steps(step, args, dev, repeats=1):
    """The timed steps submitted as one HIP graph: args.steps calls of step(i)
    captured once (torch.cuda.CUDAGraph on torch's capture stream, which every
    entry point launches on), replayed untimed for --settle-ms, then one timed
    replay right behind them, bracketed by HIP events, and repeats - 1 more
    timed replays right behind that.  Only entry points that allocate nothing
    can be captured (the fused MGN kernels).  Returns (ms per step of the first
    timed replay, settle record, ms per step of every timed replay)."""
    import torch

    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(args.steps):
            step(i)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(dev)
    settle = {"ms": 0.0, "launches": 0}
    if args.settle_ms > 0:
        settle = _settle(lambda n: g.replay(), stream, args.settle_ms)
        settle["launches"] *= args.steps
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(repeats)]
    for e0, e1 in evs:
        e0.record(stream)
        g.replay()
        e1.record(stream)
    torch.cuda.synchronize()
    blocks = [e0.elapsed_time(e1) / args.steps for e0, e1 in evs]
    return blocks[0], settle, blocks


def bench_bert(args):
    """one gp_bert_ffn_out call over M = 65,536 rows per step."""
    import torch

    import gpipes
    from gpipes.synth import bert_params, normal_fp16

    dev = torch.device("cuda:0")
    M, H, FF, eps = BERT["M"], BERT["H"], BERT["FF"], BERT["eps"]
    et = torch.bfloat16 if args.dtype == "bf16" else torch.float16
    p = {k: v.to(et).to(dev) for k, v in bert_params(H, FF, seed=0, init="bert").items()}
    x = normal_fp16(M, H, seed=0, device=dev, dtype=et)
    out = torch.empty_like(x)

    def step(i):
        gpipes.bert_ffn_out(x, p["w1"], p["b1"], p["w2"], p["b2"], p["gamma"], p["beta"], out, eps=eps,
                            act="gelu_tanh")

    call_ms, ms_per_step, settle = timed_steps(step, args, dev)
    avg_ms = sum(call_ms) / len(call_ms)
    flops = 2 * 2 * M * H * FF  # the two GEMMs; GELU, residual and LayerNorm are O(M H) and O(M FF)
    tflops = flops / (avg_ms * 1e-3) / 1e12
    bytes_ = (M * H * 2) * 2 + 2 * H * FF * 2 + (FF + 3 * H) * 2  # x in, out, weights, vectors
    rec = {
        "metric": BERT_METRIC,
        "value": M / (ms_per_step * 1e-3),
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": args.dtype,
        "data": "synthetic (X~N(0,1), W~N(0,0.02), b=0, seed 0)",
        "config": {"workload": "bert_large_ffn", "M": M, "H": H, "FF": FF, "act": "gelu_tanh", "eps": eps,
                   "layers": f"{H}-{FF}-{H}+residual+LN", "accumulate": "f32", "row_chunk": 16384},
        "roofline": {
            "bound": "mfma", "achieved": tflops, "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": tflops / MFMA_F16_PEAK_TFLOPS, "traffic": None,
            "kernel_ms_avg": avg_ms, "kernel_ms_median": spread(call_ms)["median"],
            "flops_per_launch": flops, "algorithmic_bytes_per_launch": bytes_,
            "launch": "one gp_bert_ffn_out call (one weight-transpose launch, then per 16384-row chunk: "
                      "GEMM1+bias+GELU, GEMM2+bias+residual+LayerNorm)",
        },
        "spread": spread(call_ms),
        "settle": settle,
        "cpu_baseline": None if args.no_cpu or args.dtype != "f16" else cpu_baseline_bert(),
    }
    print(json.dumps(rec), flush=True)


DLRM_BOT = [16, 512, 256, 128]
DLRM_TOP = [480, 1024, 1024, 512, 256, 1]
CHAIN_METRIC = {
    "dlrm": "rows/sec + % fp16 MFMA peak, DLRM bottom+top MLPs M=262144 (1×MI355X)",
    "nerf": "samples/sec + % fp16 MFMA peak, NeRF full MLP M=1048576 (1×MI355X)",
    "bert_addln": "rows/sec + % fp16 MFMA peak, bert_addln_ffn H=128 FF=512 M=32768 (1×MI355X)",
    "nerf_a": "samples/sec + % fp16 MFMA peak, NerfA trunk M=65536 (1×MI355X)",
    "bert_app": "rows/sec + % fp16 MFMA peak, bert_ffn app H=128 FF=512 M=32768 (1×MI355X)",
}
# The reference apps' own batches: apps/bert_addln_ffn/pipelined/perf.py (64 x 512 rows)
# and apps/nerf_a/pipelined/val.py (65,536 samples).
ADDLN = {"M": 64 * 512, "H": 128, "FF": 512}
NERF_A = {"M": 65536, "Kx": 64}


def chain_flops(widths):
    return sum(2 * widths[i] * widths[i + 1] for i in range(len(widths) - 1))


NERF_FLOPS = 2 * (64 * 256 + 4 * 256 * 256 + 320 * 256 + 2 * 256 * 256 + 256 * 1 + 256 * 256 + 283 * 128 + 128 * 3)


def cpu_baseline_chain(workload, budget_s=10.0):
    """The CPU oracle (oracle.mlp / oracle.nerf over oracle/oracle.c) on a row sample."""
    import oracle
    from gpipes.synth import (bert_addln_params, dlrm_params, nerf_a_params, nerf_inputs, nerf_params, normal_fp16,
                              padded_normal, padded_uniform)

    threads, how = host_cores()
    oracle.set_num_threads(threads)
    f = lambda ts: [t.float().numpy() for t in ts]  # noqa: E731
    if workload == "dlrm":
        Ms = 2048
        wb, bb = dlrm_params(DLRM_BOT, seed=0)
        wt, bt = dlrm_params(DLRM_TOP, seed=1)
        xb, xt = padded_uniform(Ms, 13, 16, seed=2).float().numpy(), padded_normal(Ms, 479, 480, seed=3).float().numpy()
        wb, bb, wt, bt = f(wb), f(bb), f(wt), f(bt)
        R, S = oracle.ACT_RELU, oracle.ACT_SIGMOID

        def run():
            oracle.mlp(xb, wb, bb, [R] * 3)
            oracle.mlp(xt, wt, bt, [R] * 4 + [S])
        what = f"oracle DlrmMlp bottom {DLRM_BOT} + top {DLRM_TOP} fp32 on {Ms} rows"
    elif workload == "nerf":
        Ms = 2048
        ws, bs = nerf_params(64, 27, 1, 3, seed=0)
        x, d = nerf_inputs(Ms, seed=0)
        ws, bs, x, d = f(ws), f(bs), x.float().numpy(), d.float().numpy()

        def run():
            oracle.nerf(x, d, ws, bs, oracle.ACT_SIGMOID)
        what = f"oracle Nerf fp32 on {Ms} samples"
    elif workload == "bert_addln":
        Ms = 4096
        p = {k: v.float().numpy() for k, v in bert_addln_params(seed=0).items()}
        attn, x = (normal_fp16(Ms, 128, seed=i).float().numpy() for i in (0, 1))
        keys = ("w0", "b0", "w1", "b1", "w2", "b2", "ga0", "be0", "ga2", "be2")

        def run():
            oracle.bert_addln_ffn(attn, x, *(p[k] for k in keys))
        what = f"oracle bert_addln_ffn fp32 on {Ms} rows"
    elif workload == "bert_app":
        from gpipes.synth import bert_params
        Ms = 4096
        p = {k: v.float().numpy() for k, v in bert_params(128, 512, seed=0, init="torch").items()}
        x = normal_fp16(Ms, 128, seed=0).float().numpy()

        def run():
            oracle.bert_ffn(x, p["w1"], p["b1"], p["w2"], p["b2"], p["gamma"], p["beta"], act=oracle.ACT_RELU,
                            eps=1e-5)
        what = f"oracle BertFfn fp32 on {Ms} rows"
    else:
        Ms = 2048
        ws, bs = nerf_a_params(64, seed=0)
        ws, bs = f(ws), f(bs)
        x = normal_fp16(Ms, 64, seed=0).float().numpy()

        def run():
            oracle.nerf_a(x, ws, bs)
        what = f"oracle NerfA fp32 on {Ms} samples"
    med, n, tot = _median_runs(run, budget_s, min_runs=3, warmups=1)
    return {"value": Ms / med, "unit": "samples/s" if workload.startswith("nerf") else "rows/s", "cores": threads,
            "kind": "port", "sample": f"{what}, {threads} threads ({how}), median of {n} calls ({tot:.1f} s): "
                                      f"{med * 1e3:.1f} ms"}


def bench_chain(args):
    """configs[3] (DLRM bottom + top MLP, M = 262,144), configs[4] (NeRF, M = 1,048,576), or the
    bert_addln_ffn / nerf_a apps at their reference batches."""
    import torch

    import gpipes
    from gpipes.synth import (bert_addln_params, bert_params, dlrm_params, nerf_a_params, nerf_inputs, nerf_params,
                              normal_fp16, padded_normal, padded_uniform)

    dev = torch.device("cuda:0")
    # element type of every tensor: the fp16 values drawn below, rounded to bf16 for --dtype bf16
    et = torch.bfloat16 if args.dtype == "bf16" else torch.float16
    if args.workload == "dlrm":
        M = 262144
        wb, bb = dlrm_params(DLRM_BOT, seed=0)
        wb[0][13:] = 0
        wt, bt = dlrm_params(DLRM_TOP, seed=1)
        wt[0][479:] = 0
        wb, bb, wt, bt = ([t.to(et).to(dev) for t in ts] for ts in (wb, bb, wt, bt))
        xb = padded_uniform(M, 13, 16, seed=2, device=dev).to(et)
        xt = padded_normal(M, 479, 480, seed=3, device=dev).to(et)
        ob = torch.empty((M, 128), dtype=et, device=dev)
        ot = torch.empty((M, 1), dtype=et, device=dev)

        def step(i):
            gpipes.mlp_out(xb, wb, bb, ["relu"] * 3, ob)
            gpipes.mlp_out(xt, wt, bt, ["relu"] * 4 + ["sigmoid"], ot)
        flops = M * (chain_flops(DLRM_BOT) + chain_flops(DLRM_TOP))
        bytes_ = M * (16 + 128 + 480 + 1) * 2
        config = {"workload": "dlrm_bottom_top_mlp", "M": M, "bottom": "16(13)-512-256-128 ReLU",
                  "top": "480(479)-1024-1024-512-256 ReLU, 256-1 sigmoid", "accumulate": "f32", "row_chunk": 262144}
        data = "synthetic (dense U(0,1), top input N(0,1), Xavier-uniform weights, seed 0)"
        unit = "rows/s"
    elif args.workload == "bert_addln":
        M, H, FF = ADDLN["M"], ADDLN["H"], ADDLN["FF"]
        p = {k: v.to(et).to(dev) for k, v in bert_addln_params(H, FF, seed=0).items()}
        attn, x = normal_fp16(M, H, seed=0, device=dev, dtype=et), normal_fp16(M, H, seed=1, device=dev, dtype=et)
        out = torch.empty_like(x)
        keys = ("w0", "b0", "w1", "b1", "w2", "b2", "ga0", "be0", "ga2", "be2")
        impl = "pipelined" if args.impl == "pipelined" else "fused"
        if et == torch.bfloat16 and impl == "pipelined":
            raise SystemExit("the pipelined bert_addln layout runs in f16 only")

        def step(i):
            gpipes.bert_addln_ffn_out(attn, x, *(p[k] for k in keys), out, impl=impl)
        flops = 2 * M * (H * H + H * FF + FF * H)
        bytes_ = M * H * 2 * 3
        config = {"workload": "bert_addln_ffn", "M": M, "H": H, "FF": FF, "act": "relu", "eps": 1e-5,
                  "impl": impl, "accumulate": "f32"}
        data = "synthetic (attn_out, x ~ N(0,1), nn.Linear default init, seed 0)"
        unit = "rows/s"
    elif args.workload == "bert_app":
        # the bert_ffn app at its batch (apps/bert_ffn/pipelined/val.py: 64 x 512 rows, H 128, FF 512, ReLU)
        M, H, FF = ADDLN["M"], ADDLN["H"], ADDLN["FF"]
        p = {k: v.to(et).to(dev) for k, v in bert_params(H, FF, seed=0, init="torch").items()}
        x = normal_fp16(M, H, seed=0, device=dev, dtype=et)
        out = torch.empty_like(x)
        impl = "pipelined" if args.impl == "pipelined" else "fused"
        if et == torch.bfloat16 and impl == "pipelined":
            raise SystemExit("the pipelined bert_ffn layout runs in f16 only")

        def step(i):
            gpipes.bert_ffn_out(x, p["w1"], p["b1"], p["w2"], p["b2"], p["gamma"], p["beta"], out, impl=impl)
        flops = 4 * M * H * FF
        bytes_ = M * H * 2 * 2
        config = {"workload": "bert_ffn_app", "M": M, "H": H, "FF": FF, "act": "relu", "eps": 1e-5,
                  "impl": impl, "accumulate": "f32"}
        data = "synthetic (x ~ N(0,1), nn.Linear default init, seed 0)"
        unit = "rows/s"
    elif args.workload == "nerf_a":
        M, Kx = NERF_A["M"], NERF_A["Kx"]
        ws, bs = nerf_a_params(Kx, seed=0, device=dev)
        x = normal_fp16(M, Kx, seed=0, device=dev, dtype=et)
        out = torch.empty((M, 256), dtype=et, device=dev)
        wb = [t.to(et) for pair in zip(ws, bs) for t in pair]
        impl = "pipelined" if args.impl == "pipelined" else "fused"
        if et == torch.bfloat16 and impl == "pipelined":
            raise SystemExit("the pipelined nerf_a layout runs in f16 only")

        def step(i):
            gpipes.nerf_a_out(x, *wb, out, impl=impl)
        flops = 2 * M * (Kx * 256 + 4 * 256 * 256 + (256 + Kx) * 256 + 2 * 256 * 256)
        bytes_ = M * (Kx + 256) * 2
        config = {"workload": "nerf_a", "M": M, "Kx": Kx, "layers": "5x256 ReLU, skip concat, 3x256 ReLU",
                  "impl": impl, "accumulate": "f32"}
        data = "synthetic (x ~ N(0,1), nn.Linear default init, seed 0)"
        unit = "samples/s"
    else:
        M = 1048576
        ws, bs = nerf_params(64, 27, 1, 3, seed=0, device=dev)
        ws, bs = [w.to(et) for w in ws], [b.to(et) for b in bs]
        x, d = (t.to(et) for t in nerf_inputs(M, seed=0, device=dev))
        o_r = torch.empty((M, 1), dtype=et, device=dev)
        o_rgb = torch.empty((M, 3), dtype=et, device=dev)
        wb = [t for pair in zip(ws, bs) for t in pair]

        def step(i):
            gpipes.nerf_full_out(x, d, *wb, o_r, o_rgb, rgb_act="sigmoid")
        flops = M * NERF_FLOPS
        bytes_ = M * (64 + 27 + 1 + 3) * 2
        config = {"workload": "nerf_full_mlp", "M": M, "x": "63 encoded + 1 pad", "d": 27,
                  "layers": "8x256 ReLU (skip at 5), density 1, feature 256, 283-128 ReLU, 128-3 sigmoid",
                  "accumulate": "f32", "tile_rows": 256}
        data = "synthetic (positional encodings of U(-1,1) points and unit directions, Kaiming-uniform, seed 0)"
        unit = "samples/s"
    launch = {"dlrm": "one step: the bottom MLP as a weight-packing launch plus one fused three-layer kernel "
                      "over 256-row tiles; the top MLP as one weight-preparation launch, a wide-GEMM launch for "
                      "each of its first three layers, then a weight-packing launch plus one fused kernel for "
                      "512 -> 256 -> 1 (the click head)",
              "nerf": "one step: the weight-packing kernel, then the fused 12-layer kernel over 256-row tiles",
              "bert_addln": "one step: one gp_bert_addln_ffn_out call (fused: weight transposes, then GEMM0 + b0 + x, "
                            "LN0, GEMM1 + act, GEMM2 + b2 + h0, LN2; pipelined: one queue-chained kernel)",
              "nerf_a": "one step: one gp_nerf_a_out call (fused: the weight-packing kernel, then the NeRF kernel "
                        "stopped after layer 8; pipelined: one queue-chained kernel)",
              "bert_app": "one step: one gp_bert_ffn_impl_out call (fused: GEMM1 + b1 + act, GEMM2 + b2 + x with "
                          "the LayerNorm in its epilogue; pipelined: one queue-chained kernel)"}

    call_ms, ms_per_step, settle = timed_steps(step, args, dev)
    avg_ms = sum(call_ms) / len(call_ms)
    tflops = flops / (avg_ms * 1e-3) / 1e12
    rec = {
        "metric": CHAIN_METRIC[args.workload],
        "value": M / (ms_per_step * 1e-3),
        "unit": unit,
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": args.dtype,
        "data": data,
        "config": config,
        "roofline": {
            "bound": "mfma", "achieved": tflops, "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": tflops / MFMA_F16_PEAK_TFLOPS, "traffic": None,
            "kernel_ms_avg": avg_ms, "kernel_ms_median": spread(call_ms)["median"],
            "flops_per_launch": flops, "algorithmic_bytes_per_launch": bytes_,
            "launch": launch[args.workload],
        },
        "spread": spread(call_ms),
        "settle": settle,
        "cpu_baseline": None if args.no_cpu or args.dtype != "f16" else cpu_baseline_chain(args.workload),
    }
    print(json.dumps(rec), flush=True)


QUEUE_METRIC = "GB/s of queue hand-off (producer writes + consumer reads), 32 KiB tiles (1×MI355X)"
# The reference's A100 figures for the same 32 KiB payload (charts/qperf.py:8-21, the 32 KB
# row at :14; measured with misc_tests/pipeperf/pipeperf.cu:125-215): one queue, 54 queues.
QUEUE_REF_A100 = {"1_queue_gbs": 20.56, "54_queues_gbs": 1011.64}


def bench_queue(args):
    """Queue hand-off bandwidth over the ring queue (gp_pipe_route, GP_ROUTE_HANDOFF): one
    producer / consumer pair, then every pair the GPU holds.  A step moves T generated
    128 x 128 fp16 tiles (32 KiB) producer -> two-slot queue -> consumer in every pipeline;
    bandwidth counts the producer's writes and the consumer's reads, as the reference's
    "Bandwidth Total" does (pipeperf.cu:203-211).  The checksums of every step's tiles are
    checked against the closed form after the timed region."""
    import numpy as np
    import torch

    import gpipes

    dev = torch.device("cuda:0")
    tile = 128 * 128 * 2
    legs = {}
    for name, pipes, tiles in (("single_queue", 1, 20000), ("all_queues", 0, 262144)):
        M = tiles * 128
        out = torch.zeros(tiles, dtype=torch.int32, device=dev)

        def step(i, pipes=pipes, M=M, out=out):
            gpipes.pipe_handoff(M, max_pipes=pipes, out=out)

        call_ms, ms_per_step, settle = timed_steps(step, args, dev)
        gpipes.pipeline_check()
        ok = bool(np.array_equal(out.cpu().numpy().view(np.uint32), gpipes.handoff_checksums(M)))
        if not ok:
            raise SystemExit(f"hand-off checksums wrong ({name})")
        avg = sum(call_ms) / len(call_ms)
        legs[name] = {"tiles": tiles, "max_pipes": pipes, "kernel_ms_avg": avg, "ms_per_step": ms_per_step,
                      "gbs": 2 * tiles * tile / (avg * 1e-3) / 1e9, "spread": spread(call_ms), "settle": settle,
                      "checksums": "all tiles match"}
    full = legs["all_queues"]
    rec = {
        "metric": QUEUE_METRIC,
        "value": 2 * full["tiles"] * tile / (full["ms_per_step"] * 1e-3) / 1e9,
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": full["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u32",
        "data": "synthetic (generated tile payloads, per-tile checksums verified)",
        "config": {"workload": "queue_handoff", "payload_bytes": tile, "queue_slots": 2,
                   "route": "GP_ROUTE_HANDOFF", "tiles_per_step": full["tiles"]},
        "legs": legs,
        "reference_a100": QUEUE_REF_A100,
        "roofline": None,
        "cpu_baseline": None,
    }
    print(json.dumps(rec), flush=True)


def bench_mfma_peak(args):
    """The dense MFMA ceiling of the board as it runs: the probe kernel (gp_probe_mfma:
    two waves per SIMD of back-to-back MFMAs on register data, no memory traffic;
    --mfma-shape picks 32x32x16 or 16x16x32), one launch a step, timed like the other
    workloads.  With --telemetry the line also carries the socket power and engine
    clocks it ran at."""
    import torch

    import gpipes

    dev = torch.device("cuda:0")
    et = torch.bfloat16 if args.dtype == "bf16" else torch.float16
    iters, shape = 4096, args.mfma_shape
    flops = gpipes.probe_mfma(iters, et, shape=shape)
    instr = "v_mfma_f32_32x32x16" if shape == 32 else "v_mfma_f32_16x16x32"

    def step(i):
        gpipes.probe_mfma(iters, et, shape=shape)
    call_ms, ms_per_step, settle = timed_steps(step, args, dev)
    avg_ms = sum(call_ms) / len(call_ms)
    tflops = flops / (avg_ms * 1e-3) / 1e12
    rec = {
        "metric": f"TFLOP/s, dense {args.dtype} {instr} probe without memory traffic (1×MI355X)",
        "value": tflops, "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": ms_per_step, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": args.dtype, "data": "synthetic register operands in [-1, 1)",
        "config": {"workload": "mfma_peak_probe", "iters": iters, "waves_per_simd": 2,
                   "accumulators_per_wave": 8 if shape == 32 else 16, "instruction": instr},
        "roofline": {"bound": "mfma", "achieved": tflops, "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": tflops / MFMA_F16_PEAK_TFLOPS, "traffic": None, "kernel_ms_avg": avg_ms,
                     "flops_per_launch": flops},
        "spread": spread(call_ms),
        "settle": settle,
        "cpu_baseline": None,
    }
    if "telemetry" in settle:
        rec["telemetry"] = settle["telemetry"]
    print(json.dumps(rec), flush=True)


GEMM_SHAPES = [(16384, 1024, 4096), (16384, 4096, 1024), (262144, 1024, 1024), (262144, 512, 1024),
               (262144, 1024, 512), (8192, 8192, 8192)]


def bench_gemm(args):
    """The wide GEMM stage (gp_gemm_out, bias + ReLU epilogue, weights [K, N] as a caller
    holds them) against torch.matmul (hipBLASLt, no epilogue) on the BERT-large and DLRM
    layer shapes: one line per shape, HIP events over 20 calls after 5 untimed ones."""
    import torch

    import gpipes

    dev = torch.device("cuda:0")

    def timed(fn, n=20):
        for _ in range(5):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(n):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / n

    for (M, K, N) in GEMM_SHAPES:
        g = torch.Generator(device=dev).manual_seed(M + K + N)
        a = torch.randn(M, K, device=dev, generator=g).half()
        w = (torch.randn(K, N, device=dev, generator=g) * K ** -0.5).half()
        b = torch.randn(N, device=dev, generator=g).half()
        out = torch.empty(M, N, device=dev, dtype=torch.float16)
        ours = timed(lambda: gpipes.gemm_out(a, w, b, act="relu", out=out))
        lib_ms = timed(lambda: torch.matmul(a, w))
        flops = 2 * M * K * N
        print(json.dumps({
            "metric": "TFLOP/s, wide GEMM stage (bias + ReLU epilogue) against hipBLASLt (torch.matmul)",
            "value": flops / (ours * 1e-3) / 1e12, "unit": "TFLOP/s", "n_gpus": 1, "ms_per_step": ours,
            "higher_is_better": True, "dtype": "f16", "data": "synthetic (N(0,1) inputs, N(0,1/K) weights)",
            "config": {"workload": "gemm", "M": M, "K": K, "N": N,
                       "weights": "in place" if 2.0 * M * N * K < 8e10 else "transposed copy made by the call"},
            "library": {"name": f"torch {torch.__version__} matmul (hipBLASLt), no epilogue", "ms": lib_ms,
                        "tflops": flops / (lib_ms * 1e-3) / 1e12},
        }), flush=True)


def load_traffic(workload, impl):
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as fh:
            return json.load(fh).get(f"{workload}:{impl}")
    except (OSError, ValueError):
        return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--repeats", type=int, default=5,
                    help="MGN workloads: blocks of --steps timed steps per submission (the first is the "
                         "headline, the others follow it back to back; their median is reported beside it)")
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", choices=sorted(WORKLOADS) + ["bert", "dlrm", "nerf", "bert_addln", "bert_app", "nerf_a",
                                                               "queue", "mfma_peak", "gemm"],
                    default="edge")
    ap.add_argument("--impl", choices=["fused", "pipelined", "pipelined_split_ln"], default="fused")
    ap.add_argument("--settle-ms", type=float, default=1000.0,
                    help="untimed launches for this long between the warm-up and the timed region: the "
                         "engine clock swings for tens of ms after a burst starts (launches run fast, then "
                         "up to 1.5x slower, then settle), so the timed region starts in the steady state")
    ap.add_argument("--dtype", choices=["f16", "bf16"], default="f16",
                    help="element type of every tensor (bf16: the fused / wide-GEMM kernels only, not the headline "
                         "line)")
    ap.add_argument("--eager", action="store_true",
                    help="MGN fused workloads: time the steps as eager calls only (by default the same steps "
                         "are also timed as one HIP graph replay and `value` comes from the faster of the "
                         "two; the per-launch roofline times are eager in both cases)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cus", type=int, default=0,
                    help="size every launch for this many CUs instead of all of them (GPIPES_NUM_CUS); "
                         "diagnostics only, with --phase-timers: the cycles per tile at 128, 192, 256 CUs")
    ap.add_argument("--phase-timers", action="store_true",
                    help="fused MGN workloads: load the diagnostic library (libgpipes_phase.so: the fused "
                         "kernel with s_memtime phase timers, about 1%% slower) and add the last launch's "
                         "cycles per tile and phase to the line as \"phase_cycles\"; not a headline run")
    ap.add_argument("--telemetry", action="store_true",
                    help="read the board's socket power, power cap and per-XCD engine clocks (rocm-smi, in a "
                         "child process) during a settle phase of at least 3 s, and add them to the line's "
                         "\"settle\" record (and, for the MGN workloads, as \"telemetry\")")
    ap.add_argument("--mfma-shape", type=int, choices=[32, 16], default=32,
                    help="--workload mfma_peak: the probe's MFMA form, 32 (v_mfma_f32_32x32x16, the form the "
                         "fused kernels and the wide GEMM use) or 16 (v_mfma_f32_16x16x32)")
    ap.add_argument("--copy-ref", action="store_true",
                    help="first run one plain 1 GiB device copy (a known-size reference kernel "
                         "for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE counters)")
    args = ap.parse_args()

    if args.phase_timers:
        os.environ["GPIPES_PHASE_TIMERS"] = "1"  # before gpipes is imported
    if args.cus:
        os.environ["GPIPES_NUM_CUS"] = str(args.cus)  # read when the library first queries the device
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (the path needs no cross-GPU exchange; rows shard "
              f"trivially); --gpus {args.gpus} is not supported.", file=sys.stderr)
        sys.exit(2)

    if args.workload == "bert":
        bench_bert(args)
        return
    if args.workload in ("dlrm", "nerf", "bert_addln", "bert_app", "nerf_a"):
        bench_chain(args)
        return
    if args.workload == "queue":
        bench_queue(args)
        return
    if args.workload == "mfma_peak":
        bench_mfma_peak(args)
        return
    if args.workload == "gemm":
        bench_gemm(args)
        return

    import torch

    import gpipes
    from gpipes.synth import mgn_params

    dev = torch.device("cuda:0")
    M, K, ln = WORKLOADS[args.workload]
    et = torch.bfloat16 if args.dtype == "bf16" else torch.float16
    if et == torch.bfloat16 and (args.impl != "fused" or args.workload == "edge_gather"):
        print("bf16 runs on the fused kernel (edge / node workloads) only", file=sys.stderr)
        sys.exit(2)
    p = {k: (None if v is None else v.to(dev)) for k, v in mgn_params(K, seed=0, layernorm=ln, dtype=et).items()}
    # Inputs resident in HBM.  The node batch (201 MB) would fit the 256 MB
    # MALL, so two input/output buffer pairs are rotated to keep it honest.
    nbuf = 2 if args.workload == "node" else 1
    gather = args.workload == "edge_gather"
    if gather:
        if args.impl != "fused":
            print("the gather front end exists for the fused kernel only", file=sys.stderr)
            sys.exit(2)
        g = torch.Generator().manual_seed(0)
        nf = gpipes.fill_normal(torch.empty((GATHER_NODES, 128), dtype=torch.float16, device=dev), seed=1)
        xs = [gpipes.fill_normal(torch.empty((M, 128), dtype=torch.float16, device=dev), seed=0)]  # edge features
        src = torch.randint(0, GATHER_NODES, (M,), generator=g).to(dev)
        dst = torch.randint(0, GATHER_NODES, (M,), generator=g).to(dev)
    else:
        # X ~ N(0, 1) from the builder-owned generator (Philox-4x32-10 + Box-Muller,
        # gp_fill_normal), seed = buffer index; oracle.normal gives the same values on the host
        xs = [gpipes.fill_normal(torch.empty((M, K), dtype=et, device=dev), seed=i) for i in range(nbuf)]
    outs = [torch.empty((M, 128), dtype=et, device=dev) for _ in range(nbuf)]

    def step(i):
        b = i % nbuf
        if gather:
            gpipes.mgn_edge_gather_out(nf, xs[0], src, dst, p["w1"], p["b1"], p["w2"], p["b2"], p["w3"], p["b3"],
                                       p["gamma"], p["beta"], outs[0])
        else:
            gpipes.mgn_mlp_out(xs[b], p["w1"], p["b1"], p["w2"], p["b2"], p["w3"], p["b3"], p["gamma"],
                               p["beta"], outs[b], impl=args.impl)

    if args.copy_ref:
        ref_in = torch.ones(1 << 29, dtype=torch.float16, device=dev)  # 1 GiB
        ref_out = torch.empty_like(ref_in)
        ref_out.copy_(ref_in)
        torch.cuda.synchronize()
        del ref_in, ref_out

    launch_ms, eager_ms_per_step, settle, eager_blocks = timed_steps(step, args, dev, with_repeats=True)
    avg_launch_ms = sum(launch_ms) / len(launch_ms)
    # The fused kernels allocate nothing, so the same steps can also be
    # submitted as one HIP graph; `value` comes from the faster submission.
    graph_ms_per_step, graph_settle, graph_blocks = None, None, None
    if args.impl == "fused" and not args.eager:
        graph_ms_per_step, graph_settle, graph_blocks = graph_steps(step, args, dev, args.repeats)
    use_graph = graph_ms_per_step is not None and graph_ms_per_step < eager_ms_per_step
    ms_per_step = graph_ms_per_step if use_graph else eager_ms_per_step
    bytes_, flops = algorithmic(M, K, ln, GATHER_NODES if gather else 0)
    achieved_gbs = bytes_ / (avg_launch_ms * 1e-3) / 1e9
    tflops = flops / (avg_launch_ms * 1e-3) / 1e12

    rec = {
        "metric": METRIC if args.workload == "edge" else WORKLOAD_METRIC[args.workload],
        "value": M / (ms_per_step * 1e-3),
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": args.dtype,
        "data": "synthetic (X~N(0,1) from gp_fill_normal, Philox-4x32-10 + Box-Muller, seed 0; "
                "nn.Linear default init, seed 0)",
        "config": {"workload": f"mgn_{args.workload}_mlp", "M": M, "K": K,
                   **({"nodes": GATHER_NODES, "index": "int64"} if gather else {}),
                   "layers": f"{K}-128-128-128" + ("+LN" if ln else ""), "impl": args.impl,
                   "accumulate": "f32",
                   "submission": (f"one HIP graph of the {args.steps} timed calls" if use_graph
                                  else "eager calls from Python")},
        "timing": "HIP events on the launch stream around the timed steps, which follow the settle "
                  "submissions with no synchronisation in between; synchronised before the settle phase "
                  "and after the last step; value from the faster of eager and graph submission",
        "eager_ms_per_step": eager_ms_per_step,
        "graph_ms_per_step": graph_ms_per_step,
        # the timed block and args.repeats - 1 more blocks of K steps right behind it, per submission
        "repeats": {"blocks": args.repeats, "eager_ms_per_step": eager_blocks, "graph_ms_per_step": graph_blocks,
                    "median_ms_per_step": statistics.median(graph_blocks if use_graph else eager_blocks)},
        "roofline": {
            "bound": "hbm", "achieved": achieved_gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": achieved_gbs / HBM_PEAK_GBS, "traffic": load_traffic(args.workload, args.impl),
            "kernel_ms_avg": avg_launch_ms, "kernel_ms_median": spread(launch_ms)["median"],
            "algorithmic_bytes_per_launch": bytes_,
        },
        # the dense bf16 MFMA peak equals the fp16 one (2.5 PFLOP/s)
        "mfma": {"achieved_tflops": tflops, "peak_tflops": MFMA_F16_PEAK_TFLOPS,
                 "frac": tflops / MFMA_F16_PEAK_TFLOPS, "flops_per_launch": flops},
        "spread": spread(launch_ms),
        "settle": settle,
        "graph_settle": graph_settle,
        "cpu_baseline": None if args.no_cpu or args.dtype != "f16" else cpu_baseline_torch_mgn(K, ln),
        "cpu_baseline_oracle": None if args.no_cpu or args.dtype != "f16" else cpu_baseline(K, ln),
    }
    if args.phase_timers and args.impl == "fused":
        step(0)  # the timers hold the last launch
        rec["phase_cycles"] = gpipes.phase_timers()
        rec["library"] = "libgpipes_phase.so (diagnostic build with phase timers)"
    if args.cus:
        rec["config"]["cus"] = args.cus
    if "telemetry" in settle:
        rec["telemetry"] = settle["telemetry"]
    print(json.dumps(rec), flush=True)


if __name__ == "__main__":
    main()
