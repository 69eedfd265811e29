"""Benchmark of the packed-expert routed-MoE hot path on one MI355X.

Default workload: the Qwen3-30B-A3B-shape MoE layer (hidden 2048, 128 experts of
intermediate 768, top-8 renormalised softmax over random near-uniform router logits), int4
group-128 experts with fp16 scales, bf16 activations, decoding ONE token. A step is one
token through a stack of 48 such layers, all resident in HBM (14.9 GB, so the weights
come from HBM and not the 256 MB Infinity Cache); each layer is the two decode kernels
(gate/up + down with the fixed-order weighted sum) on its own routed experts, recorded in
one HIP graph and replayed. The reported value is microseconds per token per MoE layer.

The pointer tables and activations are resident before timing starts (the engine builds a
layer's table from its routing; here routing is drawn once per layer).

    python bench.py [--steps K] [--warmup W] [--layers L] [--no-cpu]
"""
import argparse
import json
import os
import sys
import time

import numpy as np
import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "int4 MoE layer µs/token + achieved HBM GB/s (% of 8 TB/s) / MFMA util"
HBM_PEAK_GBS = 8000.0


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--layers", type=int, default=None,
                   help="resident layers per step (default 48; 8 Mixtral, 6 DeepSeek-V3)")
    p.add_argument("--distinct", type=int, default=2,
                   help="distinct random layers; the rest are byte copies at new addresses")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    p.add_argument("--no-routed", action="store_true",
                   help="headline decode: skip the routed-layer extra fields")
    p.add_argument("--one-launch", action="store_true",
                   help="decode: also time the one-launch layer (vaayu_decode_fused) and make it "
                        "the value (measured slower than the two launches on MI355X)")
    p.add_argument("--cpu-seconds", type=float, default=12.0)
    p.add_argument("--workload", default="qwen3-decode", choices=sorted(WORKLOADS),
                   help="qwen3-decode (default) is the headline line; the others are the "
                        "prefill-path shapes")
    p.add_argument("--summarize", nargs="+", metavar="DIR",
                   help="print a text summary of rocprofv3 csv output directories "
                        "(a --kernel-trace --stats run and --pmc FETCH_SIZE / WRITE_SIZE runs) "
                        "and exit; no GPU is used")
    return p.parse_args()


# ── rocprofv3 summaries ─────────────────────────────────────────────────────────────────
#
# Every run does one calibration pass first: an elementwise negation of a 256 MiB fp32
# buffer into another (reads exactly 256 MiB, writes exactly 256 MiB). FETCH_SIZE and
# WRITE_SIZE of a dispatch are scaled by (256 MiB / what the counter reads for that
# calibration dispatch), which turns the counters into HBM bytes.
CALIB_BYTES = 256 << 20
WARM_MS = 150.0              # each graph's replays before it is timed, in ms of GPU work
TRAFFIC_FILES = {"qwen3-decode": "decode_qwen3_b1_traffic.txt",
                 "mixtral-decode": "decode_mixtral_b1_traffic.txt",
                 "dsv3-decode": "decode_dsv3_b1_traffic.txt",
                 "dsv3-prefill": "prefill_dsv3_2048_traffic.txt",
                 "mixtral-prefill": "prefill_mixtral_512_traffic.txt",
                 "qwen3-prefill": "prefill_qwen3_256_traffic.txt",
                 "gptoss-20b-prefill": "fused3d_gptoss20b_prefill_2048_traffic.txt"}
GU_KERNEL = "mfma_gate_up_kernel"     # the decode gate/up kernel bf16 activations run
DN_KERNEL = "mfma_down_kernel"
PF_KERNELS = ("prefill_gate_up_kernel", "prefill_down_kernel", "prefill_reduce_kernel")
F3_KERNELS = ("fused3d_gate_up_kernel", "fused3d_down_kernel", "prefill_reduce_kernel")
TRAFFIC_KERNELS = (GU_KERNEL, DN_KERNEL) + PF_KERNELS + F3_KERNELS[:2]


def _csv_rows(d, suffix):
    import csv
    import glob
    rows = []
    for f in sorted(glob.glob(os.path.join(d, "**", "*" + suffix), recursive=True)):
        with open(f, newline="") as fh:
            rows += list(csv.DictReader(fh))
    return rows


def _short(name):
    name = name.split("(")[0]
    return name[:90]


MARK_KERNEL = "bitwise_not"            # the marker launched around each timed region


def _regions(d):
    """Per-kernel durations inside each timed region of a kernel trace: the dispatches
    between the marker dispatches that open and close it (the first marker is the one
    launched when the markers are set up; region k lies between markers 2k + 1 and 2k + 2,
    and the warm-up of the next region between 2k + 2 and 2k + 3)."""
    rows = _csv_rows(d, "kernel_trace.csv")
    rows.sort(key=lambda r: int(r["Start_Timestamp"]))
    marks = [i for i, r in enumerate(rows) if MARK_KERNEL in r["Kernel_Name"]][1:]
    out = []
    for k, (a, b) in enumerate(zip(marks[0::2], marks[1::2])):
        inside = rows[a + 1:b]
        if not inside:
            continue
        per = {}
        for r in inside:
            per.setdefault(_short(r["Kernel_Name"]), []).append(
                (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
        span = (int(inside[-1]["End_Timestamp"]) - int(inside[0]["Start_Timestamp"])) / 1e3
        out.append(f"region {k}: {len(inside)} dispatches, span {span:.1f} us "
                   f"(first start to last end)")
        for name, ds in sorted(per.items()):
            out.append(f"  {name:<88} {len(ds):>7} {sum(ds) / len(ds):>9.3f} {min(ds):>9.3f} "
                       f"{max(ds):>9.3f}")
    return out


def summarize(dirs):
    """Text summary of rocprofv3 csv output: per-kernel durations (kernel_stats.csv), the
    same inside each timed region (kernel_trace.csv, cut at the marker dispatches), and
    per-kernel average FETCH_SIZE / WRITE_SIZE and SQ counters (counter_collection.csv),
    the byte counters scaled by the calibration dispatch."""
    out = []
    for d in dirs:
        for r in _csv_rows(d, "kernel_stats.csv"):
            if not out:
                out.append(f"{'kernel':<90} {'calls':>7} {'avg us':>9} {'min us':>9} "
                           f"{'max us':>9} {'%':>6}")
            out.append(f"{_short(r['Name']):<90} {int(r['Calls']):>7} "
                       f"{float(r['AverageNs']) / 1e3:>9.3f} {float(r['MinNs']) / 1e3:>9.3f} "
                       f"{float(r['MaxNs']) / 1e3:>9.3f} {float(r['Percentage']):>6.2f}")
    for d in dirs:
        regions = _regions(d)
        if regions:
            out.append("")
            out.append(f"timed regions (kernel, dispatches, avg us, min us, max us):")
            out += regions
    per = {}
    for d in dirs:
        for r in _csv_rows(d, "counter_collection.csv"):
            key = (_short(r["Kernel_Name"]), r["Counter_Name"])
            per.setdefault(key, []).append(float(r["Counter_Value"]))
    if per:
        factors = {}
        for (name, ctr), vals in per.items():
            if "neg" in name and ctr in ("FETCH_SIZE", "WRITE_SIZE"):
                factors[ctr] = CALIB_BYTES / (max(vals) * 1024.0)   # 256 MiB each way
        out.append("")
        out.append("counter scale factors (HBM bytes per KiB counted, from the calibration "
                   "copy of 256 MiB): " + ", ".join(f"{c} {f * 1024:.4f}"
                                                     for c, f in sorted(factors.items())))
        out.append(f"{'kernel':<90} {'counter':>10} {'dispatches':>10} {'avg KiB':>12} "
                   f"{'bytes/launch':>14}")
        for (name, ctr), vals in sorted(per.items()):
            avg = sum(vals) / len(vals)
            if ctr not in ("FETCH_SIZE", "WRITE_SIZE"):
                out.append(f"{name:<90} {ctr:>10} {len(vals):>10} {avg:>12.1f}")
                continue
            scaled = avg * 1024.0 * factors.get(ctr, 1.0)
            out.append(f"{name:<90} {ctr:>10} {len(vals):>10} {avg:>12.1f} {scaled:>14.0f}")
            tag = next((k for k in TRAFFIC_KERNELS if k in name), None)
            if tag is not None:
                out.append(f"traffic_bytes {tag} {ctr} {scaled:.0f}")
        # bytes read from memory by L2 misses, counted by request size: exact for the
        # calibration copy (no scale factor), unlike FETCH_SIZE on this chip
        sizes = {"TCC_EA0_RDREQ_32B_sum": 32, "TCC_EA0_RDREQ_64B_sum": 64,
                 "TCC_EA0_RDREQ_128B_sum": 128}
        names = sorted({n for (n, c) in per if c in sizes})
        if names:
            out.append("")
            out.append(f"{'kernel':<90} {'read bytes/dispatch (32/64/128-byte requests)':>46}")
        for name in names:
            if not all((name, c) in per for c in sizes):
                continue
            rb = sum(w * sum(per[(name, c)]) / len(per[(name, c)]) for c, w in sizes.items())
            out.append(f"{name:<90} {rb:>46.0f}")
            tag = next((k for k in TRAFFIC_KERNELS if k in name), None)
            if tag is not None:
                out.append(f"traffic_bytes {tag} READ_BYTES {rb:.0f}")
    return "\n".join(out)


def traffic_from_profile(workload, kernels, launches=1):
    """HBM bytes per call of the named kernels (bytes read + WRITE_SIZE per dispatch, times
    `launches` dispatches of each per call) from the committed counter summary of this
    workload, or None when any of them is missing there. Bytes read are the per-size
    request counts (READ_BYTES) where the summary has them, else the scaled FETCH_SIZE."""
    path = os.path.join(ROOT, "profiles", TRAFFIC_FILES.get(workload, "-"))
    if not os.path.exists(path):
        return None
    got = {}
    for line in open(path):
        f = line.split()
        if len(f) == 4 and f[0] == "traffic_bytes" and f[1] in kernels:
            got[(f[1], f[2])] = float(f[3])
    total = 0.0
    for k in kernels:
        read = got.get((k, "READ_BYTES"), got.get((k, "FETCH_SIZE")))
        if read is None or (k, "WRITE_SIZE") not in got:
            return None
        total += read + got[(k, "WRITE_SIZE")]
    return round(total * launches)


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def calibrate_counters(dev):
    """A plain elementwise pass of known size (256 MiB read, 256 MiB written), so a counter
    profile of this run can scale FETCH_SIZE / WRITE_SIZE to bytes."""
    src = torch.ones(CALIB_BYTES // 4, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    torch.neg(src, out=dst)
    torch.cuda.synchronize()
    del src, dst


class Marks:
    """A one-element bitwise-not launched between timed regions, so a kernel trace of this
    run can be cut into exactly the replays each figure of the line comes from. It is
    launched once at construction: the first launch of a torch kernel in a process loads
    its code, and that load slowed the GPU work timed right after it (the Mixtral prefill
    layer 654 -> 770 us, for the first region only)."""

    def __init__(self, dev):
        self.buf = torch.zeros(1, dtype=torch.int32, device=dev)
        self()
        torch.cuda.synchronize()

    def __call__(self):
        self.buf.bitwise_not_()


def timed_regions(graphs, steps, warmup, dev):
    """{name: ms per replay} of each (name, graph): each graph gets `warmup` replays, then
    replays for WARM_MS more, right before `steps` replays between HIP events on the
    current stream, bracketed by a marker dispatch on each side. The timed replays so run
    in the GPU's sustained state under that load: after a few ms of replays the prefill
    layers ran up to 14 % slower than after 150 ms (Mixtral 742 vs 651 us), while the
    decode layer runs about 1.5 % faster before its clocks settle (10.14 vs 10.30 us)."""
    mark = Marks(dev)
    spans = []
    for _name, graph in graphs:
        for _ in range(warmup):
            graph.replay()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        graph.replay()
        b.record()
        torch.cuda.synchronize()
        for _ in range(int(WARM_MS / max(a.elapsed_time(b), 1e-3))):
            graph.replay()
        torch.cuda.synchronize()
        mark()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(steps):
            graph.replay()
        b.record()
        mark()
        spans.append((a, b))
    torch.cuda.synchronize()
    return {name: a.elapsed_time(b) / steps for (name, _g), (a, b) in zip(graphs, spans)}


def host_cpus():
    """What the host offers the CPU baseline: os.cpu_count(), lscpu's topology, and the
    cgroup's CPU quota when one is set."""
    info = {"os_cpu_count": os.cpu_count()}
    try:
        import subprocess
        text = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        kv = dict(line.split(":", 1) for line in text.splitlines() if ":" in line)
        get = lambda k: kv.get(k, "").strip()
        info["lscpu"] = (f"{get('Socket(s)')} sockets x {get('Core(s) per socket')} cores x "
                         f"{get('Thread(s) per core')} threads = {get('CPU(s)')} CPUs "
                         f"({get('Model name')})")
    except Exception as exc:
        info["lscpu"] = f"unavailable: {exc}"
    try:
        quota, period = open("/sys/fs/cgroup/cpu.max").read().split()
        info["cgroup_cpus"] = None if quota == "max" else round(int(quota) / int(period), 2)
    except Exception:
        info["cgroup_cpus"] = None
    return info


def cpu_leg(run_one, seconds, unit_per_call):
    """The CPU baseline timed at torch's thread count for the whole host (os.cpu_count())
    and at the cgroup's CPU share when that is smaller: (best, {threads: value}). `run_one(i)`
    runs the i-th call of the bounded sample; each setting runs for about `seconds`."""
    info = host_cpus()
    settings = [info["os_cpu_count"] or 1]
    share = info.get("cgroup_cpus")
    if share and int(share) < settings[0]:
        settings.append(max(int(share), 1))
    default = torch.get_num_threads()
    by_threads = {}
    for threads in settings:
        torch.set_num_threads(threads)
        run_one(0)                                         # warm
        n, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < seconds or n == 0:
            run_one(n)
            n += 1
        by_threads[threads] = ((time.perf_counter() - t0) * unit_per_call / n, n,
                               time.perf_counter() - t0)
    torch.set_num_threads(default)
    best = min(by_threads, key=lambda t: by_threads[t][0])
    return best, by_threads, info


def route(logits, top_k):
    """softmax of fp32 logits, top-k, renormalised (the fused forward's bare-logits branch)."""
    w, idx = torch.topk(logits.float().softmax(dim=-1), top_k, dim=-1)
    return w / w.sum(dim=-1, keepdim=True), idx


# ── prefill-path workloads ──────────────────────────────────────────────────────────────
#
# A multi-token call runs the three grouped kernels (gate/up, down, the expert-id-order
# reduce) over the call's tables. The tables and activations are resident before timing
# (the engine builds them from the call's routing on the host); the three launches are
# recorded in one HIP graph and replayed.
WORKLOADS = {
    "qwen3-decode": None,      # the headline decode line (main)
    "qwen3-fp8-decode": dict(name="Qwen3-30B-A3B-shape MoE layer decode, 1 token, FP8 e4m3 "
                                  "experts with fp32 scales per 128 x 128 block", fmt="e4m3"),
    "qwen3-mxfp4-decode": dict(name="Qwen3-30B-A3B-shape MoE layer decode, 1 token, MXFP4 "
                                    "e2m1 experts with E8M0 scales per 32", fmt="mxfp4"),
    "qwen3-decode-routed": dict(name="Qwen3-30B-A3B-shape MoE layer decode, 1 token, int4 g128 "
                                     "fp16 scales, router product + softmax top-k + pair table "
                                     "on the GPU in the same graph", fmt="int4", routed=True),
    "dsv3-prefill": dict(name="DeepSeek-V3-shape MoE layer prefill, 2048 tokens", hidden=7168,
                         inter=2048, experts=256, top_k=8, tokens=2048, routing="zipf",
                         shared=True, bound="mfma"),
    "mixtral-prefill": dict(name="Mixtral-8x7B-shape MoE layer prefill, 512 tokens", hidden=4096,
                            inter=14336, experts=8, top_k=2, tokens=512, routing="softmax",
                            shared=False, bound="mfma"),
    "qwen3next-gdn-decode": dict(name="Qwen3-Next-80B-shape gated-delta mixer decode, 1 token: "
                                      "conv update + recurrent rule + gated norm",
                                 gdn=True, HV=32, HK=16, K=128, V=128, W=4, mixers=36,
                                 copies=8),
    "gptoss-20b-prefill": dict(name="gpt-oss-20b-shape fused-3D MXFP4 MoE layer prefill, 2048 "
                                    "tokens (32 experts, hidden 2880, inter 2880, top-4)",
                               fused3d=True, hidden=2880, inter=2880, experts=32, top_k=4,
                               tokens=2048),
    "mixtral-decode": dict(name="Mixtral-8x7B-shape MoE layer decode, 1 token, int4 g128 fp16 "
                                "scales", fmt="int4", decode_shape=dict(hidden=4096, inter=14336,
                                experts=8, top_k=2, layers=8, shared=False)),
    "dsv3-decode": dict(name="DeepSeek-V3-shape MoE layer decode, 1 token, int4 g128 fp16 "
                             "scales, 8 of 256 routed experts + 1 shared expert", fmt="int4",
                        decode_shape=dict(hidden=7168, inter=2048, experts=256, top_k=8,
                                          layers=6, shared=True)),
    "qwen3-decode-b8": dict(name="Qwen3-30B-A3B-shape MoE layer decode, batch of 8 tokens",
                            hidden=2048, inter=768, experts=128, top_k=8, tokens=8,
                            routing="softmax", shared=False, bound="hbm"),
    "qwen3-prefill": dict(name="Qwen3-30B-A3B-shape MoE layer prefill, 256 tokens", hidden=2048,
                          inter=768, experts=128, top_k=8, tokens=256, routing="softmax",
                          shared=False, bound="hbm"),
    "qwen3-fp8-prefill": dict(name="Qwen3-30B-A3B-shape MoE layer prefill, 256 tokens, FP8 e4m3 "
                                   "experts with fp32 scales per 128 x 128 block", hidden=2048,
                              inter=768, experts=128, top_k=8, tokens=256, routing="softmax",
                              shared=False, bound="hbm", fmt="e4m3"),
    "qwen3-mxfp4-prefill": dict(name="Qwen3-30B-A3B-shape MoE layer prefill, 256 tokens, MXFP4 "
                                     "e2m1 experts with E8M0 scales per 32", hidden=2048,
                                inter=768, experts=128, top_k=8, tokens=256, routing="softmax",
                                shared=False, bound="hbm", fmt="mxfp4"),
}
MFMA_PEAK_TFLOPS = 2500.0


def measured_mfma_peak(dev, blocks=4096, iters=2048):
    """bf16 dense MFMA TFLOP/s this device sustains (`vaayu_probe_mfma`: 16 independent
    v_mfma_f32_16x16x32_bf16 chains per wave from registers, 16 waves per CU), best of 3."""
    from vaayu_amd import _lib
    lib = _lib.load()
    out = torch.empty(blocks * 256, dtype=torch.float32, device=dev)
    st = torch.cuda.current_stream(dev).cuda_stream
    _lib.check(lib.vaayu_probe_mfma(out.data_ptr(), blocks, 16, st), "mfma probe")
    best = None
    for _ in range(3):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        _lib.check(lib.vaayu_probe_mfma(out.data_ptr(), blocks, iters, st), "mfma probe")
        b.record()
        torch.cuda.synchronize()
        tf = blocks * 4 * iters * 16 * 16384 / (a.elapsed_time(b) * 1e-3) / 1e12
        best = tf if best is None else max(best, tf)
    return round(best, 1)


def zipf_routing(tokens, experts, top_k, s, gen):
    """top_k distinct experts per token drawn with probability proportional to
    1 / rank^s over a random ranking of the experts; weights softmax(random logits) of
    the chosen, renormalised."""
    rank = torch.randperm(experts, generator=gen)
    p = 1.0 / (rank.double() + 1.0) ** s
    idx = torch.multinomial(p.expand(tokens, experts), top_k, replacement=False, generator=gen)
    w = torch.randn(tokens, top_k, generator=gen).softmax(-1)
    return w, idx


def bench_prefill(args, spec):
    import vaayu_amd.packed_expert_kernels as pk
    from vaayu_amd.synth import random_expert
    from oracle import oracle as O

    if pk.triton is None:
        raise SystemExit("vaayu_amd kernel library missing: run `python -m vaayu_amd.build`")
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    H, I, E, K, T = spec["hidden"], spec["inter"], spec["experts"], spec["top_k"], spec["tokens"]
    BITS, GS = 4, 128
    t0 = time.time()
    gen = torch.Generator(device=dev).manual_seed(1234)
    n_exp = E + (1 if spec["shared"] else 0)
    fmt = spec.get("fmt")
    if fmt is None:
        blobs = {e: random_expert(H, I, BITS, GS, generator=gen, device=dev, std=0.02,
                                  scale_dtype=torch.float16) for e in range(n_exp)}
    else:
        from vaayu_amd.block_formats import random_format_expert
        blobs = {e: random_format_expert(fmt, H, I, generator=gen, device=dev, std=0.02)
                 for e in range(n_exp)}
    torch.cuda.synchronize()
    per_expert = sum(t.numel() * t.element_size() for t in blobs[0]["flat"].values())
    log(f"{n_exp} experts resident: {n_exp * per_expert / 1e9:.2f} GB ({time.time() - t0:.1f} s)")
    cg = torch.Generator().manual_seed(99)
    x = torch.randn(T, H, generator=cg).to(torch.bfloat16).to(dev)
    if spec["routing"] == "zipf":
        w, eidx = zipf_routing(T, E, K, 1.1, cg)
    else:
        w, eidx = route(torch.randn(T, E, generator=cg), K)
    w = w.to(dev)
    geom = blobs[0]["geom"]
    sc = pk._SCALE_CODE[blobs[0]["flat"]["scale"].dtype]

    # calls of this layer: the routed experts, then (DeepSeek) the shared expert as a
    # one-slot call over every token with weight 1, added after the routed sum is cast
    calls = [(eidx, w, K)]
    if spec["shared"]:
        calls.append((torch.full((T, 1), E, dtype=torch.int64), torch.ones(T, 1, device=dev), 1))
    prepared = []
    for ei, wi, k in calls:
        plan = pk._prefill_plan(ei)
        tbl, rows, order, n_blocks = pk._prefill_tables(ei, plan, blobs, dev)
        work = tbl.vaayu_work.clone()                                  # off the table ring
        tbl, rows, order = tbl.clone(), rows.clone(), order.clone()
        h = torch.empty(T * k, I, dtype=torch.bfloat16, device=dev)
        y = torch.empty(T * k, H, dtype=torch.float32, device=dev)
        out = torch.empty(T, H, dtype=torch.float32, device=dev)
        prepared.append((tbl, rows, order, n_blocks, work, k, wi, h, y, out,
                         int(plan[1].numel())))
    torch.cuda.synchronize()

    def run_layer():
        for tbl, rows, order, n_blocks, work, k, wi, h, y, out, _live in prepared:
            pk._gate_up_g(x, tbl, rows, n_blocks, k, geom, sc, h=h, work=work)
            pk._down_g(h, tbl, rows, n_blocks, wi, geom, sc, y=y, work=work)
            pk._reduce(y, order, out, k)

    def run_stage(stage):
        for tbl, rows, order, n_blocks, work, k, wi, h, y, out, _live in prepared:
            if stage == "gate_up":
                pk._gate_up_g(x, tbl, rows, n_blocks, k, geom, sc, h=h, work=work)
            elif stage == "down":
                pk._down_g(h, tbl, rows, n_blocks, wi, geom, sc, y=y, work=work)
            else:
                pk._reduce(y, order, out, k)

    run_layer()
    torch.cuda.synchronize()

    def capture(fn):
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            fn()
        return graph

    calibrate_counters(dev)
    steps = max(1, args.steps // (5 if T >= 512 else 1))
    # each stage ten times in one graph: a graph of one short kernel replays at the host's
    # launch rate, not the GPU's (the stages are idempotent). Marked regions: 0 the layer,
    # 1 gate/up, 2 down, 3 reduce.
    rep = 10
    stages = [(st, capture(lambda st=st: [run_stage(st) for _ in range(rep)]))
              for st in ("gate_up", "down", "reduce")]
    graphs = [("layer", capture(run_layer))] + stages
    timed = timed_regions(graphs, steps, args.warmup, dev)
    ms = timed["layer"]
    stage_ms = {st: timed[st] / rep for st in ("gate_up", "down", "reduce")}
    peak_meas = measured_mfma_peak(dev)
    flops = 2 * T * K * 3 * H * I + (2 * T * 3 * H * I if spec["shared"] else 0)
    live = sum(p[-1] for p in prepared)
    wbytes = live * per_expert
    act_bytes = sum(T * H * 2 + 2 * T * k * I * 2 + T * k * H * 4 * 2 + T * H * 4
                    for *_r, k, _wi, _h, _y, _o, _l in prepared)
    tflops = flops / (ms * 1e-3) / 1e12
    gbs = (wbytes + act_bytes) / (ms * 1e-3) / 1e9
    log(f"layer {ms * 1000:.1f} us = {ms * 1000 / T:.3f} us/token; {tflops:.1f} TFLOP/s "
        f"({tflops / MFMA_PEAK_TFLOPS:.1%} of bf16 MFMA peak), {gbs:.0f} GB/s; stages "
        + ", ".join(f"{k} {v * 1000:.1f} us" for k, v in stage_ms.items()))

    # parity: a few tokens against the oracle (each token's output depends on its own
    # routing only)
    outs = [p[9] for p in prepared]            # each call's out
    n_chk = 2 if H * I > 4e6 else 8
    tok = torch.randperm(T, generator=cg)[:n_chk].tolist()
    cpu_blob = {}

    def cblob(e):
        if e not in cpu_blob:
            cpu_blob[e] = {"flat": {n: t.cpu() for n, t in blobs[e]["flat"].items()}, "geom": geom}
        return cpu_blob[e]

    worst = {"relL2": 0.0, "max_abs": 0.0}
    for t in tok:
        for (ei, wi, k), out in zip(calls, outs):
            ids = ei[t].tolist()
            order = sorted(range(k), key=lambda s: ids[s])
            ref = O.stock_decode(x[t:t + 1].cpu(), [(cblob(ids[s]), s) for s in order],
                                 wi[t].cpu())
            got = out[t:t + 1].cpu().numpy()
            worst["relL2"] = max(worst["relL2"], O.rel_l2(got, ref))
            worst["max_abs"] = max(worst["max_abs"], float(np.abs(got - ref).max()))
    parity = dict(worst, tokens_checked=n_chk, tolerance={"relL2": 5e-3, "max_abs": 2e-2},
                  within_tolerance=bool(worst["relL2"] <= 5e-3 and worst["max_abs"] <= 2e-2))
    log(f"parity vs oracle on {n_chk} tokens: {parity}")

    cpu = None
    if not args.no_cpu:
        sub = 2 if H * I > 4e6 else 8
        ei, wi, k = calls[0]
        cb = {e: cblob(e) for e in set(ei[:sub].reshape(-1).tolist())}
        o = torch.empty(sub, H)
        xs_c, ws_c = x[:sub].cpu(), wi[:sub].cpu()
        best, by_threads, info = cpu_leg(
            lambda i: O.stock_prefill_torch(xs_c, ei[:sub], ws_c, cb, o), args.cpu_seconds,
            1e6 / sub)
        value, n_calls, secs = by_threads[best]
        cpu = {"value": round(value, 1), "unit": "us/token per MoE layer", "cores": best,
               "kind": "port",
               "sample": f"{n_calls} stock prefill calls of {sub} tokens of this layer's routed "
                         f"experts on torch CPU at {best} threads (bf16 weights dequantized per "
                         f"call), {secs:.1f} s",
               "by_threads": {str(t): round(v[0], 1) for t, v in by_threads.items()},
               "host": info}
        log(f"cpu baseline {cpu}")

    bound = spec["bound"]
    roof = ({"bound": "mfma", "achieved": round(tflops, 1), "peak": MFMA_PEAK_TFLOPS,
             "unit": "TFLOP/s", "frac": round(tflops / MFMA_PEAK_TFLOPS, 4)}
            if bound == "mfma" else
            {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
             "frac": round(gbs / HBM_PEAK_GBS, 4)})
    roof.update({"traffic": traffic_from_profile(args.workload, PF_KERNELS, len(prepared)),
                 "kernels": "prefill_gate_up + prefill_down + prefill_reduce",
                 "flops_per_call": flops, "bytes_per_call": wbytes + act_bytes,
                 "measured_mfma_peak_tflops": peak_meas,
                 "frac_of_measured_mfma_peak": (round(tflops / peak_meas, 4)
                                                if peak_meas else None)})
    result = {
        "metric": METRIC, "value": round(ms * 1000 / T, 4), "unit": "us/token",
        "n_gpus": 1, "steps": steps, "warmup": args.warmup, "ms_per_step": round(ms, 4),
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": spec["name"] + ("" if fmt else ", int4 g128 fp16 scales"),
                   "hidden": H,
                   "experts": E, "inter": I, "top_k": K, "tokens": T,
                   "shared_expert": spec["shared"], "routing": spec["routing"],
                   "parallelism": "none (one GPU)"},
        "tokens_per_s_per_layer": round(T / (ms * 1e-3), 1),
        "stage_us": {k: round(v * 1000, 2) for k, v in stage_ms.items()},
        "roofline": roof, "parity": parity, "cpu_baseline": cpu,
    }
    print(json.dumps(result), flush=True)


def bench_fused3d(args, spec):
    """gpt-oss fused-3D MXFP4 experts: the two grouped GEMMs + the slot reduce over one
    call's prepared tables, recorded in one graph."""
    import vaayu_amd.packed_expert_kernels as pk
    from vaayu_amd.fused3d import Fused3DExperts
    from oracle import fused3d as F3
    from oracle import oracle as O

    if pk.triton is None:
        raise SystemExit("vaayu_amd kernel library missing: run `python -m vaayu_amd.build`")
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    H, I, E, K, T = spec["hidden"], spec["inter"], spec["experts"], spec["top_k"], spec["tokens"]
    gen = torch.Generator(device=dev).manual_seed(7)

    def codes(*shape):
        return torch.randint(0, 256, shape, generator=gen, device=dev, dtype=torch.uint8)

    def scales(*shape):                    # 2^-10 .. 2^-6 per 32 codes: O(1) activations
        return torch.randint(117, 122, shape, generator=gen, device=dev).to(torch.uint8)

    layer = dict(gu_blocks=codes(E, 2 * I, H // 32, 16), gu_scales=scales(E, 2 * I, H // 32),
                 gu_bias=torch.randn(E, 2 * I, generator=gen, device=dev) * 0.1,
                 dn_blocks=codes(E, H, I // 32, 16), dn_scales=scales(E, H, I // 32),
                 dn_bias=torch.randn(E, H, generator=gen, device=dev) * 0.1)
    mod = Fused3DExperts(layer["gu_blocks"], layer["gu_scales"], layer["gu_bias"],
                         layer["dn_blocks"], layer["dn_scales"], layer["dn_bias"])
    wbytes = sum(t.numel() * t.element_size() for t in layer.values())
    log(f"{E} experts resident: {wbytes / 1e9:.2f} GB")
    cg = torch.Generator().manual_seed(99)
    x = torch.randn(T, H, generator=cg).to(torch.bfloat16).to(dev)
    logits = torch.randn(T, E, generator=cg)
    top, eidx = torch.topk(logits, K, dim=-1)        # gpt-oss: top-k logits, softmax of them
    w = torch.softmax(top, dim=-1).to(dev)
    tables = tuple(t.clone() if hasattr(t, "clone") else t for t in mod.tables(eidx))
    xp = torch.zeros(T, mod.Hp, dtype=torch.bfloat16, device=dev)
    xp[:, :H] = x
    h = torch.zeros(T * K, mod.Ip, dtype=torch.bfloat16, device=dev)
    y = torch.empty(T * K, H, dtype=torch.float32, device=dev)
    out = torch.empty(T, H, dtype=torch.float32, device=dev)
    gammas = w.reshape(-1).float().contiguous()

    def run():
        mod.launch(xp, h, y, out, tables, gammas, K)

    run()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run()
    calibrate_counters(dev)
    steps = max(1, args.steps // 5)
    # timed in the sustained state, as the packed-expert prefill layers are
    ms = timed_regions([("layer", graph)], steps, args.warmup, dev)["layer"]
    flops = 2 * T * K * 3 * H * I
    tflops = flops / (ms * 1e-3) / 1e12
    log(f"layer {ms * 1000:.1f} us = {ms * 1000 / T:.3f} us/token; {tflops:.1f} TFLOP/s "
        f"({tflops / MFMA_PEAK_TFLOPS:.1%} of bf16 MFMA peak)")

    # parity: two tokens against the oracle
    got = out.to(torch.bfloat16).float().cpu().numpy()
    lay_cpu = {k_: v.cpu() for k_, v in layer.items()}
    worst = {"relL2": 0.0, "max_abs": 0.0}
    for t in (0, T - 1):
        ref = F3.fused3d_experts(x[t:t + 1].cpu(), eidx[t:t + 1], w[t:t + 1].cpu(), **lay_cpu)
        worst["relL2"] = max(worst["relL2"], O.rel_l2(got[t:t + 1], ref))
        worst["max_abs"] = max(worst["max_abs"], float(np.abs(got[t:t + 1] - ref).max()))
    parity = dict(worst, tokens_checked=2, tolerance={"relL2": 5e-3, "max_abs": 2e-2})
    log(f"parity vs oracle: {parity}")

    cpu = None
    if not args.no_cpu:
        wgu, wdn = {}, {}                       # the first 8 tokens' experts, dequantized
        for e in sorted(set(eidx[:8].reshape(-1).tolist())):
            wgu[e] = F3.dequant_fused3d(lay_cpu["gu_blocks"][e:e + 1],
                                        lay_cpu["gu_scales"][e:e + 1])[0]
            wdn[e] = F3.dequant_fused3d(lay_cpu["dn_blocks"][e:e + 1],
                                        lay_cpu["dn_scales"][e:e + 1])[0]
        n_tok, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < args.cpu_seconds:
            t = n_tok % 8
            F3.fused3d_experts(x[t:t + 1].cpu(), eidx[t:t + 1], w[t:t + 1].cpu(), **lay_cpu,
                               w_gu=wgu, w_dn=wdn)
            n_tok += 1
        cpu_s = time.perf_counter() - t0
        cpu = {"value": round(cpu_s * 1e6 / n_tok, 1), "unit": "us/token",
               "cores": 1, "kind": "port",
               "sample": f"{n_tok} tokens through the oracle (numpy float64, the 8 cycled "
                         f"tokens' experts dequantized beforehand), {cpu_s:.1f} s"}
        log(f"cpu baseline {cpu}")

    result = {
        "metric": "fused-3D MXFP4 MoE layer µs/token / MFMA util", "value": round(ms * 1000 / T, 4),
        "unit": "us/token", "n_gpus": 1, "steps": steps, "warmup": args.warmup,
        "ms_per_step": round(ms, 4), "higher_is_better": False, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": spec["name"], "hidden": H, "experts": E, "inter": I,
                   "top_k": K, "tokens": T, "parallelism": "none (one GPU)"},
        "roofline": {"bound": "mfma", "achieved": round(tflops, 1), "peak": MFMA_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(tflops / MFMA_PEAK_TFLOPS, 4),
                     "traffic": traffic_from_profile(args.workload, F3_KERNELS),
                     "kernels": "fused3d_gate_up + fused3d_down + prefill_reduce",
                     "flops_per_call": flops, "weight_bytes": wbytes},
        "parity": parity, "cpu_baseline": cpu,
    }
    print(json.dumps(result), flush=True)


def bench_gdn(args, spec):
    """A gated-delta mixer's decode step (conv update -> recurrent rule -> gated norm) for
    `mixers` x `copies` mixers with their own HBM-resident states, recorded in one graph."""
    import vaayu_amd.gated_delta_kernels as gdk
    from oracle import gated_delta as G
    from oracle import oracle as O

    if gdk.triton is None:
        raise SystemExit("vaayu_amd kernel library missing: run `python -m vaayu_amd.build`")
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    HV, HK, K, V, W = spec["HV"], spec["HK"], spec["K"], spec["V"], spec["W"]
    D = 2 * HK * K + HV * V
    n = spec["mixers"] * spec["copies"]
    gen = torch.Generator(device=dev).manual_seed(5)

    def rnd(*shape, dtype=torch.bfloat16, s=1.0):
        return (torch.randn(*shape, generator=gen, device=dev) * s).to(dtype)

    mix = [dict(conv_state=rnd(1, W, D).transpose(1, 2), conv_w=rnd(D, W, s=0.3),
                h=rnd(1, HV, K, V, dtype=torch.float32, s=0.1),
                norm_w=(1 + rnd(V, dtype=torch.float32, s=0.1)).bfloat16(),
                x=rnd(1, 1, D).transpose(1, 2), g=-torch.rand(1, 1, HV, device=dev),
                beta=torch.rand(1, 1, HV, device=dev).bfloat16(), z=rnd(1, 1, HV, V))
           for _ in range(n)]
    log(f"{n} mixers, states {n * (HV * K * V * 4 + D * W * 2) / 1e9:.2f} GB")

    def step(m):
        qkv = gdk.fused_conv_update(m["x"], m["conv_state"], m["conv_w"])[..., 0]
        q, k, v = torch.split(qkv, [HK * K, HK * K, HV * V], -1)
        q = q.reshape(1, 1, HK, K).repeat_interleave(HV // HK, 2)
        k = k.reshape(1, 1, HK, K).repeat_interleave(HV // HK, 2)
        o, m["ht"] = gdk.fused_recurrent_rule(q, k, v.reshape(1, 1, HV, V), m["g"], m["beta"],
                                              m["h"], True, True)
        m["out"] = gdk.fused_gated_norm(m["norm_w"], 1e-6, o, m["z"])

    def rule_only(m):
        gdk.fused_recurrent_rule(m["q"], m["k"], m["v"], m["g"], m["beta"], m["h"], True, True)

    for m in mix:                               # eager once; inputs for the rule-only graph
        saved = m["conv_state"].clone()
        step(m)
        m["conv_state"].copy_(saved)
        m["q"] = rnd(1, 1, HV, K)
        m["k"] = rnd(1, 1, HV, K)
        m["v"] = rnd(1, 1, HV, V)
    torch.cuda.synchronize()

    def capture(body):
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for m in mix:
                body(m)
        return graph

    def time_graph(graph):
        for _ in range(args.warmup):
            graph.replay()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(args.steps):
            graph.replay()
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b) / args.steps

    ms_step = time_graph(capture(step))
    ms_rule = time_graph(capture(rule_only))
    us_mixer, us_rule = ms_step * 1000 / n, ms_rule * 1000 / n
    rule_bytes = 2 * HV * K * V * 4 + 2 * HV * K * 2 + 2 * HV * V * 2 + HV * 8
    gbs = rule_bytes / (us_rule * 1e-6) / 1e9
    log(f"mixer step {us_mixer:.2f} us; rule kernel {us_rule:.2f} us per launch = {gbs:.0f} GB/s")

    # parity of one mixer's step against the oracle (conv -> rule -> norm, inputs from the
    # step itself so each stage is checked on what it was given)
    m = mix[0]
    st0 = m["conv_state"].clone()
    qkv = gdk.fused_conv_update(m["x"], m["conv_state"], m["conv_w"])
    ro, _rs = G.gdn_conv_update(m["x"], st0, m["conv_w"])
    q, k, v = torch.split(qkv[..., 0], [HK * K, HK * K, HV * V], -1)
    q = q.reshape(1, 1, HK, K).repeat_interleave(HV // HK, 2)
    k = k.reshape(1, 1, HK, K).repeat_interleave(HV // HK, 2)
    o, ht = gdk.fused_recurrent_rule(q, k, v.reshape(1, 1, HV, V), m["g"], m["beta"], m["h"],
                                     True, True)
    r_o, r_h = G.gdn_rule(q, k, v.reshape(1, 1, HV, V), m["g"], m["beta"], m["h"])
    out = gdk.fused_gated_norm(m["norm_w"], 1e-6, o, m["z"])
    r_n = G.gdn_gated_norm(o, m["z"], m["norm_w"], 1e-6, "bf16", True)
    parity = {"conv_relL2": O.rel_l2(O.to_np(qkv), ro), "rule_relL2": O.rel_l2(O.to_np(o), r_o),
              "state_relL2": O.rel_l2(O.to_np(ht), r_h),
              "norm_relL2": O.rel_l2(O.to_np(out), r_n)}
    log(f"parity vs oracle: {parity}")

    cpu = None
    if not args.no_cpu:
        xs = [{k_: O.to_np(t) for k_, t in mix[i].items() if isinstance(t, torch.Tensor)}
              for i in range(4)]
        n_calls, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < args.cpu_seconds:
            c = xs[n_calls % 4]
            qkv_c, _ = G.gdn_conv_update(c["x"], c["conv_state"], c["conv_w"])
            qc, kc, vc = np.split(qkv_c[..., 0], [HK * K, 2 * HK * K], -1)
            qc = np.repeat(qc.reshape(1, 1, HK, K), HV // HK, 2)
            kc = np.repeat(kc.reshape(1, 1, HK, K), HV // HK, 2)
            oc, _ = G.gdn_rule(qc, kc, vc.reshape(1, 1, HV, V), c["g"], c["beta"], c["h"])
            G.gdn_gated_norm(oc, c["z"], c["norm_w"], 1e-6)
            n_calls += 1
        cpu_s = time.perf_counter() - t0
        cpu = {"value": round(cpu_s * 1e6 / n_calls, 1), "unit": "us per mixer decode step",
               "cores": 1, "kind": "port",
               "sample": f"{n_calls} mixer steps through the oracle (numpy, float64), "
                         f"{cpu_s:.1f} s"}
        log(f"cpu baseline {cpu}")

    result = {
        "metric": "gated-delta mixer decode µs/token (conv + rule + norm)",
        "value": round(us_mixer, 3), "unit": "us/token per mixer", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_step, 4),
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "fp32",
        "data": "synthetic",
        "config": {"workload": spec["name"] + f", {n} HBM-resident mixer states per step",
                   "num_v_heads": HV, "num_k_heads": HK, "head_k_dim": K, "head_v_dim": V,
                   "conv_width": W, "conv_dim": D, "mixers": n, "parallelism": "none (one GPU)"},
        "roofline": {"bound": "hbm", "kernel": "gdn_rule_kernel", "achieved": round(gbs, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                     "traffic": None, "bytes_per_launch": rule_bytes,
                     "us_per_launch": round(us_rule, 3)},
        "parity": parity, "cpu_baseline": cpu,
    }
    print(json.dumps(result), flush=True)


def main():
    args = parse()
    if args.summarize:
        print(summarize(args.summarize))
        return
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path "
              "(expert-parallel sharding is a design note only). Run with --gpus 1.",
              file=sys.stderr)
        sys.exit(2)
    spec = WORKLOADS[args.workload]
    if spec is not None and spec.get("fused3d"):
        bench_fused3d(args, spec)
        return
    if spec is not None and spec.get("gdn"):
        bench_gdn(args, spec)
        return
    if spec is not None and "tokens" in spec:
        bench_prefill(args, spec)
        return
    fmt = spec["fmt"] if spec is not None else "int4"

    import vaayu_amd.packed_expert_kernels as pk
    from vaayu_amd import _lib
    from vaayu_amd.synth import clone_blob, random_expert
    from vaayu_amd.block_formats import random_format_expert

    if pk.triton is None:
        raise SystemExit("vaayu_amd kernel library missing: run `python -m vaayu_amd.build`")
    lib = _lib.load()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    shape = dict(hidden=2048, inter=768, experts=128, top_k=8, layers=48, shared=False)
    if spec is not None:
        shape.update(spec.get("decode_shape", {}))
    H, E, I, K, BITS, GS = (shape["hidden"], shape["experts"], shape["inter"], shape["top_k"],
                            4, 128)
    L = args.layers or shape["layers"]
    SHARED = shape["shared"]
    n_exp = E + (1 if SHARED else 0)        # the shared expert is blob E of a layer

    # ── experts: `distinct` random layers, the rest byte copies at fresh addresses ─────
    t0 = time.time()
    gen = torch.Generator(device=dev).manual_seed(1234)
    if fmt == "int4":
        make = lambda: random_expert(H, I, BITS, GS, generator=gen, device=dev, std=0.02,
                                     scale_dtype=torch.float16)
    else:
        make = lambda: random_format_expert(fmt, H, I, generator=gen, device=dev, std=0.02)
    base = [[make() for _ in range(n_exp)] for _ in range(min(args.distinct, L))]
    layers = [base[l] if l < len(base) else [clone_blob(b) for b in base[l % len(base)]]
              for l in range(L)]
    torch.cuda.synchronize()
    per_expert = sum(t.numel() * t.element_size() for t in layers[0][0]["flat"].values())
    log(f"{L} layers x {n_exp} experts resident: {L * n_exp * per_expert / 1e9:.2f} GB "
        f"({time.time() - t0:.1f} s)")
    geom = layers[0][0]["geom"]
    sc = pk._SCALE_CODE[layers[0][0]["flat"]["scale"].dtype]
    g = _lib.geom_struct(geom)

    # ── one token's routing per layer, its table and buffers ────────────────────────────
    cg = torch.Generator().manual_seed(99)
    x = torch.randn(1, H, generator=cg).to(torch.bfloat16).to(dev)
    tables, rws, hs, outs, routed = [], [], [], [], []
    for l in range(L):
        logits = torch.randn(1, E, generator=cg).to(torch.bfloat16)
        w, idx = route(logits, K)
        ids = idx[0].tolist()
        order = sorted(range(K), key=lambda s: ids[s])
        pairs = [(layers[l][ids[s]], s) for s in order]
        routed.append((ids, order, w))
        tables.append(torch.tensor(pk._table_values(pairs), dtype=torch.int64, device=dev))
        rws.append(w.to(dev))
        hs.append(torch.empty(K, I, dtype=torch.bfloat16, device=dev))
        outs.append(torch.empty(1, H, dtype=torch.float32, device=dev))
    # DeepSeek's always-on shared expert: a one-slot call of weight 1 per layer (the
    # engine adds its output after the routed sum is cast to bf16; that add is not timed)
    sh = []
    if SHARED:
        one = torch.ones(1, 1, dtype=torch.float32, device=dev)
        for l in range(L):
            sh.append((torch.tensor(pk._table_values([(layers[l][E], 0)]), dtype=torch.int64,
                                    device=dev),
                       torch.empty(1, I, dtype=torch.bfloat16, device=dev),
                       torch.empty(1, H, dtype=torch.float32, device=dev)))

    def gate_up(l, stream):
        rc = lib.vaayu_decode_gate_up(x.data_ptr(), tables[l].data_ptr(), hs[l].data_ptr(),
                                      K, g, 0, sc, stream)
        if SHARED and rc == 0:
            rc = lib.vaayu_decode_gate_up(x.data_ptr(), sh[l][0].data_ptr(), sh[l][1].data_ptr(),
                                          1, g, 0, sc, stream)
        return rc

    def down(l, stream):
        rc = lib.vaayu_decode_down(hs[l].data_ptr(), tables[l].data_ptr(), rws[l].data_ptr(),
                                   2, outs[l].data_ptr(), K, g, 0, sc, 0, stream)
        if SHARED and rc == 0:
            rc = lib.vaayu_decode_down(sh[l][1].data_ptr(), sh[l][0].data_ptr(), one.data_ptr(),
                                       2, sh[l][2].data_ptr(), 1, g, 0, sc, 0, stream)
        return rc

    def capture(body):
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            st = torch.cuda.current_stream().cuda_stream
            for l in range(L):
                body(l, st)
        return graph

    def check(rc):
        _lib.check(rc, "bench launch")

    calibrate_counters(dev)

    # the one-launch layer (vaayu_decode_fused): its own h and zeroed sync buffer per layer
    # (and per shared-expert call)
    fused = None
    words = lib.vaayu_decode_fused_sync_words(K, g, 0, sc)
    if words > 0 and args.one_launch:
        syncs = [torch.zeros(words, dtype=torch.int32, device=dev) for _ in range(L)]
        fhs = [torch.empty(K, I, dtype=torch.bfloat16, device=dev) for _ in range(L)]
        if SHARED:
            swords = lib.vaayu_decode_fused_sync_words(1, g, 0, sc)
            ssyncs = [torch.zeros(swords, dtype=torch.int32, device=dev) for _ in range(L)]

        def fused(l, stream):
            rc = lib.vaayu_decode_fused(x.data_ptr(), tables[l].data_ptr(), rws[l].data_ptr(), 2,
                                        outs[l].data_ptr(), fhs[l].data_ptr(), syncs[l].data_ptr(),
                                        K, g, 0, sc, 0, 0, stream)
            if SHARED and rc == 0:
                rc = lib.vaayu_decode_fused(x.data_ptr(), sh[l][0].data_ptr(), one.data_ptr(), 2,
                                            sh[l][2].data_ptr(), sh[l][1].data_ptr(),
                                            ssyncs[l].data_ptr(), 1, g, 0, sc, 0, 0, stream)
            return rc

    # eager once (validates every launch), then graphs
    st = torch.cuda.current_stream().cuda_stream
    for l in range(L):
        check(gate_up(l, st))
        check(down(l, st))
    torch.cuda.synchronize()
    two_launch_out = [o.clone() for o in outs]
    if fused is not None:
        for l in range(L):
            check(fused(l, st))
        torch.cuda.synchronize()
        same = all(torch.equal(a, b) for a, b in zip(outs, two_launch_out))
        log(f"one-launch layer equals the two-launch layer bitwise: {same}")
        if not same:
            raise SystemExit("the one-launch decode disagrees with the two-launch decode")
    full = capture(lambda l, s: (gate_up(l, s), down(l, s)))
    gu_only = capture(gate_up)
    dn_only = capture(down)

    # ── routed: the router product, the routing and the pair table on the GPU too ───────
    # (the headline workload carries it as extra fields; `qwen3-decode-routed` makes it the
    # line's value)
    routed_layer = None
    as_value = spec is not None and spec.get("routed")
    if as_value or (spec is None and not args.no_routed):
        from vaayu_amd.device_routing import ResidentExperts, router_logits
        rg = torch.Generator(device=dev).manual_seed(7)
        rxs = [ResidentExperts(layers[l]) for l in range(L)]
        # the model's gate weight [experts, hidden]; its product runs as router_logits
        w_rt = [(torch.randn(E, H, generator=rg, device=dev) * 0.05).to(torch.bfloat16)
                for _ in range(L)]
        r_logits = [torch.empty(1, E, dtype=torch.bfloat16, device=dev) for _ in range(L)]
        r_bufs = [rx.buffers(K, x.dtype) for rx in rxs]
        r_outs = [torch.empty(1, H, dtype=torch.float32, device=dev) for _ in range(L)]

        def routed_layer(l, _stream):
            router_logits(x, w_rt[l], out=r_logits[l])
            rxs[l].decode(x, r_logits[l], K, r_outs[l], bufs=r_bufs[l])

        for l in range(L):
            routed_layer(l, st)
        torch.cuda.synchronize()
        routed_graph = capture(routed_layer)

    # layer 0 launched L times in one graph: its 19.5 MB stay in the 256 MB MALL, so this is
    # the warm figure beside the line's cold one (every layer's weights from HBM)
    warm_graph = capture(lambda _l, s: (gate_up(0, s), down(0, s)))

    # warm every graph, then time each in its own marked region (region 0: the layer,
    # 1: gate/up alone, 2: down alone, 3: layer 0 repeated (weights in MALL), 4: the routed
    # layer)
    graphs = [("layer", full), ("gate_up", gu_only), ("down", dn_only), ("warm", warm_graph)]
    if routed_layer is not None:
        graphs.append(("routed", routed_graph))
    if fused is not None:                    # the last region: the one-launch layer
        graphs.append(("fused", capture(fused)))
    ms = timed_regions(graphs, args.steps, args.warmup, dev)
    ms_two = ms["layer"]
    # the same layers launched eagerly, no graph: what a caller without graphs pays per layer
    # (host launch cost included)
    eager = {}
    for name, body in (("two_launch", lambda l: (gate_up(l, st), down(l, st))),
                       ("one_launch", fused)):
        if body is None:
            continue
        for l in range(L):
            body(l) if name == "two_launch" else body(l, st)
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(args.steps):
            for l in range(L):
                body(l) if name == "two_launch" else body(l, st)
        b.record()
        torch.cuda.synchronize()
        eager[name] = round(a.elapsed_time(b) * 1000.0 / (args.steps * L), 3)
    log(f"eager (no graph) us per layer: {eager}")
    if fused is not None:
        ms["layer"] = ms["fused"]
    ms_step, ms_gu, ms_dn = ms["layer"], ms["gate_up"], ms["down"]
    us_tok_layer = ms_step * 1000.0 / L
    log(f"step {ms_step:.3f} ms = {us_tok_layer:.2f} us/token/layer "
        f"({'one launch' if fused is not None else 'two launches'}); two-launch layer "
        f"{ms_two * 1000 / L:.2f} us, gate_up {ms_gu * 1000 / L:.2f} us, down "
        f"{ms_dn * 1000 / L:.2f} us per layer")
    routed_extra = None
    if routed_layer is not None:
        ms_routed = ms["routed"]
        # ResidentExperts.decode runs the two-launch expert kernels after the routing
        routed_extra = {"us_per_token_per_layer": round(ms_routed * 1000.0 / L, 3),
                        "expert_kernels_us_per_layer": round(ms_two * 1000.0 / L, 3),
                        "router_and_routing_us_per_layer":
                            round((ms_routed - ms_two) * 1000.0 / L, 3)}
        if as_value:
            ms_step, us_tok_layer = ms_routed, ms_routed * 1000.0 / L
        log(f"routed layer {ms_routed * 1000.0 / L:.2f} us/token/layer {routed_extra}")

    # algorithmic bytes (distinct routed experts' codes + scales + activations)
    from vaayu_amd.block_formats import geom_format
    _f, bits, group, brows = geom_format(geom)
    sc_el = layers[0][0]["flat"]["scale"].element_size()

    def role_bytes(rows, cols):             # codes + scales of one role
        return rows * cols * bits // 8 + (rows // brows) * (cols // group) * sc_el

    NX = K + (1 if SHARED else 0)             # expert blobs one token reads per layer
    NL = 2 if SHARED else 1                   # launches of each kernel per layer
    gu_bytes = NX * 2 * role_bytes(I, H) + H * 2 * (2 if SHARED else 1) + NX * I * 2
    dn_bytes = NX * role_bytes(H, I) + NX * I * 2 + H * 4 * (2 if SHARED else 1)
    gu_gbs = gu_bytes / (ms_gu * 1e-3 / L) / 1e9
    dn_gbs = dn_bytes / (ms_dn * 1e-3 / L) / 1e9
    layer_gbs = (gu_bytes + dn_bytes) / (us_tok_layer * 1e-6) / 1e9
    if routed_extra is not None:
        routed_extra["hbm_gbs"] = round((gu_bytes + dn_bytes)
                                        / (routed_extra["us_per_token_per_layer"] * 1e-6) / 1e9, 1)
        routed_extra["frac_of_8tbs"] = round(routed_extra["hbm_gbs"] / HBM_PEAK_GBS, 4)

    # ── parity of layer 0 against the CPU oracle (the checker) ──────────────────────────
    from oracle import oracle as O
    ids, order, w = routed[0]
    cpu_pairs = [({"flat": {n: t.cpu() for n, t in layers[0][ids[s]]["flat"].items()},
                   "geom": geom}, s) for s in order]
    # the numpy restatement takes minutes per call at Mixtral's expert size; its torch
    # port of the stock loop (pinned against it in the oracle's tests) checks those shapes
    big = H * I > 4e6

    def stock(xc, pairs, wc):
        if not big:
            return O.stock_decode(xc, pairs, wc)
        o = torch.empty(1, H)
        O.stock_decode_torch(xc, pairs, wc, o)
        return o.numpy()

    ref = stock(x.cpu(), cpu_pairs, w)
    got = outs[0].cpu().numpy()
    parity = {"relL2": O.rel_l2(got, ref), "max_abs": float(np.abs(got - ref).max()),
              "tolerance": {"relL2": 5e-3, "max_abs": 2e-2}}
    parity["within_tolerance"] = bool(parity["relL2"] <= 5e-3 and parity["max_abs"] <= 2e-2)
    if SHARED:
        sref = stock(x.cpu(), [({"flat": {n: t.cpu() for n, t in
                                                   layers[0][E]["flat"].items()},
                                          "geom": geom}, 0)], torch.ones(1, 1))
        sgot = sh[0][2].cpu().numpy()
        parity["shared"] = {"relL2": O.rel_l2(sgot, sref),
                            "max_abs": float(np.abs(sgot - sref).max())}
    if routed_layer is not None:             # layer 0 as routed on the GPU
        want_w, want_ids = O.route_softmax_topk(r_logits[0].cpu().float(), K)
        got_ids, got_w = r_bufs[0].ids.cpu().numpy(), r_bufs[0].weights.cpu()
        e = got_ids[0].tolist()
        pairs = [({"flat": {n: t.cpu() for n, t in layers[0][e[s]]["flat"].items()},
                   "geom": geom}, s) for s in sorted(range(K), key=e.__getitem__)]
        ref = O.stock_decode(x.cpu(), pairs, got_w)
        got = r_outs[0].cpu().numpy()
        parity["routed"] = {
            "ids_equal": bool(np.array_equal(got_ids, want_ids)),
            "weights_max_rel": float(np.abs(got_w.numpy() - want_w).max() / np.abs(want_w).max()),
            "relL2": O.rel_l2(got, ref), "max_abs": float(np.abs(got - ref).max())}
    log(f"parity layer 0 vs oracle: {parity}")

    # ── CPU baseline: the stock loop on torch CPU, bounded sample ───────────────────────
    cpu = None
    if not args.no_cpu:
        xc = x.cpu()
        samples = []
        for l in range(min(L, 8)):
            ids, order, w = routed[l]
            samples.append(([({"flat": {n: t.cpu() for n, t in layers[l][ids[s]]["flat"].items()},
                               "geom": geom}, s) for s in order], w))
        out = torch.empty(1, H)
        s_pair = ([({"flat": {n: t.cpu() for n, t in layers[0][E]["flat"].items()},
                     "geom": geom}, 0)] if SHARED else None)
        s_out, s_w = torch.empty(1, H), torch.ones(1, 1)

        def one_call(i):
            pairs, w = samples[i % len(samples)]
            O.stock_decode_torch(xc, pairs, w, out)
            if s_pair is not None:
                O.stock_decode_torch(xc, s_pair, s_w, s_out)

        best, by_threads, info = cpu_leg(one_call, args.cpu_seconds, 1e6)
        value, n_calls, secs = by_threads[best]
        cpu = {"value": round(value, 1), "unit": "us/token per MoE layer", "cores": best,
               "kind": "port",
               "sample": f"{n_calls} one-token decodes of the same layer shape (8 layers' "
                         f"routed experts{' and the shared expert' if SHARED else ''} copied "
                         f"to host, cycled), torch CPU bf16 stock loop at {best} threads, "
                         f"{secs:.1f} s",
               "by_threads": {str(t): round(v[0], 1) for t, v in by_threads.items()},
               "host": info}
        log(f"cpu baseline {cpu}")

    # a layer with the shared expert runs each kernel twice (routed, shared): its figures
    # are per layer, i.e. per pair of launches
    per, unit = ("", "launch") if NL == 1 else ("routed_and_shared_", "layer")
    gu_traffic = traffic_from_profile(args.workload, (GU_KERNEL,), NL)
    dn_traffic = traffic_from_profile(args.workload, (DN_KERNEL,), NL)
    result = {
        "metric": METRIC, "value": round(us_tok_layer, 3), "unit": "us/token",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4), "higher_is_better": False, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": (spec["name"] if spec is not None else
                                "Qwen3-30B-A3B-shape MoE layer decode, 1 token, int4 g128 fp16 "
                                "scales") + f", {L} HBM-resident layers per step",
                   "hidden": H, "experts": E, "inter": I, "top_k": K, "layers": L,
                   "shared_expert": SHARED, "tokens": 1, "parallelism": "none (one GPU)"},
        "tokens_per_s_per_layer": round(1e6 / us_tok_layer, 1),
        # the layer: both kernels' algorithmic bytes over the layer's time (graph replays of
        # all layers, HIP events); each kernel beside it, timed alone the same way
        "roofline": {"bound": "hbm",
                     "kernel": ("decode layer, one launch (fused_decode_kernel)"
                                if fused is not None else
                                f"decode layer ({GU_KERNEL} + {DN_KERNEL})"),
                     "two_launch_us_per_layer": round(ms_two * 1000.0 / L, 3),
                     # the same launches over layer 0 only, its weights resident in the MALL
                     "warm_in_mall_us_per_layer": round(ms["warm"] * 1000.0 / L, 3),
                     "eager_us_per_layer": eager,
                     "achieved": round(layer_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(layer_gbs / HBM_PEAK_GBS, 4),
                     "traffic": (gu_traffic + dn_traffic
                                 if gu_traffic is not None and dn_traffic is not None else None),
                     "bytes_per_layer": gu_bytes + dn_bytes,
                     "us_per_layer": round(us_tok_layer, 3),
                     "kernels": {
                         "gate_up": {"name": GU_KERNEL, "achieved": round(gu_gbs, 1),
                                     "frac": round(gu_gbs / HBM_PEAK_GBS, 4),
                                     "traffic": gu_traffic, per + "bytes_per_" + unit: gu_bytes,
                                     per + "us_per_" + unit: round(ms_gu * 1000 / L, 3)},
                         "down": {"name": DN_KERNEL, "achieved": round(dn_gbs, 1),
                                  "frac": round(dn_gbs / HBM_PEAK_GBS, 4),
                                  "traffic": dn_traffic, per + "bytes_per_" + unit: dn_bytes,
                                  per + "us_per_" + unit: round(ms_dn * 1000 / L, 3)}}},
        "parity": parity,
        "cpu_baseline": cpu,
    }
    if routed_extra is not None:
        result["routed_layer"] = routed_extra
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
