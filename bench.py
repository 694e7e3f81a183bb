#!/usr/bin/env python3
"""Benchmark of the routed-expert MoE hot path on one MI355X.

Headline (a "step"): one full MoE layer at decode, M=1 token, D=4096, I=2048:
router (bf16 gate [256, 4096] + fp32 bias, sqrt(softplus), top-6) -> 6 routed
FP4 experts (packed e2m1 + E8M0 per 32) -> + one FP8 e4m3 shared expert, one
launch of moe_layer_kernel, synthetic seeded weights generated on the device.
Steps rotate over --layers distinct layers (each with its own 256 experts,
router and input token), so consecutive reuses of the same weights are
>= 860 MB apart and the 256 MB Infinity Cache cannot serve them.  One HIP
graph holds a rotation and one the remainder, so exactly --steps launches
run; HIP events around every replay give per-launch samples (median and
spread reported).  The layer kernel's status word is checked after timing.

The same line carries the other workloads under "configs":
  0  one routed FP4 expert, M=1 (hsmoe_moe_decode with one id)
  2  MTP verify T=3: the layer at M=3 + lm_head [129280, 4096] + greedy
     acceptance of seeded drafts (argmax-equal with p = 0.7)
  3  prefill, M=512, Zipf(1.1) routing (hsmoe_moe_prefill)
  4  the 43-layer decode stack with MTP verify, tok/s
each with its own roofline and cpu_baseline: the reference's CPU PyTorch route
restated op for op in torch (oracle/cpu_ref.py, per-call dequant), on the
host's cores, on a bounded sample of the same workload and the same weights
(copied from the device), median of >= 5 runs.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

import __graft_entry__  # noqa: E402

D, I, E, K, VOCAB = 4096, 2048, 256, 6, 129280
EXPERT_BYTES = 3 * I * D // 2 + 3 * I * D // 32          # 13,369,344
GATE_UP_BYTES = 2 * (I * D // 2 + I * D // 32)            # w1 + w3 + scales of one routed expert
DOWN_BYTES = D * I // 2 + D * I // 32                      # w2 + scales
SHARED_GATE_UP = 2 * I * D + 2 * (I // 128) * (D // 128) * 4
SHARED_DOWN = D * I + (D // 128) * (I // 128) * 4
SHARED_BYTES = SHARED_GATE_UP + SHARED_DOWN
ROUTER_BYTES = E * D * 2 + E * 4
EXPERT_WEIGHT_BYTES = K * EXPERT_BYTES + SHARED_BYTES       # routed + shared expert weights
LAYER_IO_BYTES = EXPERT_WEIGHT_BYTES + ROUTER_BYTES + 2 * D * 2             # + router weights, x in, out
LM_HEAD_BYTES = VOCAB * D * 2
HBM_PEAK_GBS = 8000.0
METRIC = "MoE layer FP4 expert GB/s (% HBM peak) at M=1/M=3; MTP-verify decode tok/s"
DTYPE = "fp4-e2m1 weights, bf16 MFMA, fp32 accumulate"


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None, help="default 800 (headline) / 64 (stack) / 50 (prefill)")
    ap.add_argument("--warmup", type=int, default=None, help="default 40 (headline) / 4 (stack) / 5 (prefill)")
    ap.add_argument("--workload", choices=("all", "layer", "expert", "verify", "stack", "prefill"), default="all",
                    help="all: the headline layer line with configs 0, 2, 3, 4 under 'configs'; "
                         "layer: the headline only; expert / verify / stack / prefill: config 0 / 2 / 4 / 3 as "
                         "the line")
    ap.add_argument("--configs", default="0,2,3,4", help="sub-workloads of --workload all")
    ap.add_argument("--stack-layers", type=int, default=43)
    ap.add_argument("--stack-steps", type=int, default=64,
                    help="decode steps of config 4 under --workload all (the config's 64-step decode loop)")
    ap.add_argument("--layers", type=int, default=8, help="distinct layers rotated through (MALL defeat)")
    ap.add_argument("--seed", type=int, default=1234)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=8.0, help="CPU time budget per config")
    ap.add_argument("--no-chain-check", action="store_true",
                    help="config 4: skip the greedy-chain check and the expert-byte count after timing (profiling "
                         "runs: then every decode-step kernel after the build belongs to the warm-up or timed steps)")
    ap.add_argument("--calib-copy", action="store_true",
                    help="finish with 3 copies of a 256 MiB buffer (known bytes) to scale PMC byte counters")
    ap.add_argument("--path", choices=("fused", "staged"), default="fused",
                    help="fused: one persistent launch per layer (hsmoe_moe_layer_decode); "
                         "staged: router, gate/up and down launches")
    args = ap.parse_args()
    if args.steps is None:
        args.steps = {"stack": 64, "prefill": 50}.get(args.workload, 800)
    if args.warmup is None:
        args.warmup = {"stack": 4, "prefill": 5}.get(args.workload, 40)
    if args.steps < 1:
        ap.error("--steps must be >= 1")
    return args


# ---------------------------------------------------------------- timing helpers

def spread(samples_us: list[float]) -> dict:
    s = sorted(samples_us)
    q = lambda p: s[min(len(s) - 1, int(round(p * (len(s) - 1))))]
    return {"n": len(s), "median_us": round(statistics.median(s), 3), "p10_us": round(q(0.1), 3),
            "p90_us": round(q(0.9), 3), "min_us": round(s[0], 3), "max_us": round(s[-1], 3)}


def capture(torch, stream, fn):
    """fn run once eagerly on `stream` (creates workspaces), then captured."""
    with torch.cuda.stream(stream):
        fn()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            fn()
    return g


def timed_launches(torch, stream, launch, n_rot: int, steps: int, warmup: int):
    """Exactly `steps` calls launch(j % n_rot), j = 0..steps-1: a graph of one
    rotation replayed steps // n_rot times, then a graph of the first
    steps % n_rot calls.  -> (total ms, per-call samples in us: one per replay,
    the replay's time over its calls)."""
    full = capture(torch, stream, lambda: [launch(j) for j in range(n_rot)])
    rem = steps % n_rot
    part = capture(torch, stream, lambda: [launch(j) for j in range(rem)]) if rem else None
    for _ in range(max(1, warmup // n_rot)):
        full.replay()
    torch.cuda.synchronize()
    plan = [(full, n_rot)] * (steps // n_rot) + ([(part, rem)] if rem else [])
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(len(plan) + 1)]
    with torch.cuda.stream(stream):
        evs[0].record(stream)
        for j, (g, _) in enumerate(plan):
            g.replay()
            evs[j + 1].record(stream)
    torch.cuda.synchronize()
    samples = [evs[j].elapsed_time(evs[j + 1]) * 1e3 / n for j, (_, n) in enumerate(plan)]
    return evs[0].elapsed_time(evs[-1]), samples


def roofline(kernel: str, nbytes: int, us: float, traffic=None, **extra) -> dict:
    ach = nbytes / (us * 1e-6) / 1e9
    return {"bound": "hbm", "kernel": kernel, "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": traffic, "algorithmic_bytes_per_launch": nbytes,
            "avg_launch_us": round(us, 3), **extra}


def read_ceiling(torch, buf, stream) -> dict:
    """The HBM read rate a single pass over resident weights reaches on this
    device: hsmoe_xor_checksum (a read-only stream, 8 loads of 16 bytes in
    flight per lane, one workgroup per CU) over distinct slices of `buf` in
    rotation, far beyond the 256 MB Infinity Cache.  The median time per call
    over 1 GiB slices and over 2 GiB slices is fitted as t = a + bytes / rate,
    so that the rate leaves out a call's fixed cost (its one-workgroup fold
    launch and the gap before it, ~3% of a 1 GiB call)."""
    from home_seek_amd import ops
    gib = 1 << 30

    def per_call(size):
        n = min(8, buf.numel() // size)
        if n < 1:
            return None, 0
        slices = [buf[j * size:(j + 1) * size] for j in range(n)]
        outs = [torch.empty(16, dtype=torch.uint8, device=buf.device) for _ in range(n)]
        _, samples = timed_launches(torch, stream, lambda j: ops.xor_checksum(slices[j], outs[j]), n, max(4 * n, 8), n)
        return statistics.median(samples), n

    t1, n1 = per_call(gib)
    t2, n2 = per_call(2 * gib)
    if t1 is None or t2 is None or t2 <= t1:
        return None
    gbs = gib / ((t2 - t1) * 1e-6) / 1e9
    return {"gbs": round(gbs, 1), "us_per_gib": round(t2 - t1, 2), "call_overhead_us": round(2 * t1 - t2, 2),
            "us_per_call_1gib": round(t1, 2), "us_per_call_2gib": round(t2, 2), "slices": [n1, n2],
            "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
            "method": "hsmoe_xor_checksum over distinct 1 GiB and 2 GiB slices of the store, each size rotated in a HIP "
                      "graph; median time per call fitted as t = a + bytes / rate (a: the fold launch and the gap "
                      "before it)"}


def with_ceiling(roof: dict | None, ceiling: dict | None) -> dict | None:
    """Adds the fraction of the measured read ceiling to a roofline (and its nested ones)."""
    if roof is None or not ceiling:
        return roof
    roof["read_ceiling_gbs"] = ceiling["gbs"]
    roof["frac_of_read_ceiling"] = round(roof["achieved"] / ceiling["gbs"], 4)
    for v in roof.values():
        if isinstance(v, dict) and "achieved" in v:
            with_ceiling(v, ceiling)
    return roof


def pmc_traffic(name: str):
    """HBM bytes per launch from a committed rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE summary."""
    p = ROOT / "profiles" / name
    return json.loads(p.read_text()).get("traffic_bytes_per_launch") if p.exists() else None


# ---------------------------------------------------------------- CPU baseline helpers

def cpu_setup():
    """Threads for the CPU legs: this process's CPU share (affinity), capped by
    OMP_NUM_THREADS when set; the host CPU model and physical core count (what
    lscpu reports) from /proc/cpuinfo, read without starting a child process."""
    import torch
    n = len(os.sched_getaffinity(0))
    env = os.environ.get("OMP_NUM_THREADS")
    if env and env.isdigit() and int(env) > 0:
        n = min(n, int(env))
    torch.set_num_threads(n)
    info = {"threads": n}
    try:
        model, cores, phys = None, set(), None
        for ln in Path("/proc/cpuinfo").read_text().splitlines():
            k, _, v = ln.partition(":")
            k, v = k.strip(), v.strip()
            if k == "model name" and model is None:
                model = v
            elif k == "physical id":
                phys = v
            elif k == "core id":
                cores.add((phys, v))
        info["cpu_model"] = model
        if cores:
            info["host_physical_cores"] = len(cores)
    except OSError:
        pass
    return info


def cpu_median(fn, budget_s: float, min_runs: int = 5):
    """One warm-up, then runs until >= min_runs and >= budget_s -> (median s, runs)."""
    fn()
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < min_runs or time.perf_counter() < t_end:
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
        if len(times) >= 200:
            break
    return statistics.median(times), len(times)


def cpu_line(value, unit, info, sample, **extra):
    return {"value": value, "unit": unit, "cores": info["threads"], "kind": "port",
            "cpu_model": info.get("cpu_model"), "host_physical_cores": info.get("host_physical_cores"),
            "sample": sample, **extra}


def rel_l2(a, b) -> float:
    a, b = a.float().reshape(-1), b.float().reshape(-1)
    return float((a - b).norm() / b.norm().clamp(min=1e-30))


# ---------------------------------------------------------------- the headline: config 1

class LayerBench:
    """L layers of config 1 on the device: store, routers, inputs."""

    def __init__(self, torch, args):
        from home_seek_amd import expert_store, synthetic
        self.torch, self.args = torch, args
        self.dev = torch.device("cuda:0")
        L = self.L = args.layers
        self.store = expert_store.HbmExpertStore(L, E, D, I, self.dev, with_shared=True)
        self.store.fill_synthetic(args.seed)
        self.routers = [synthetic.router_weights(args.seed, l, E, D, self.dev) for l in range(L)]
        self.tables = [self.store.table(l) for l in range(L)]
        self.shareds = [self.store.shared_entry(l) for l in range(L)]
        self.stream = torch.cuda.Stream()
        torch.cuda.synchronize()

    def cpu_loader(self, layer):
        """load_expert(eid) for the CPU route: the device store's checkpoint-format
        tensors copied to the host once (the reference's pinned FP4 tier)."""
        cache = {}

        def load(eid):
            if eid not in cache:
                w1, s1, w3, s3, w2, s2 = self.store.expert_views(layer, eid)
                cache[eid] = tuple(t.view(self.torch.uint8).cpu() for t in (w1, s1, w3, s3, w2, s2))
            return cache[eid]
        return load

    def cpu_shared(self, layer):
        return tuple(t.view(self.torch.uint8).cpu() if t.dtype != self.torch.float32 else t.cpu()
                     for t in self.store.shared_views(layer))


def run_headline(torch, args, lb: LayerBench, cpu_info):
    from home_seek_amd import ops, synthetic
    L, dev = lb.L, lb.dev
    xs = [synthetic.hidden(args.seed, 1000 + l, 1, D, dev) for l in range(L)]
    idx_buf = [torch.empty(1, K, dtype=torch.int64, device=dev) for _ in range(L)]
    w_buf = [torch.empty(1, K, dtype=torch.float32, device=dev) for _ in range(L)]
    outs = [torch.empty(1, D, dtype=torch.bfloat16, device=dev) for _ in range(L)]
    fused = args.path == "fused"

    def step(l):
        if fused:
            ops.moe_layer_decode(xs[l], lb.routers[l][0], lb.routers[l][1], lb.tables[l], ops.SCALE_E8M0,
                                 lb.shareds[l], I, K, 1.5, 10.0, out_bf16=outs[l], idx_out=idx_buf[l], w_out=w_buf[l])
            return
        idx, w = ops.router_topk(xs[l], lb.routers[l][0], lb.routers[l][1], K, 1.5, out=(idx_buf[l], w_buf[l]))
        ops.moe_decode(xs[l], idx, w, lb.tables[l], ops.SCALE_E8M0, lb.shareds[l], 10.0, out_bf16=outs[l], d=D, i=I)

    for j in range(max(1, args.warmup)):
        step(j % L)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    total_ms, samples = timed_launches(torch, lb.stream, step, L, args.steps, args.warmup)
    wall = time.perf_counter() - t0
    # after the timed region: the same rotation replayed 100 times, a larger
    # sample of the per-launch time (reported beside the timed one, not used for value)
    _, long_samples = timed_launches(torch, lb.stream, step, L, 100 * L, L)
    ops.check_moe_layer_status(dev)
    sp = spread(samples)
    us = sp["median_us"]
    routed_gbs = K * EXPERT_BYTES / (us * 1e-6) / 1e9
    if fused:
        roof = roofline("moe_layer_kernel (router + 6 routed FP4 + FP8 shared expert, one launch)", LAYER_IO_BYTES, us,
                        pmc_traffic("moe_layer_kernel_m1_pmc.json"))
    else:
        roof = roofline("router + moe_gate_up_kernel + moe_down_kernel (staged)", LAYER_IO_BYTES, us)

    cpu = None
    if not args.no_cpu_baseline:
        from oracle import cpu_ref
        n_s = min(L, 4)
        cases = []
        for l in range(n_s):
            gate = lb.routers[l][0].cpu()
            bias = lb.routers[l][1].cpu()
            cases.append((xs[l].cpu(), gate, bias, lb.cpu_loader(l), lb.cpu_shared(l)))
        outs_cpu = {}

        def one(c=[0]):
            l = c[0] % n_s
            c[0] += 1
            x, gate, bias, load, sh = cases[l]
            idx, w = cpu_ref.router(x, gate, bias, K, 1.5)
            outs_cpu[l] = (idx, cpu_ref.moe_ffn(x, idx, w, load, sh))
        for l in range(n_s):  # loads every selected expert to the host before timing
            one([l])
        t_med, runs = cpu_median(one, args.cpu_seconds)
        ids_match = all(torch.equal(outs_cpu[l][0], idx_buf[l].cpu()) for l in range(n_s))
        cpu = cpu_line(round(K * EXPERT_BYTES / t_med / 1e9, 4), "GB/s", cpu_info,
                       f"{runs} MoE layers at M=1 over {n_s} layers (router + _forward_legacy with per-call FP4 "
                       f"dequant of 6 experts + FP8 shared expert, torch bf16 on the CPU); median "
                       f"{1e3 * t_med:.1f} ms/layer",
                       ms_per_step=round(1e3 * t_med, 3), ids_match_gpu=ids_match,
                       rel_l2_vs_gpu=round(max(rel_l2(outs_cpu[l][1], outs[l].cpu()) for l in range(n_s)), 5))

    line = {
        "metric": METRIC,
        "value": round(routed_gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(us * 1e-3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": DTYPE,
        "data": "synthetic (seeded on device; normals are Irwin-Hall(4) approximations, |z| <= 3.46)",
        "config": {
            "workload": "config 1: one MoE layer at decode M=1: router top-6 of 256 + 6 FP4 experts + FP8 shared "
                        "expert, D=4096 I=2048",
            "global_batch": 1,
            "seq_len": 1,
            "parallelism": "none (1 GPU)",
            "layers_rotated": L,
        },
        "timing": {**sp, "mean_us": round(total_ms * 1e3 / args.steps, 3), "timed_ms": round(total_ms, 3),
                   "method": "HIP events around each graph replay (rotation of --layers launches, remainder graph "
                             "for --steps % --layers); value and ms_per_step from the median"},
        "timing_check": {**spread(long_samples), "launches": 100 * L,
                         "method": "after the timed region, 100 replays of the same rotation graph (not used for "
                                   "value)"},
        "layer_status": 0,
        "pct_hbm_peak": round(100.0 * routed_gbs / HBM_PEAK_GBS, 2),
        "expert_gbs": round(EXPERT_WEIGHT_BYTES / (us * 1e-6) / 1e9, 1),
        "full_layer_gbs": round(LAYER_IO_BYTES / (us * 1e-6) / 1e9, 1),
        "path": args.path,
        "wall_s_timed": round(wall, 3),
        "roofline": roof,
        "cpu_baseline": cpu,
    }
    return line


# ---------------------------------------------------------------- config 0

def run_config0(torch, args, lb: LayerBench, cpu_info):
    """One routed FP4 expert at M=1: the layer kernel with one given id and no
    shared expert (hsmoe_moe_layer_decode_routed), 32 (layer, expert) pairs
    rotated (428 MB)."""
    from home_seek_amd import ops, synthetic
    dev = lb.dev
    pairs = [(l, (37 * j + 11 * l) % E) for l in range(lb.L) for j in range(32 // lb.L)]
    xs = [synthetic.hidden(args.seed, 4000 + j, 1, D, dev) for j in range(len(pairs))]
    idx = [torch.tensor([[e]], dtype=torch.int64, device=dev) for _, e in pairs]
    outs = [torch.empty(1, D, dtype=torch.bfloat16, device=dev) for _ in pairs]

    def launch(j):
        l, _ = pairs[j]
        ops.moe_layer_decode_routed(xs[j], idx[j], lb.tables[l], ops.SCALE_E8M0, None, I, weight_all=1.0, top_k=1,
                                    out_bf16=outs[j])

    steps = 8 * len(pairs)
    total_ms, samples = timed_launches(torch, lb.stream, launch, len(pairs), steps, len(pairs))
    ops.check_moe_layer_status(dev)
    sp = spread(samples)
    us = sp["median_us"]
    gbs = EXPERT_BYTES / (us * 1e-6) / 1e9
    res = {"workload": "config 0: one routed FP4 expert (dequant + SwiGLU FFN), M=1, D=4096 I=2048",
           "value": round(gbs, 1), "unit": "GB/s", "steps": steps, "warmup": len(pairs),
           "ms_per_step": round(us * 1e-3, 5),
           "timing": sp, "pct_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 2),
           "roofline": roofline("moe_layer_kernel with one given id (one launch)", EXPERT_BYTES + 2 * D * 2, us,
                                pmc_traffic("expert_m1_pmc.json")),
           "cpu_baseline": None}
    if not args.no_cpu_baseline:
        from oracle import cpu_ref
        l, e = pairs[0]
        w1, s1, w3, s3, w2, s2 = lb.cpu_loader(l)(e)
        x = xs[0].cpu()
        box = {}

        def run():
            box["y"] = cpu_ref.ffn_pt(x, cpu_ref.dequant_fp4(w1, s1), cpu_ref.dequant_fp4(w3, s3),
                                      cpu_ref.dequant_fp4(w2, s2))
        t_med, runs = cpu_median(run, args.cpu_seconds / 2)
        res["cpu_baseline"] = cpu_line(round(EXPERT_BYTES / t_med / 1e9, 4), "GB/s", cpu_info,
                                       f"{runs} single-expert FFNs at M=1 (per-call FP4 dequant of w1/w3/w2 + "
                                       f"fused_expert_ffn_pt, torch bf16); median {1e3 * t_med:.2f} ms",
                                       ms_per_step=round(1e3 * t_med, 3),
                                       rel_l2_vs_gpu=round(rel_l2(box["y"], outs[0].cpu()), 5))
    return res


# ---------------------------------------------------------------- config 2

def run_config2(torch, args, lb: LayerBench, cpu_info):
    """MTP verify T=3: the layer at M=3 (per-token routing) + lm_head + acceptance
    of seeded drafts (each draft argmax-equal with p = 0.7, else uniform)."""
    import numpy as np
    from home_seek_amd import ops, synthetic
    L, dev = lb.L, lb.dev
    xs3 = [synthetic.hidden(args.seed, 2000 + l, 3, D, dev) for l in range(L)]
    idx3 = [torch.empty(3, K, dtype=torch.int64, device=dev) for _ in range(L)]
    w3 = [torch.empty(3, K, dtype=torch.float32, device=dev) for _ in range(L)]
    outs3 = [torch.empty(3, D, dtype=torch.bfloat16, device=dev) for _ in range(L)]
    lm = synthetic.normal_bf16(args.seed, synthetic.tag(synthetic.KIND_LM_HEAD), (VOCAB, D), 0.0, 0.02, dev)
    hs = [synthetic.hidden(args.seed, 3000 + l, 3, D, dev) for l in range(L)]
    rng = np.random.Generator(np.random.PCG64(args.seed + 2))
    ids, results = [], [torch.empty(2, dtype=torch.int64, device=dev) for _ in range(L)]
    for l in range(L):
        _, pred, _ = ops.lm_head_accept(hs[l], lm, torch.zeros(3, dtype=torch.int64, device=dev), want_logits=False)
        p = pred.cpu().tolist()
        drafts = [p[j] if rng.random() < 0.7 else int(rng.integers(VOCAB)) for j in range(2)]
        ids.append(torch.tensor([int(rng.integers(VOCAB))] + drafts, dtype=torch.int64, device=dev))

    def layer(l):
        ops.moe_layer_decode(xs3[l], lb.routers[l][0], lb.routers[l][1], lb.tables[l], ops.SCALE_E8M0, lb.shareds[l],
                             I, K, 1.5, 10.0, out_bf16=outs3[l], idx_out=idx3[l], w_out=w3[l])

    def head(l):
        _, _, r = ops.lm_head_accept(hs[l], lm, ids[l], want_logits=False)
        results[l].copy_(r)

    n = 8 * L
    ms_l, s_l = timed_launches(torch, lb.stream, layer, L, n, L)
    ms_h, s_h = timed_launches(torch, lb.stream, head, L, 2 * L, L)
    ms_s, s_s = timed_launches(torch, lb.stream, lambda l: (layer(l), head(l)), L, n, L)
    ops.check_moe_layer_status(dev)
    uniq = [len(set(idx3[l].reshape(-1).tolist())) for l in range(L)]
    acc = [int(results[l][0]) for l in range(L)]
    sl, sh, ss = spread(s_l), spread(s_h), spread(s_s)
    u_avg = sum(uniq) / L
    layer_bytes = int(u_avg * EXPERT_BYTES) + SHARED_BYTES + ROUTER_BYTES + 2 * 3 * D * 2
    gbs = u_avg * EXPERT_BYTES / (sl["median_us"] * 1e-6) / 1e9
    res = {"workload": "config 2: MTP verify T=3: MoE layer at M=3 (per-token top-6) + lm_head [129280, 4096] + "
                       "greedy acceptance of 2 seeded drafts (argmax-equal with p = 0.7)",
           "value": round(gbs, 1), "unit": "GB/s (routed-expert bytes of the M=3 layer)",
           "ms_per_step": round(ss["median_us"] * 1e-3, 5), "steps": n,
           "layer_us": sl, "lm_head_accept_us": sh, "step_us": ss,
           "unique_experts_avg": u_avg, "accepted": acc, "pct_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 2),
           "roofline": roofline("moe_layer_kernel at M=3", layer_bytes, sl["median_us"],
                                pmc_traffic("moe_layer_kernel_m3_pmc.json"),
                                lm_head=roofline("lm_head_mfma_kernel + accept (T=3)", LM_HEAD_BYTES, sh["median_us"])),
           "cpu_baseline": None}
    if not args.no_cpu_baseline:
        from oracle import cpu_ref
        n_s = min(L, 2)
        lm_c = lm.cpu()
        cases = [(xs3[l].cpu(), lb.routers[l][0].cpu(), lb.routers[l][1].cpu(), lb.cpu_loader(l), lb.cpu_shared(l),
                  hs[l].cpu(), ids[l].cpu().tolist()) for l in range(n_s)]
        got = {}

        def one(c=[0]):
            l = c[0] % n_s
            c[0] += 1
            x, gate, bias, load, shr, h, cid = cases[l]
            idx, w = cpu_ref.router(x, gate, bias, K, 1.5)
            y = cpu_ref.moe_ffn(x, idx, w, load, shr)
            _, n_acc, row = cpu_ref.lm_head_accept(h, lm_c, cid)
            got[l] = (idx, y, n_acc)
        for l in range(n_s):
            one([l])
        t_med, runs = cpu_median(one, args.cpu_seconds)
        res["cpu_baseline"] = cpu_line(
            round(u_avg * EXPERT_BYTES / t_med / 1e9, 4), "GB/s", cpu_info,
            f"{runs} verify steps over {n_s} layers (router + _forward_legacy union of the 3 tokens' experts with "
            f"per-call dequant + shared expert + lm_head matmul [3, 4096] x [4096, 129280] + argmax acceptance, "
            f"torch bf16); median {1e3 * t_med:.1f} ms/step",
            ms_per_step=round(1e3 * t_med, 3),
            ids_match_gpu=all(torch.equal(got[l][0], idx3[l].cpu()) for l in range(n_s)),
            accepted_match_gpu=all(got[l][2] == acc[l] for l in range(n_s)),
            rel_l2_vs_gpu=round(max(rel_l2(got[l][1], outs3[l].cpu()) for l in range(n_s)), 5))
    del lm
    return res


# ---------------------------------------------------------------- config 3

def run_prefill(torch, args, cpu_info, steps=None, warmup=None, ceiling=None):
    """Prefill MoE layer: M=512 tokens, 256 FP4 experts, top-6 with Zipf(1.1)
    popularity drawn without replacement per token, routed experts only (the
    shared expert timed separately); one hsmoe_moe_prefill call (group,
    gate/up, down, combine) per step, captured in a HIP graph."""
    import numpy as np
    from home_seek_amd import expert_store, ops, synthetic

    dev = torch.device("cuda:0")
    steps = args.steps if steps is None else steps
    warmup = args.warmup if warmup is None else warmup
    m = 512
    store = expert_store.HbmExpertStore(1, E, D, I, dev, with_shared=True)
    store.fill_synthetic(args.seed)
    x = synthetic.hidden(args.seed, 5000, m, D, dev)
    idx_h, w_h = synthetic.zipf_routing(args.seed, m, E, K)
    idx, w = torch.as_tensor(idx_h, device=dev), torch.as_tensor(w_h, device=dev)
    counts = [int(c) for c in np.bincount(idx_h.reshape(-1), minlength=E)]
    touched = sum(1 for c in counts if c)
    table, shared = store.table(0), store.shared_entry(0)
    out = torch.empty(m, D, dtype=torch.bfloat16, device=dev)
    stream = torch.cuda.Stream()
    torch.cuda.synchronize()
    fn = lambda sh: (lambda j: ops.moe_prefill(x, idx, w, table, ops.SCALE_E8M0, sh, 10.0, out_bf16=out, i=I))
    ms, samples = timed_launches(torch, stream, fn(None), 1, steps, warmup)
    ms_sh, s_sh = timed_launches(torch, stream, fn(shared), 1, max(5, steps // 5), 2)
    sp, sp_sh = spread(samples), spread(s_sh)
    us = sp["median_us"]
    routed_bytes = touched * EXPERT_BYTES
    io_bytes = m * D * 2 * 2 + m * K * 12
    flops = 3 * 2 * D * I * m * K
    gbs = routed_bytes / (us * 1e-6) / 1e9
    tflops = flops / (us * 1e-6) / 1e12
    res = {"workload": f"config 3: prefill MoE layer, M={m} tokens, D={D} I={I}, {E} FP4 experts top-{K}, Zipf(1.1) "
                       "popularity (grouped gate/up + down GEMM), routed experts only",
           "value": round(gbs, 1), "unit": "GB/s", "steps": steps, "warmup": warmup,
           "ms_per_step": round(us * 1e-3, 5), "timing": sp,
           "touched_experts": touched, "max_tokens_per_expert": max(counts),
           "pct_hbm_peak": round(100.0 * gbs / HBM_PEAK_GBS, 2), "mfma_tflops": round(tflops, 2),
           "pct_bf16_mfma_peak": round(100.0 * tflops / 2500.0, 3),
           "with_shared_expert": {"ms": round(sp_sh["median_us"] * 1e-3, 5),
                                  "gbs": round((routed_bytes + SHARED_BYTES) / (sp_sh["median_us"] * 1e-6) / 1e9, 1)},
           "roofline": roofline("hsmoe_moe_prefill call (group + gate/up + down + combine launches)",
                                routed_bytes + io_bytes, us, pmc_traffic("prefill_m512_pmc.json")),
           "cpu_baseline": None}
    if ceiling is None:
        ceiling = read_ceiling(torch, store.buf, stream)
        res["read_ceiling"] = ceiling
    with_ceiling(res["roofline"], ceiling)
    if not args.no_cpu_baseline:
        from oracle import cpu_ref
        union = [e for e in range(E) if counts[e]][:8]
        views = {e: tuple(t.view(torch.uint8).cpu() for t in store.expert_views(0, e)) for e in union}
        xc = x.cpu()
        keep = np.isin(idx_h, union)
        idx_c = torch.from_numpy(np.where(keep, idx_h, -1))
        w_c = torch.from_numpy(w_h)
        t_med, runs = cpu_median(lambda: cpu_ref.forward_legacy(xc, idx_c, w_c, views.get), args.cpu_seconds, 3)
        res["cpu_baseline"] = cpu_line(
            round(len(union) * EXPERT_BYTES / t_med / 1e9, 4), "GB/s", cpu_info,
            f"_forward_legacy at M=512 as written (a dense union GEMM: every token against every union expert, "
            f"~43x the needed FLOPs at the full union) over {len(union)} of the {touched} touched experts "
            f"(ids of the others set to -1), per-call dequant, torch bf16; {runs} runs, median {t_med:.2f} s; "
            f"GB/s counts the sampled experts' bytes",
            ms_per_step=round(1e3 * t_med, 2))
    del store
    return res


# ---------------------------------------------------------------- config 4

def run_stack(torch, args, cpu_info, steps=None, warmup=None, ceiling=None):
    """The MoE-only decode stack: all layers' experts resident, greedy decode with
    MTP verify, one step = M=1 forward + 2 MTP drafts + T=3 verify, captured as
    one HIP graph and replayed; tok/s over the timed steps."""
    from home_seek_amd import ops, stack
    from home_seek_amd.engine import GreedyDecoder

    dev = torch.device("cuda:0")
    steps = args.steps if steps is None else steps
    warmup = args.warmup if warmup is None else warmup
    n_layers = args.stack_layers
    t0 = time.perf_counter()
    eng = stack.build_stack(args.seed, n_layers=n_layers, n_experts=E, d=D, i=I, vocab=VOCAB, top_k=K, n_hash=3,
                            device=dev, log=lambda m: print(f"[stack] {m} ({time.perf_counter() - t0:.1f} s)",
                                                            file=sys.stderr, flush=True))
    torch.cuda.synchronize()
    t_build = time.perf_counter() - t0
    print(f"[stack] {n_layers} layers + MTP block built in {t_build:.1f} s "
          f"({eng.store.buf.numel() / 1e9:.1f} GB expert store)", file=sys.stderr, flush=True)
    dec = GreedyDecoder(eng, max(steps, warmup, 1))
    first = 1 + args.seed % (VOCAB - 1)
    dec.reset(first)
    dec.run(warmup)
    torch.cuda.synchronize()
    start_tok = int(dec.cur.item())
    dec.reset()
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    t1 = time.perf_counter()
    evs[0].record()
    for j in range(steps):
        dec.run(1)
        evs[j + 1].record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t1
    ms = evs[0].elapsed_time(evs[-1])
    samples = [evs[j].elapsed_time(evs[j + 1]) * 1e3 for j in range(steps)]
    tokens, accs = dec.result()  # raises when a layer launch's cross-workgroup wait gave up
    rows = dec.rows[:steps].cpu().tolist()
    print(f"[stack] {steps} steps in {ms:.1f} ms, {len(tokens)} tokens", file=sys.stderr, flush=True)

    if args.no_chain_check:
        sp = spread(samples)
        return {"workload": f"config 4: {n_layers}-layer MoE-only decode stack (no chain check: profiling run)",
                "value": round(len(tokens) / (ms * 1e-3), 2), "unit": "tok/s", "steps": steps, "warmup": warmup,
                "ms_per_step": round(ms / steps, 4), "timing": sp, "tokens": len(tokens),
                "decode_steps_run": steps + warmup + 1, "build_s": round(t_build, 1), "cpu_baseline": None}
    # Every token's routing is a function of the token alone (no attention), so
    # the M=1 forward of each token gives the experts the verify reads.
    routing = {}

    def route_of(tok):
        if tok not in routing:
            sets = []
            h = eng._embed(torch.tensor([[tok]], device=dev))
            for l in range(n_layers):
                h, _ = eng._forward_layer(h, eng._get_layer_weights(l), l, torch.tensor([[tok]], device=dev))
                sets.append(set(eng._last_routed_idx.reshape(-1).tolist()))
            routing[tok] = (sets, h)
        return routing[tok]

    def next_of(tok):
        _, h = route_of(tok)
        _, pred, _ = ops.lm_head_accept(eng._final_hidden(h), eng.lm_head, None, want_logits=False)
        return int(pred.item())

    chain, t = [], start_tok
    for _ in range(len(tokens)):
        t = next_of(t)
        chain.append(t)
    verify_experts = 0
    for r in rows:  # verify [A, d0, d1]: the union of the three tokens' experts per layer
        ver = [route_of(x)[0] for x in r[:3]]
        for l in range(n_layers):
            verify_experts += len(ver[0][l] | ver[1][l] | ver[2][l])
    # layer launches at M=1 (main forward + two MTP drafts) and at M=3 (verify), lm_head passes
    m1_bytes = steps * ((n_layers + 2) * (K * EXPERT_BYTES + SHARED_BYTES) + (n_layers - 3 + 2) * ROUTER_BYTES)
    m3_bytes = verify_experts * EXPERT_BYTES + steps * (n_layers * SHARED_BYTES + (n_layers - 3) * ROUTER_BYTES)
    lm_bytes = steps * 4 * LM_HEAD_BYTES                                 # main, 2 drafts, verify
    total = m1_bytes + m3_bytes + lm_bytes
    # HBM traffic per step from the kernels' measured traffic / algorithmic ratios (rocprofv3 FETCH_SIZE +
    # WRITE_SIZE of the same kernels: the M=1 and M=3 layer launches, the lm_head)
    ratio = {}
    for key, name in (("m1", "moe_layer_kernel_m1_pmc.json"), ("m3", "moe_layer_kernel_m3_pmc.json"),
                      ("lm", "lm_head_t3_pmc.json")):
        pth = ROOT / "profiles" / name
        if pth.exists():
            d = json.loads(pth.read_text())
            ratio[key] = d["traffic_bytes_per_launch"] / d["algorithmic_bytes_per_launch"]
    traffic = (int((m1_bytes * ratio["m1"] + m3_bytes * ratio["m3"] + lm_bytes * ratio["lm"]) / steps)
               if len(ratio) == 3 else None)
    sp = spread(samples)
    res = {"workload": f"config 4: {n_layers}-layer MoE-only decode stack (attention replaced by a seeded residual), "
                       f"{E} FP4 experts + FP8 shared per layer, D={D} I={I}, vocab {VOCAB}; per step M=1 forward + "
                       "2 MTP drafts + T=3 verify, greedy, one HIP graph per step",
           "value": round(len(tokens) / (ms * 1e-3), 2), "unit": "tok/s", "steps": steps, "warmup": warmup,
           "ms_per_step": round(ms / steps, 4), "timing": sp, "tokens": len(tokens),
           "accepted_per_step": round(sum(accs) / len(accs), 4),
           "tokens_per_step": round(len(tokens) / steps, 4), "greedy_chain_match": tokens == chain,
           "layer_status": 0,
           "roofline": roofline("whole decode step (all kernels of one graph replay)", total // steps, ms / steps * 1e3,
                                traffic, lm_head_bytes_per_step=lm_bytes // steps,
                                traffic_method="per kernel class: algorithmic bytes x the traffic / algorithmic "
                                               "ratio rocprofv3 measured for that kernel (profiles/"
                                               "moe_layer_kernel_m1_pmc.json, moe_layer_kernel_m3_pmc.json, "
                                               "lm_head_t3_pmc.json)"),
           "build_s": round(t_build, 1), "wall_s_timed": round(wall, 3), "cpu_baseline": None}
    if ceiling is None:
        ceiling = read_ceiling(torch, eng.store.buf, torch.cuda.Stream())
        res["read_ceiling"] = ceiling
    with_ceiling(res["roofline"], ceiling)
    if not args.no_cpu_baseline:
        res["cpu_baseline"] = stack_cpu_baseline(torch, eng, rows[0], n_layers, res["tokens_per_step"], args, cpu_info)
    del eng, dec
    return res


def stack_cpu_baseline(torch, eng, row, n_layers, tokens_per_step, args, cpu_info):
    """One decode step of the stack on the CPU route, sampled over 4 of the
    layers and extrapolated to all of them: per sampled layer the M=1 pass and
    the T=3 verify pass (norm + residual, router or hash ids, _forward_legacy
    with per-call dequant, shared expert); plus the MTP block twice and the 4
    lm_head passes.  Weights are the device's, copied to the host."""
    from oracle import cpu_ref
    sample = [0, 3, n_layers // 2, n_layers - 1]
    a, drafts = row[0], row[1:3]
    lm = eng.lm_head.cpu()
    hn_w = eng.norm_weight.cpu()

    emb = {t: eng.embed[t].cpu() for t in [a] + drafts}

    def layer_pass(l, ids, lw, load, shr):
        def run():
            h = torch.stack([emb[t] for t in ids])
            h = h + lw["attn.residual"]
            hn = cpu_ref.rms_norm(h, lw["ffn_norm.weight"])
            if "ffn.gate.tid2eid" in lw:
                idx = lw["ffn.gate.tid2eid"][torch.tensor(ids)]
                w = torch.full(idx.shape, 1.0 / K)
            else:
                idx, w = cpu_ref.router(hn, lw["ffn.gate.weight"], lw["ffn.gate.bias"], K, 1.5)
            return h + cpu_ref.moe_ffn(hn, idx, w, load, shr)
        return run

    def host_layer(l, lw_dev):
        lw = {k: (v.cpu() if hasattr(v, "cpu") else v) for k, v in lw_dev.items() if k != "layer_idx"}
        cache = {}

        def load(eid):
            if eid not in cache:
                cache[eid] = tuple(t.view(torch.uint8).cpu() for t in eng.store.expert_views(l, eid))
            return cache[eid]
        shr = tuple(t.view(torch.uint8).cpu() if t.dtype != torch.float32 else t.cpu()
                    for t in eng.store.shared_views(l))
        return lw, load, shr

    t_layers = {}
    budget = args.cpu_seconds / (2 * len(sample) + 2)
    for l in sample:
        lw, load, shr = host_layer(l, eng._get_layer_weights(l))
        t1, _ = cpu_median(layer_pass(l, [a], lw, load, shr), budget, 3)
        t3, _ = cpu_median(layer_pass(l, [a] + drafts, lw, load, shr), budget, 3)
        t_layers[l] = t1 + t3
    mw = eng._mtp_weights
    lw_m, load_m, shr_m = host_layer(n_layers, mw["layer"])
    t_mtp, _ = cpu_median(layer_pass(n_layers, [a], lw_m, load_m, shr_m), budget, 3)
    h1 = torch.zeros(1, D, dtype=torch.bfloat16)
    h3 = torch.zeros(3, D, dtype=torch.bfloat16)
    t_lm1, _ = cpu_median(lambda: cpu_ref.lm_head_accept(cpu_ref.rms_norm(h1, hn_w), lm, [a]), budget, 3)
    t_lm3, _ = cpu_median(lambda: cpu_ref.lm_head_accept(cpu_ref.rms_norm(h3, hn_w), lm, [a] + drafts), budget, 3)
    hashed = [l for l in sample if l < 3]
    routed = [l for l in sample if l >= 3]
    t_hash = sum(t_layers[l] for l in hashed) / len(hashed)
    t_routed = sum(t_layers[l] for l in routed) / len(routed)
    step_s = 3 * t_hash + (n_layers - 3) * t_routed + 2 * t_mtp + 3 * t_lm1 + t_lm3
    return cpu_line(round(tokens_per_step / step_s, 5), "tok/s", cpu_info,
                    f"one decode step sampled over layers {sample} (M=1 + T=3 verify passes each, median of >= 3), "
                    f"the MTP layer and the lm_head at M=1 and T=3, extrapolated to {n_layers} layers + 2 drafts + "
                    f"4 lm_head passes: {step_s:.2f} s/step; tokens/step taken from the GPU run",
                    ms_per_step=round(1e3 * step_s, 1))


# ---------------------------------------------------------------- main

def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build has no multi-GPU path "
              "(expert-parallel sharding is described in DESIGN.md, not run). Use --gpus 1.", file=sys.stderr)
        sys.exit(2)
    import torch
    __graft_entry__.package()
    torch.cuda.set_device(0)
    cpu_info = cpu_setup() if not args.no_cpu_baseline else {"threads": 0}
    if args.workload in ("verify", "stack", "prefill", "expert"):
        if args.workload in ("verify", "expert"):
            lb = LayerBench(torch, args)
            res = (run_config2 if args.workload == "verify" else run_config0)(torch, args, lb, cpu_info)
            res.setdefault("warmup", args.layers)
            res["read_ceiling"] = read_ceiling(torch, lb.store.buf, lb.stream)
            with_ceiling(res["roofline"], res["read_ceiling"])
        else:
            fn = run_stack if args.workload == "stack" else run_prefill
            res = fn(torch, args, cpu_info)
        wl = res.pop("workload")
        line = {"metric": METRIC, "value": res.pop("value"), "unit": res.pop("unit"), "n_gpus": 1,
                "steps": res.pop("steps"), "warmup": res.pop("warmup"), "ms_per_step": res.pop("ms_per_step"),
                "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": DTYPE,
                "data": "synthetic (seeded on device)",
                "config": {"workload": wl, "global_batch": {"prefill": 512, "verify": 3}.get(args.workload, 1),
                           "seq_len": {"prefill": 512, "verify": 3}.get(args.workload, 1),
                           "parallelism": "none (1 GPU)"}}
        line.update(res)
        calib_copy(torch, args)
        print(json.dumps(line))
        return

    lb = LayerBench(torch, args)
    line = run_headline(torch, args, lb, cpu_info)
    ceiling = read_ceiling(torch, lb.store.buf, lb.stream)
    line["read_ceiling"] = ceiling
    with_ceiling(line["roofline"], ceiling)
    if args.workload == "all":
        want = [c.strip() for c in args.configs.split(",") if c.strip()]
        configs = {}
        for c in want:
            print(f"[bench] config {c}", file=sys.stderr, flush=True)
            if c == "0":
                configs["0"] = run_config0(torch, args, lb, cpu_info)
            elif c == "2":
                configs["2"] = run_config2(torch, args, lb, cpu_info)
        if "3" in want or "4" in want:
            del lb
            torch.cuda.empty_cache()
        if "3" in want:
            print("[bench] config 3", file=sys.stderr, flush=True)
            configs["3"] = run_prefill(torch, args, cpu_info, steps=50, warmup=5)
            torch.cuda.empty_cache()
        if "4" in want:
            print("[bench] config 4", file=sys.stderr, flush=True)
            configs["4"] = run_stack(torch, args, cpu_info, steps=args.stack_steps, warmup=2)
        for res in configs.values():
            with_ceiling(res.get("roofline"), ceiling)
        line["configs"] = configs
    calib_copy(torch, args)
    print(json.dumps(line))


def calib_copy(torch, args):
    """--calib-copy: three copies of a 256 MiB buffer (known bytes) that scale
    the PMC byte counters of the same run."""
    if args.calib_copy:
        src = torch.ones(256 << 20, dtype=torch.uint8, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()


if __name__ == "__main__":
    main()
