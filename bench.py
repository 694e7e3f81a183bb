#!/usr/bin/env python3
"""Benchmark of the routed-expert MoE hot path on one MI355X.

Workload (a "step"): one full MoE layer at decode, M=1 token, D=4096, I=2048:
router (bf16 gate [256, 4096] + fp32 bias, sqrt(softplus), top-6) -> 6 routed
FP4 experts (packed e2m1 + E8M0 per 32) -> + one FP8 e4m3 shared expert, with
synthetic seeded weights generated on the device.  Steps rotate over
--layers distinct layers (each with its own 256 experts, router and input
token), so consecutive reuses of the same weights are >= 860 MB apart and
the 256 MB Infinity Cache cannot serve them.  The step sequence is captured
in a HIP graph; the timed region replays it.

metric/value: routed-expert bytes (6 x 13,369,344 B) / step time, GB/s.
roofline: the dominant kernel (stage 1: gate/up of the routed + shared
experts) -- algorithmic bytes per launch / its average duration, timed live
with HIP events over a graph of back-to-back launches.
cpu_baseline: the CPU oracle (a restatement of the reference's PyTorch path:
per-call FP4/FP8 dequant + fp32 FFN + router) on one thread, on a bounded
sample of the same workload.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

import __graft_entry__  # noqa: E402

D, I, E, K = 4096, 2048, 256, 6
EXPERT_BYTES = 3 * I * D // 2 + 3 * I * D // 32          # 13,369,344
GATE_UP_BYTES = 2 * (I * D // 2 + I * D // 32)            # w1 + w3 + scales of one routed expert
DOWN_BYTES = D * I // 2 + D * I // 32                      # w2 + scales
SHARED_GATE_UP = 2 * I * D + 2 * (I // 128) * (D // 128) * 4
SHARED_DOWN = D * I + (D // 128) * (I // 128) * 4
ROUTER_BYTES = E * D * 2 + E * 4
EXPERT_WEIGHT_BYTES = K * EXPERT_BYTES + SHARED_GATE_UP + SHARED_DOWN     # routed + shared expert weights
LAYER_IO_BYTES = EXPERT_WEIGHT_BYTES + ROUTER_BYTES + 2 * D * 2             # + router weights, x in, out
HBM_PEAK_GBS = 8000.0


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None, help="default 400 (layer) / 64 (stack)")
    ap.add_argument("--warmup", type=int, default=None, help="default 40 (layer) / 4 (stack)")
    ap.add_argument("--workload", choices=("layer", "stack", "prefill"), default="layer",
                    help="layer: one MoE layer at decode M=1 (+ M=3 and lm_head side measurements); "
                         "stack: the 43-layer MoE-only decode loop with MTP verify, tok/s; "
                         "prefill: the M=512 grouped GEMM over Zipf(1.1)-routed experts")
    ap.add_argument("--stack-layers", type=int, default=43)
    ap.add_argument("--layers", type=int, default=8, help="distinct layers rotated through (MALL defeat)")
    ap.add_argument("--seed", type=int, default=1234)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--no-extras", action="store_true", help="skip the M=3 and lm_head side measurements")
    ap.add_argument("--calib-copy", action="store_true",
                    help="finish with 3 copies of a 256 MiB buffer (known bytes) to scale PMC byte counters")
    ap.add_argument("--path", choices=("fused", "staged"), default="fused",
                    help="fused: one persistent launch per layer (hsmoe_moe_layer_decode); "
                         "staged: router, gate/up and down launches")
    args = ap.parse_args()
    stack = args.workload == "stack"
    if args.steps is None:
        args.steps = {"stack": 64, "prefill": 50}.get(args.workload, 400)
    if args.warmup is None:
        args.warmup = {"stack": 4, "prefill": 5}.get(args.workload, 40)
    return args


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build has no multi-GPU path "
              "(expert-parallel sharding is described in DESIGN.md, not run). Use --gpus 1.", file=sys.stderr)
        sys.exit(2)
    import torch
    __graft_entry__.package()
    if args.workload in ("stack", "prefill"):
        print(json.dumps((run_stack if args.workload == "stack" else run_prefill)(args, torch)))
        return
    from home_seek_amd import expert_store, ops, synthetic

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    L = args.layers
    store = expert_store.HbmExpertStore(L, E, D, I, dev, with_shared=True)
    store.fill_synthetic(args.seed)
    routers = [synthetic.router_weights(args.seed, l, E, D, dev) for l in range(L)]
    xs = [synthetic.hidden(args.seed, 1000 + l, 1, D, dev) for l in range(L)]
    tables = [store.table(l) for l in range(L)]
    shareds = [store.shared_entry(l) for l in range(L)]
    idx_buf = [torch.empty(1, K, dtype=torch.int64, device=dev) for _ in range(L)]
    w_buf = [torch.empty(1, K, dtype=torch.float32, device=dev) for _ in range(L)]
    outs = [torch.empty(1, D, dtype=torch.bfloat16, device=dev) for _ in range(L)]
    torch.cuda.synchronize()

    fused = args.path == "fused"

    def step(l):
        if fused:
            ops.moe_layer_decode(xs[l], routers[l][0], routers[l][1], tables[l], ops.SCALE_E8M0, shareds[l], I, K,
                                 1.5, 10.0, out_bf16=outs[l], idx_out=idx_buf[l], w_out=w_buf[l])
            return
        idx, w = ops.router_topk(xs[l], routers[l][0], routers[l][1], K, 1.5, out=(idx_buf[l], w_buf[l]))
        ops.moe_decode(xs[l], idx, w, tables[l], ops.SCALE_E8M0, shareds[l], 10.0, out_bf16=outs[l], d=D, i=I)

    # warm-up (creates workspaces), then capture one rotation
    for j in range(max(1, args.warmup)):
        step(j % L)
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        for l in range(L):
            step(l)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            for l in range(L):
                step(l)
    replays = max(1, (args.steps + L - 1) // L)
    steps = replays * L
    for _ in range(max(1, args.warmup // L)):
        graph.replay()
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record()
    for _ in range(replays):
        graph.replay()
    ev1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_step = ev0.elapsed_time(ev1) / steps
    routed_gbs = K * EXPERT_BYTES / (ms_step * 1e-3) / 1e9

    # ---- dominant kernel
    # fused: a step is exactly one launch of moe_layer_kernel, so its average
    # duration is the step graph's event time per step (events on the stream
    # the graph replays on).  staged: stage 1 (gate/up) alone, back-to-back in
    # a graph of its own.
    def stage_graph(stage):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.stream(stream):
            for l in range(L):
                ops.moe_decode_stage(stage, xs[l], idx_buf[l], w_buf[l], tables[l], ops.SCALE_E8M0, shareds[l], 10.0,
                                     D, I, out_bf16=outs[l])
            torch.cuda.synchronize()
            with torch.cuda.graph(g, stream=stream):
                for l in range(L):
                    ops.moe_decode_stage(stage, xs[l], idx_buf[l], w_buf[l], tables[l], ops.SCALE_E8M0, shareds[l],
                                         10.0, D, I, out_bf16=outs[l])
        for _ in range(3):
            g.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        with torch.cuda.stream(stream):
            for _ in range(replays):
                g.replay()
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / (replays * L) * 1e3  # us per launch

    pmc_name = "moe_layer_kernel_m1_pmc.json" if fused else "moe_gate_up_kernel_m1_pmc.json"
    traffic = None
    pmc = ROOT / "profiles" / pmc_name
    if pmc.exists():  # HBM bytes per launch from the committed rocprofv3 --pmc FETCH_SIZE/WRITE_SIZE runs
        traffic = json.loads(pmc.read_text()).get("traffic_bytes_per_launch")
    if fused:
        us_launch = ms_step * 1e3
        kernel_bytes = LAYER_IO_BYTES
        roof = {"kernel": "moe_layer_kernel (router + 6 routed FP4 + FP8 shared expert, one launch)"}
    else:
        us_launch = stage_graph(1)
        us_stage2 = stage_graph(2)
        kernel_bytes = K * GATE_UP_BYTES + SHARED_GATE_UP + D * 2 + (K + 1) * 2 * I * 2
        stage2_bytes = K * DOWN_BYTES + SHARED_DOWN + (K + 1) * 2 * I * 2 + D * 6
        roof = {"kernel": "moe_gate_up_kernel (stage 1)",
                "stage2": {"kernel": "moe_down_kernel", "avg_launch_us": round(us_stage2, 3),
                           "achieved": round(stage2_bytes / (us_stage2 * 1e-6) / 1e9, 1),
                           "algorithmic_bytes_per_launch": stage2_bytes}}
    ach = kernel_bytes / (us_launch * 1e-6) / 1e9
    roof = {"bound": "hbm", **roof, "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": traffic, "algorithmic_bytes_per_launch": kernel_bytes,
            "avg_launch_us": round(us_launch, 3)}

    extras = {}
    if not args.no_extras:
        extras = side_measurements(torch, ops, synthetic, store, routers, tables, shareds, stream, args, L, fused)

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(args)

    line = {
        "metric": "MoE layer FP4 expert GB/s (% HBM peak) at M=1/M=3; MTP-verify decode tok/s",
        "value": round(routed_gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp4-e2m1 weights, bf16 MFMA, fp32 accumulate",
        "data": "synthetic (seeded on device)",
        "config": {
            "workload": "one MoE layer at decode M=1: router top-6 of 256 + 6 FP4 experts + FP8 shared expert, "
                        "D=4096 I=2048",
            "global_batch": 1,
            "seq_len": 1,
            "parallelism": "none (1 GPU)",
            "layers_rotated": L,
        },
        "pct_hbm_peak": round(100.0 * routed_gbs / HBM_PEAK_GBS, 2),
        "expert_gbs": round(EXPERT_WEIGHT_BYTES / (ms_step * 1e-3) / 1e9, 1),
        "full_layer_gbs": round(LAYER_IO_BYTES / (ms_step * 1e-3) / 1e9, 1),
        "path": args.path,
        "wall_s_timed": round(wall, 3),
        "roofline": roof,
        "cpu_baseline": cpu,
    }
    line.update(extras)
    if args.calib_copy:
        src = torch.ones(256 << 20, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
    print(json.dumps(line))


def side_measurements(torch, ops, synthetic, store, routers, tables, shareds, stream, args, L, fused):
    """M=3 verify layer (per-token distinct routing) and the T=3 lm_head + acceptance kernel."""
    xs3 = [synthetic.hidden(args.seed, 2000 + l, 3, D, store.device) for l in range(L)]
    uniq = []
    for l in range(L):
        idx, _ = ops.router_topk(xs3[l], routers[l][0], routers[l][1], K, 1.5)
        uniq.append(len(set(idx.reshape(-1).tolist())))
    outs = [torch.empty(3, D, dtype=torch.bfloat16, device=store.device) for _ in range(L)]

    def step3(l):
        if fused:
            ops.moe_layer_decode(xs3[l], routers[l][0], routers[l][1], tables[l], ops.SCALE_E8M0, shareds[l], I, K,
                                 1.5, 10.0, out_bf16=outs[l])
            return
        idx, w = ops.router_topk(xs3[l], routers[l][0], routers[l][1], K, 1.5)
        ops.moe_decode(xs3[l], idx, w, tables[l], ops.SCALE_E8M0, shareds[l], 10.0, out_bf16=outs[l], d=D, i=I)

    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        for l in range(L):
            step3(l)
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=stream):
            for l in range(L):
                step3(l)
    reps = max(2, args.steps // (4 * L))
    for _ in range(2):
        g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    with torch.cuda.stream(stream):
        for _ in range(reps):
            g.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    ms3 = e0.elapsed_time(e1) / (reps * L)
    m3_gbs = (sum(uniq) / L) * EXPERT_BYTES / (ms3 * 1e-3) / 1e9

    vocab = 129280
    lm = synthetic.normal_bf16(args.seed, synthetic.tag(synthetic.KIND_LM_HEAD), (vocab, D), 0.0, 0.02, store.device)
    h = synthetic.hidden(args.seed, 3000, 3, D, store.device)
    ids = torch.tensor([1, 2, 3], device=store.device)
    gl = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        ops.lm_head_accept(h, lm, ids)
        torch.cuda.synchronize()
        with torch.cuda.graph(gl, stream=stream):
            ops.lm_head_accept(h, lm, ids)
    gl.replay()
    torch.cuda.synchronize()
    reps_l = 20
    e0.record(stream)
    with torch.cuda.stream(stream):
        for _ in range(reps_l):
            gl.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    ms_lm = e0.elapsed_time(e1) / reps_l
    del lm
    return {
        "m3_layer": {"ms_per_step": round(ms3, 5), "unique_experts_avg": sum(uniq) / L,
                     "routed_gbs": round(m3_gbs, 1), "pct_hbm_peak": round(100 * m3_gbs / HBM_PEAK_GBS, 2)},
        "lm_head_t3_accept": {"ms": round(ms_lm, 4), "gbs": round(vocab * D * 2 / (ms_lm * 1e-3) / 1e9, 1)},
    }


def run_stack(args, torch):
    """The MoE-only decode stack: all layers' experts resident, greedy decode with
    MTP verify, one step = M=1 forward + 2 MTP drafts + T=3 verify, captured
    as one HIP graph and replayed; tok/s over the timed steps."""
    from home_seek_amd import ops, stack
    from home_seek_amd.engine import GreedyDecoder

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    n_layers, vocab = args.stack_layers, 129280
    t0 = time.perf_counter()
    eng = stack.build_stack(args.seed, n_layers=n_layers, n_experts=E, d=D, i=I, vocab=vocab, top_k=K, n_hash=3,
                            device=dev, log=lambda m: print(f"[stack] {m} ({time.perf_counter() - t0:.1f} s)",
                                                            file=sys.stderr, flush=True))
    torch.cuda.synchronize()
    t_build = time.perf_counter() - t0
    print(f"[stack] {n_layers} layers + MTP block built in {t_build:.1f} s "
          f"({eng.store.buf.numel() / 1e9:.1f} GB expert store)", file=sys.stderr, flush=True)
    dec = GreedyDecoder(eng, max(args.steps, args.warmup, 1))
    first = 1 + args.seed % (vocab - 1)
    dec.reset(first)
    dec.run(args.warmup)
    torch.cuda.synchronize()
    start_tok = int(dec.cur.item())
    dec.reset()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t1 = time.perf_counter()
    ev0.record()
    dec.run(args.steps)
    ev1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t1
    ms = ev0.elapsed_time(ev1)
    tokens, accs = dec.result()
    rows = dec.rows[:args.steps].cpu().tolist()
    print(f"[stack] {args.steps} steps in {ms:.1f} ms, {len(tokens)} tokens", file=sys.stderr, flush=True)

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
    expert_bytes = 0
    for r in rows:  # M=1 forward: K distinct experts per layer; verify [A, d0, d1]: their union
        ver = [route_of(x)[0] for x in r[:3]]
        for l in range(n_layers):
            expert_bytes += (K + len(ver[0][l] | ver[1][l] | ver[2][l])) * EXPERT_BYTES
    expert_bytes += args.steps * 2 * K * EXPERT_BYTES                       # MTP block, two drafts
    shared_bytes = args.steps * (2 * n_layers + 2) * (SHARED_GATE_UP + SHARED_DOWN)
    router_bytes = args.steps * (2 * (n_layers - 3) + 2) * ROUTER_BYTES
    lm_bytes = args.steps * 4 * vocab * D * 2                                 # main, 2 drafts, verify
    total = expert_bytes + shared_bytes + router_bytes + lm_bytes
    ach = total / (ms * 1e-3) / 1e9
    return {
        "metric": "MoE layer FP4 expert GB/s (% HBM peak) at M=1/M=3; MTP-verify decode tok/s",
        "value": round(len(tokens) / (ms * 1e-3), 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp4-e2m1 weights, bf16 MFMA, fp32 accumulate",
        "data": "synthetic (seeded on device)",
        "config": {
            "workload": f"{n_layers}-layer MoE-only decode stack (attention replaced by a seeded residual), "
                        f"{E} FP4 experts + FP8 shared per layer, D={D} I={I}, vocab {vocab}; per step M=1 "
                        "forward + 2 MTP drafts + T=3 verify, greedy",
            "global_batch": 1,
            "seq_len": 1,
            "parallelism": "none (1 GPU)",
        },
        "tokens": len(tokens),
        "accepted_per_step": round(sum(accs) / len(accs), 4),
        "tokens_per_step": round(len(tokens) / args.steps, 4),
        "greedy_chain_match": tokens == chain,
        "roofline": {"bound": "hbm", "kernel": "whole decode step (all kernels of one graph replay)",
                     "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": None,
                     "algorithmic_bytes_per_step": total // args.steps,
                     "lm_head_bytes_per_step": lm_bytes // args.steps},
        "build_s": round(t_build, 1),
        "wall_s_timed": round(wall, 3),
        "cpu_baseline": None,
    }


def run_prefill(args, torch):
    """Prefill MoE layer: M=512 tokens, 256 FP4 experts, top-6 with Zipf(1.1)
    popularity drawn without replacement per token, routed experts only (the
    shared expert is timed separately as an extra); one hsmoe_moe_prefill call
    (group, gate/up, down, combine) per step, steps captured in a HIP graph."""
    from home_seek_amd import expert_store, ops, synthetic

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    m = 512
    store = expert_store.HbmExpertStore(1, E, D, I, dev, with_shared=True)
    store.fill_synthetic(args.seed)
    x = synthetic.hidden(args.seed, 5000, m, D, dev)
    idx_h, w_h = synthetic.zipf_routing(args.seed, m, E, K)
    idx, w = torch.as_tensor(idx_h, device=dev), torch.as_tensor(w_h, device=dev)
    counts = [int(c) for c in __import__("numpy").bincount(idx_h.reshape(-1), minlength=E)]
    touched = sum(1 for c in counts if c)
    table, shared = store.table(0), store.shared_entry(0)
    out = torch.empty(m, D, dtype=torch.bfloat16, device=dev)
    torch.cuda.synchronize()

    def timed(sh, steps, warmup):
        fn = lambda: ops.moe_prefill(x, idx, w, table, ops.SCALE_E8M0, sh, 10.0, out_bf16=out, i=I)
        stream = torch.cuda.Stream()
        with torch.cuda.stream(stream):
            fn()
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=stream):
                fn()
        for _ in range(warmup):
            g.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            g.replay()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / steps

    ms = timed(None, args.steps, args.warmup)
    ms_sh = timed(shared, max(5, args.steps // 5), 2)
    routed_bytes = touched * EXPERT_BYTES
    io_bytes = m * D * 2 * 2 + m * K * 12
    flops = 3 * 2 * D * I * m * K  # gate, up, down of every (token, expert) pair
    gbs = routed_bytes / (ms * 1e-3) / 1e9
    ach = (routed_bytes + io_bytes) / (ms * 1e-3) / 1e9
    tflops = flops / (ms * 1e-3) / 1e12
    return {
        "metric": "MoE layer FP4 expert GB/s (% HBM peak) at M=1/M=3; MTP-verify decode tok/s",
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp4-e2m1 weights, bf16 MFMA, fp32 accumulate",
        "data": "synthetic (seeded on device; Zipf(1.1) routing seeded on the host)",
        "config": {
            "workload": f"prefill MoE layer, M={m} tokens, D={D} I={I}, {E} FP4 experts top-{K}, Zipf(1.1) "
                        "popularity (grouped gate/up + down GEMM), routed experts only",
            "global_batch": m,
            "seq_len": m,
            "parallelism": "none (1 GPU)",
        },
        "touched_experts": touched,
        "max_tokens_per_expert": max(counts),
        "pct_hbm_peak": round(100.0 * gbs / HBM_PEAK_GBS, 2),
        "mfma_tflops": round(tflops, 2),
        "pct_bf16_mfma_peak": round(100.0 * tflops / 2500.0, 3),
        "with_shared_expert": {"ms": round(ms_sh, 5),
                               "gbs": round((routed_bytes + SHARED_GATE_UP + SHARED_DOWN) / (ms_sh * 1e-3) / 1e9, 1)},
        "roofline": {"bound": "hbm", "kernel": "hsmoe_moe_prefill call (group + gate/up + down + combine launches)",
                     "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": None,
                     "algorithmic_bytes_per_launch": routed_bytes + io_bytes, "avg_launch_us": round(ms * 1e3, 2)},
        "cpu_baseline": None,
    }


def cpu_baseline(args):
    """Times the CPU oracle on a bounded sample of the same workload (one thread)."""
    import numpy as np
    try:
        from threadpoolctl import threadpool_limits
    except ImportError:  # pragma: no cover
        threadpool_limits = None
    from oracle import oracle as orc

    seed = args.seed
    n_layers = min(args.layers, 4)
    prepared = []
    for l in range(n_layers):
        gate = orc.gen_normal_bf16(orc.key(seed, orc.tag(orc.KIND_GATE_W, l)), E * D, 0.0, 0.02).reshape(E, D)
        bias = orc.gen_normal_f32(orc.key(seed, orc.tag(orc.KIND_GATE_BIAS, l)), E, 0.0, 0.01)
        x = orc.gen_normal_bf16(orc.key(seed, orc.tag(orc.KIND_HIDDEN, 0, 1000 + l)), D, 0.0, 1.0).reshape(1, D)
        idx, _ = orc.router(x, gate, bias, K, 1.5)
        raw = {}
        for e in idx[0]:
            ex = {}
            for sub, (nm, r, c) in enumerate((("w1", I, D), ("w3", I, D), ("w2", D, I))):
                ex[nm] = orc.gen_bytes(orc.key(seed, orc.tag(orc.KIND_FP4_DATA, l, int(e), sub)), r * c // 2).reshape(r, c // 2)
                ex[nm + "_scale"] = orc.gen_e8m0(orc.key(seed, orc.tag(orc.KIND_FP4_SCALE, l, int(e), sub)), r * c // 32).reshape(r, c // 32)
            raw[int(e)] = ex
        sh = orc.gen_shared_expert(seed, l, D, I)
        prepared.append((gate, bias, x, raw, sh))

    def one_layer(gate, bias, x, raw, sh):
        idx, w = orc.router(x, gate, bias, K, 1.5)
        experts = {}
        for e, ex in raw.items():
            experts[e] = {nm + "_bf16": orc.dequant_fp4(ex[nm], ex[nm + "_scale"]) for nm in ("w1", "w3", "w2")}
        shared = {nm + "_bf16": orc.dequant_fp8(sh[nm], sh[nm + "_scale"]) for nm in ("w1", "w3", "w2")}
        return orc.moe_layer_fp32(x, idx, w, experts, shared, 10.0)

    ctx = threadpool_limits(limits=1) if threadpool_limits else None
    if ctx:
        ctx.__enter__()
    try:
        one_layer(*prepared[0])
        n = 0
        t0 = time.perf_counter()
        while time.perf_counter() - t0 < args.cpu_seconds or n < 2:
            one_layer(*prepared[n % n_layers])
            n += 1
        dt = time.perf_counter() - t0
    finally:
        if ctx:
            ctx.__exit__(None, None, None)
    return {
        "value": round(n * K * EXPERT_BYTES / dt / 1e9, 4),
        "unit": "GB/s",
        "cores": 1,
        "kind": "port",
        "sample": f"{n} MoE layers at M=1 (router + per-call FP4/FP8 dequant + fp32 FFN of 6 routed + 1 shared "
                  f"expert), {dt:.1f} s on one thread; ms/layer {1e3 * dt / n:.1f}",
    }


if __name__ == "__main__":
    main()
