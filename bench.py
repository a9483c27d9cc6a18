"""MoE-layer benchmark on one MI355X (BASELINE.json metric).

Workload (configs[1] of BASELINE.json): OLMoE-1B-7B-shaped layer, hidden 2048,
64 experts of intermediate 1024, top-8 softmax routing, per-expert 2/3/4-bit
(50/25/25) group-64 HQQ weights, fp16 activations, synthetic data.  A step is
one full layer forward (route, permute, grouped gate/up + SiLU*mul, grouped
down, combine) over a 2048-token prefill batch already resident in HBM;
`value` is prefill tokens/s, measured after a short untimed clock settle.
The same run also reports prefill at 512 tokens, decode at batch 1 / 8 / 32 of
this layer and at batch 1 / 16 / 64 of the Mixtral-shaped layer of configs[4]
(HBM-bound; a stack of distinct layers whose experts exceed the last-level
cache, graph-replayed, as the reference times decode under CUDA graphs; per
layer), the live roofline of the dominant
kernel (the grouped gate/up GEMM, MFMA-bound at this size) with its HBM
traffic from the committed rocprofv3 counter summary, and the CPU baseline:
the oracle's fp32 dequantize-then-matmul expert loop on a bounded token
sample.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--config NAME]
                       [--tokens T] [--no-cpu] [--no-decode] [--no-mixtral]
"""

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "MoE-layer prefill+decode tokens/sec on 1 GPU; % HBM BW / % MFMA peak"
PEAK_MFMA_F16_TFLOPS = 2500.0  # MI355X dense fp16/bf16
PEAK_HBM_GBS = 8000.0
SETTLE_S = 0.3  # untimed layer forwards before the first measurement
DECODE_LAYERS = 4  # distinct layers in the decode stack of the headline config


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="olmoe_mixed")
    ap.add_argument("--tokens", type=int, default=2048)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--no-mixtral", action="store_true", help="skip the Mixtral-shaped decode and stack lines")
    ap.add_argument("--no-others", action="store_true", help="skip the OLMoE 2-bit T=128, Qwen3 and DeepSeek prefill lines")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="run one 256 MiB device-to-device copy first (reference size for HBM counters)")
    return ap.parse_args()


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def settle(fn, seconds):
    """Runs fn untimed for `seconds` (the GPU raises its clocks over the first
    tens of ms of load); returns the number of calls."""
    import torch
    n = 0
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end:
        for _ in range(10):
            fn()
        torch.cuda.synchronize()
        n += 10
    return n


def time_events(fn, steps, warmup, stream):
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record(stream)
    for _ in range(steps):
        fn()
    t1.record(stream)
    torch.cuda.synchronize()
    return t0.elapsed_time(t1) / steps  # ms


def time_graph(fn, steps, warmup, stream):
    """Device time of a short stage: fn is captured once in a CUDA graph and
    the graph replayed, so the Python and ctypes cost of each call (larger
    than a few-microsecond kernel) is not in the measurement."""
    import torch
    fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(stream)
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            fn()
    stream.wait_stream(s)
    torch.cuda.synchronize()
    return time_events(g.replay, steps, warmup, stream)


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": f"bench.py runs on exactly one GPU; --gpus {args.gpus} is not supported "
                                   "(the expert path is single-GPU here, multi-GPU sharding is design-only)"}))
        sys.exit(2)
    import numpy as np
    import torch

    from robustgemq_amd import ops
    from robustgemq_amd.synthetic import CONFIGS, build_block, flops, make_inputs, make_weights

    dev = torch.device("cuda:0")
    if args.calibrate_copy:
        src = torch.ones(64 * 1024 * 1024, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)  # reads and writes exactly 256 MiB
        torch.cuda.synchronize()
        del src, dst
    cfg = CONFIGS[args.config]
    T = args.tokens
    log(f"[bench] building {cfg.name} (synthetic weights, seed 0)")
    w = make_weights(cfg, seed=0, quant_device=dev)
    block = build_block(cfg, w, device=dev)
    layer = block._layer
    x = make_inputs(cfg, T, seed=0).to(dev)
    stream = torch.cuda.current_stream(dev)

    # ---------------- the step: full layer forward, T tokens
    out = torch.empty((T, cfg.hidden), dtype=cfg.act_dtype, device=dev)
    logits = torch.empty((T, cfg.n_experts), dtype=torch.float32 if cfg.family == "deepseekv2" else cfg.act_dtype,
                         device=dev)

    def step():
        layer.forward(x, out=out, logits=logits)

    # Clock settle: the GPU raises its clocks over the first tens of ms of
    # load (a cold 20-step loop reads ~15% slower than the same loop warm), so
    # the layer runs untimed for SETTLE_S before any measurement; every number
    # below is a sustained rate.
    settle_steps = settle(step, SETTLE_S)

    # ---------------- the timed steps (headline): W warmup, then exactly K.
    # Each timed step also records a pair of HIP events around its gate/up
    # launch (moeq_moe_forward_timed): the dominant kernel's duration inside
    # the timed region, for the roofline.
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
    for a, b in ev:  # torch creates an event at its first record
        a.record(stream)
        b.record(stream)
    log(f"[bench] prefill T={T}: warmup {args.warmup}, steps {args.steps}")
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        layer.forward(x, out=out, logits=logits, gate_up_events=ev[i])
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = wall * 1e3 / args.steps
    value = T * args.steps / wall

    # ---------------- stage timings and the dominant kernel's live roofline
    _, idx, wt = ops.route(x, layer.gate_w, layer.top_k, layer.norm_topk, logits=False, logit_bias=layer.logit_bias)
    plan = layer.plan(T)
    bm = plan["bm"]
    perm = ops.permute(idx, layer.n_experts, layer.n_shared, bm=bm)
    rows = T * layer.top_k + layer.n_shared * T
    counts = perm["counts"].cpu().numpy()
    hit = [e for e in range(layer.n_experts + layer.n_shared) if counts[e] > 0]

    def gate_up():
        return ops.grouped_gemm(x, rows, layer.inter, perm["tiles"], perm["n_tiles"], perm["max_tiles"], bm,
                                layer.w1, p1=layer.w3, row_src=perm["row_token"])

    h = gate_up()

    def down():
        return ops.grouped_gemm(h, rows, layer.hidden, perm["tiles"], perm["n_tiles"], perm["max_tiles"], bm,
                                layer.w2, out_dtype=torch.float16)

    def route_only():
        ops.route(x, layer.gate_w, layer.top_k, layer.norm_topk, logits=True, logit_bias=layer.logit_bias)

    def permute_only():
        ops.permute(idx, layer.n_experts, layer.n_shared, bm=bm)

    y = down()

    def combine_only():
        ops.combine(y, perm["inv_perm"], wt, T, layer.top_k, layer.n_shared, cfg.act_dtype)

    kt = {}
    for name, fn in (("route", route_only), ("permute", permute_only), ("gate_up", gate_up), ("down", down),
                     ("combine", combine_only)):
        timer = time_events if name in ("gate_up", "down") else time_graph
        kt[name] = timer(fn, args.steps, 3, stream)
    gu_ctx = sum(a.elapsed_time(b) for a, b in ev) / len(ev)  # ms, inside the timed steps
    gu_flops = 2.0 * rows * 2 * cfg.hidden * cfg.inter
    dn_flops = 2.0 * rows * cfg.hidden * cfg.inter
    gu_tflops = gu_flops / (gu_ctx * 1e-3) / 1e12
    w_bytes_gu = layer.w1.weight_bytes(hit) + layer.w3.weight_bytes(hit)
    kname = "grouped_gemm_kernel<BM=%d> gate/up (SiLU*mul epilogue)" % bm
    traffic, tsrc = profile_traffic(kname, f"{cfg.name} T={T}")
    roofline = {"bound": "mfma", "achieved": round(gu_tflops, 2), "peak": PEAK_MFMA_F16_TFLOPS, "unit": "TFLOP/s",
                "frac": round(gu_tflops / PEAK_MFMA_F16_TFLOPS, 4), "traffic": traffic,
                "kernel": kname, "flops_per_launch": gu_flops, "avg_launch_ms": round(gu_ctx, 4),
                "timing": "HIP events around the gate/up launch of each timed layer step",
                "algorithmic_bytes_per_launch": w_bytes_gu + rows * cfg.hidden * 2 + rows * cfg.inter * 2,
                "traffic_source": tsrc}
    layer_flops = flops(cfg, T)
    extra = {
        "settle": {"seconds": SETTLE_S, "steps": settle_steps},
        "stage_ms": {k: round(v, 4) for k, v in kt.items()},
        "layer_tflops": round(layer_flops / (ms_per_step * 1e-3) / 1e12, 2),
        "down_tflops": round(dn_flops / (kt["down"] * 1e-3) / 1e12, 2),
        "gate_up_weight_bytes": w_bytes_gu, "plan": plan, "hit_experts": len(hit),
    }

    # ---------------- secondary lines: prefill 512, decode (graph replay)
    runs = {}
    for tp in [t for t in cfg.runs.get("prefill", ()) if t != T]:
        xp = make_inputs(cfg, tp, seed=1).to(dev)
        settle(lambda: layer.forward(xp, want_logits=False), 0.2)
        ms = time_events(lambda: layer.forward(xp, want_logits=False), args.steps, args.warmup, stream)
        runs[f"prefill_T{tp}"] = {"tokens_per_s": round(tp / (ms * 1e-3), 1), "ms": round(ms, 4)}
    if not args.no_decode:
        # four distinct layers (seeds 0..3, ~600 MB of experts: more than the
        # 256 MB last-level cache) so a decode step streams its experts from HBM
        extra_layers = []
        for sd in range(1, DECODE_LAYERS):
            ew = make_weights(cfg, seed=sd, quant_device=dev)
            extra_layers.append(build_block(cfg, ew, device=dev)._layer)
            del ew
        runs.update(decode_runs(cfg, [layer] + extra_layers, cfg.runs.get("decode", ()), args, stream, ""))
        del extra_layers
        torch.cuda.empty_cache()
    if not args.no_mixtral and args.config != "mixtral_mixed":
        # the HBM-bound decode (two 55-100 MB experts per token) and
        # the 16-layer stack at 1024-token prefill
        mcfg = CONFIGS["mixtral_mixed"]
        log("[bench] building mixtral_mixed (synthetic weights, seed 0)")
        mw = make_weights(mcfg, seed=0, quant_device=dev)
        mlayer = build_block(mcfg, mw, device=dev)._layer
        del mw
        mw2 = make_weights(mcfg, seed=1, quant_device=dev)
        mlayer2 = build_block(mcfg, mw2, device=dev)._layer  # two layers: 1.2 GB of experts
        del mw2
        runs.update(decode_runs(mcfg, [mlayer, mlayer2], mcfg.runs.get("decode", ()), args, stream, "mixtral_"))
        del mlayer2
        runs.update(stack_run(mcfg, mlayer, 16, 1024, args, stream))
        del mlayer
        torch.cuda.empty_cache()
    if not args.no_others:
        # configs[0], configs[2] and configs[3] at their prefill sizes
        for name in ("olmoe_2bit", "qwen3_mixed", "deepseek_v2_lite"):
            if name == args.config:
                continue
            ocfg = CONFIGS[name]
            log(f"[bench] building {name} (synthetic weights, seed 0)")
            ow = make_weights(ocfg, seed=0, quant_device=dev)
            olayer = build_block(ocfg, ow, device=dev)._layer
            del ow
            for tp in ocfg.runs.get("prefill", ()):
                xp = make_inputs(ocfg, tp, seed=1).to(dev)
                settle(lambda: olayer.forward(xp, want_logits=False), 0.2)
                ms = time_events(lambda: olayer.forward(xp, want_logits=False), args.steps, args.warmup, stream)
                tf = flops(ocfg, tp) / (ms * 1e-3) / 1e12
                runs[f"{name}_prefill_T{tp}"] = {"tokens_per_s": round(tp / (ms * 1e-3), 1), "ms": round(ms, 4),
                                                 "layer_tflops": round(tf, 1),
                                                 "mfma_frac_layer": round(tf / PEAK_MFMA_F16_TFLOPS, 4)}
            if ocfg.runs.get("decode") and not args.no_decode:
                # a second layer (seed 1): two layers' experts exceed the
                # last-level cache, so the decode stack streams them from HBM
                ow2 = make_weights(ocfg, seed=1, quant_device=dev)
                olayer2 = build_block(ocfg, ow2, device=dev)._layer
                del ow2
                runs.update(decode_runs(ocfg, [olayer, olayer2], ocfg.runs["decode"], args, stream, f"{name}_"))
                del olayer2
            del olayer
            torch.cuda.empty_cache()
    extra["runs"] = runs

    # ---------------- CPU baseline: oracle fp32 expert loop, bounded sample
    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(cfg, w, args.cpu_seconds)

    line = {
        "metric": METRIC, "value": round(value, 1), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_per_step, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f16", "data": "synthetic",
        "config": {"workload": f"{cfg.name} MoE layer, prefill T={T} (BASELINE configs[1])", "hidden": cfg.hidden,
                   "inter": cfg.inter, "experts": cfg.n_experts, "top_k": cfg.top_k, "group_size": cfg.group_size,
                   "bits": dict(sorted({b: w["bits"].count(b) for b in set(w["bits"])}.items())),
                   "tokens": T, "act_dtype": str(cfg.act_dtype).replace("torch.", "")},
        "roofline": roofline, "cpu_baseline": cpu, "extra": extra,
    }
    print(json.dumps(line))


def stack_run(cfg, layer, n_layers, T, args, stream):
    """The n-layer stack of configs[4] at T-token prefill, timed end to end:
    each layer's output feeds the next.  The layers share one set of synthetic
    weights (581 MB, more than the 256 MB last-level cache, so every layer
    still streams its experts from HBM)."""
    import torch

    from robustgemq_amd.synthetic import flops, make_inputs
    dev = torch.device("cuda:0")
    x0 = make_inputs(cfg, T, seed=4).to(dev)
    bufs = [torch.empty_like(x0), torch.empty_like(x0)]

    def stack():
        h = x0
        for i in range(n_layers):
            layer.forward(h, out=bufs[i & 1], want_logits=False)
            h = bufs[i & 1]

    settle(stack, 0.2)
    ms = time_events(stack, max(2, args.steps // 4), 1, stream)
    tf = n_layers * flops(cfg, T) / (ms * 1e-3) / 1e12
    return {f"mixtral_stack{n_layers}_prefill_T{T}": {
        "tokens_per_s": round(T / (ms * 1e-3), 1), "ms": round(ms, 3), "layers": n_layers,
        "tflops": round(tf, 1), "mfma_frac": round(tf / PEAK_MFMA_F16_TFLOPS, 4),
        "weights": "one synthetic layer's weights reused by all layers"}}


def decode_runs(cfg, layers, batches, args, stream, tag):
    """Decode steps of a stack of distinct layers (each layer's output feeds
    the next, as in a model), captured in one CUDA graph and replayed, as the
    reference times decode under CUDA graphs; per-layer time = replay time / L.
    The layers' experts together exceed the 256 MB last-level cache, so the
    weights come from HBM rather than from the previous replay's cache lines.
    Each replay's output is checked against the eager stack.  HBM fraction =
    algorithmic bytes per layer (packed codes + scale/zero of the hit experts,
    router, activations; averaged over the stack) / per-layer time / 8 TB/s."""
    import torch

    from robustgemq_amd import ops
    from robustgemq_amd.synthetic import make_inputs
    dev = torch.device("cuda:0")
    out = {}
    L = len(layers)
    for B in batches:
        xb = make_inputs(cfg, B, seed=2).to(dev)
        hs = [torch.empty((B, cfg.hidden), dtype=cfg.act_dtype, device=dev) for _ in range(L)]

        def stack():
            h = xb
            for i, ly in enumerate(layers):
                # batch 1 is forward_one_token, as the reference decodes
                ly.forward(h, out=hs[i], want_logits=False, one_token=B == 1)
                h = hs[i]

        stack()  # sizes the workspaces before capture
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        s = torch.cuda.Stream(dev)
        s.wait_stream(stream)
        with torch.cuda.stream(s):
            stack()
            torch.cuda.synchronize()
            with torch.cuda.graph(g, stream=s):
                stack()
        stream.wait_stream(s)
        ref = hs[-1].clone()
        settle(g.replay, 0.2)
        ms_graph = time_events(g.replay, args.steps * 5, args.warmup, stream) / L
        assert torch.equal(hs[-1], ref), "graph replay changed the decode output"
        ms_eager = time_events(stack, args.steps, args.warmup, stream) / L
        bytes_b = 0
        h = xb
        for i, ly in enumerate(layers):
            idx_b = ops.route(h, ly.gate_w, ly.top_k, ly.norm_topk, logits=False, logit_bias=ly.logit_bias)[1]
            hit_b = sorted(set(idx_b.cpu().numpy().reshape(-1).tolist()))
            bytes_b += (ly.w1.weight_bytes(hit_b) + ly.w3.weight_bytes(hit_b) + ly.w2.weight_bytes(hit_b)
                        + cfg.n_experts * cfg.hidden * 2 + 2 * B * cfg.hidden * 2)
            h = hs[i]
        bytes_b //= L
        out[f"{tag}decode_B{B}"] = {"tokens_per_s": round(B / (ms_graph * 1e-3), 1), "ms_graph": round(ms_graph, 4),
                                     "ms_eager": round(ms_eager, 4), "layers": L,
                                     "alg_bytes": bytes_b,
                                     "hbm_frac_layer": round(bytes_b / (ms_graph * 1e-3) / (PEAK_HBM_GBS * 1e9), 4)}
    return out


def profile_traffic(kernel, workload):
    """HBM bytes per launch of `kernel` on `workload` from the committed
    rocprofv3 --pmc summary (FETCH_SIZE x 2.0 + WRITE_SIZE x 1.0, the factors a
    256 MiB copy calibrates), or None when no summary for them is committed."""
    import re
    path = os.path.join(ROOT, "profiles", "grouped_gemm_hbm_traffic.md")
    if not os.path.exists(path):
        return None, None
    for line in open(path):
        m = re.match(r"\|\s*`([^`]+)`\s*\|\s*`([^`]+)`\s*\|.*\|\s*(\d+)\s*\|\s*$", line)
        if m and m.group(1) == kernel and m.group(2) == workload:
            return int(m.group(3)), "profiles/grouped_gemm_hbm_traffic.md"
    return None, None


def cpu_baseline(cfg, w, budget_s):
    """Oracle fp32 dequantize-then-matmul loop (the reference's forward_n_tokens
    restated, gemq/inference/moe_block.py:781-815) on a bounded token sample;
    dense weights are materialized before timing, as the reference's fake
    model holds them."""
    import numpy as np
    import threadpoolctl
    import torch

    from oracle import moe as om
    from oracle import quant as oq
    from robustgemq_amd.synthetic import make_inputs

    log("[bench] cpu baseline: dequantizing weights on the host")

    def dense(t):
        N, K = t.shape
        return oq.dequant_hqq(t.Q.cpu().numpy(), t.scales.cpu().numpy(), t.zeros.cpu().numpy()).reshape(
            N, K).astype(np.float32)

    W1 = [dense(e["gate_proj"]) for e in w["experts"]]
    W3 = [dense(e["up_proj"]) for e in w["experts"]]
    W2 = [dense(e["down_proj"]) for e in w["experts"]]
    gate = w["gate"].float().numpy()
    ldt = "f16" if cfg.act_dtype == torch.float16 else "bf16"
    Ts = 256
    x = make_inputs(cfg, Ts, seed=3).float().numpy()
    cores = os.cpu_count()
    with threadpoolctl.threadpool_limits(limits=cores):
        info = threadpoolctl.threadpool_info()
        threads = max([i.get("num_threads", 1) for i in info] or [1])
        om.moe_forward(x, gate, ldt, cfg.top_k, cfg.norm_topk, W1, W3, W2)  # warm-up
        times = []
        t_start = time.perf_counter()
        while len(times) < 5 or (time.perf_counter() - t_start < budget_s and len(times) < 50):
            t0 = time.perf_counter()
            om.moe_forward(x, gate, ldt, cfg.top_k, cfg.norm_topk, W1, W3, W2)
            times.append(time.perf_counter() - t0)
    med = float(np.median(times))
    model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"value": round(Ts / med, 1), "unit": "tokens/s", "cores": int(threads), "kind": "port",
            "sample": f"{Ts}-token prefill of the same layer (median of {len(times)} reps, "
                      f"fp32 numpy BLAS, weights pre-dequantized), host {model} x{cores}"}


if __name__ == "__main__":
    main()
