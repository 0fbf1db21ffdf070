"""bench.py - TinyStrata's MoE expert matmul on one MI355X.

    python bench.py [--steps K] [--warmup W] [--config decode|verify|plumb|prefill|prefill_long] [--eager] [--no-cpu]

Default: the decode MoE layer stack of BASELINE.json configs[1].  A step is one pass of the hot path over one batch:
  decode / verify / plumb   T tokens (1 or 4) through 40 MoE layers with distinct weights (so experts stream from
                            HBM): routing, grouping, Q8_1 activations, the grouped experts (and the shared expert) and
                            the weighted combine, each layer's output feeding the next (x <- x + moe(x)).
  prefill / prefill_long    a prompt chunk (512 or 4096 tokens) through 4 such layers with the prompt path: routing,
                            expert sort, Q8_1 activations, the grouped gate/up with SwiGLU (f16 MFMA on exact integer
                            codes), the grouped down product and the combine.
Inputs are synthetic (N(0,0.02) weights quantized by this library, N(0,1) activations, N(0,1) router logits with the
config's skew) and resident in HBM before the timed region.  Prints one JSON line: the driver's contract plus the
roofline of the dominant launch (timed with HIP events on its stream) and the reference CPU path timed on this host.
The default decode line carries a "secondary" block with the other four BASELINE configurations measured the same
way, each with its roofline and CPU baseline; the verify step also times its tokens through the one-token layer one
at a time ("per_token").
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "MoE layer tokens/s; decode HBM GB/s and prefill int8-MFMA % of peak"
HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
INT8_PEAK_TOPS = 5000.0        # MI355X dense int8 MFMA
F16_PEAK_TFLOPS = 2500.0       # MI355X dense f16 MFMA: the engine the prompt products run on

CONFIGS = {
    "decode": dict(gu=18, d=21, N=2048, FF=512, E=256, k=8, shared=True, T=1, layers=40, route="normal",
                   desc="configs[1]: decode, 256 experts top-8 + shared, IQ3_XXS/IQ3_S"),
    "verify": dict(gu=18, d=21, N=2048, FF=512, E=256, k=8, shared=True, T=4, layers=40, route="correlated",
                   desc="configs[2]: speculative verify M=4, correlated routing"),
    "plumb": dict(gu=8, d=8, N=2048, FF=768, E=128, k=8, shared=False, T=1, layers=40, route="normal",
                  desc="configs[0]: decode, 128 experts top-8, Q8_0"),
    "prefill": dict(gu=12, d=12, N=2048, FF=768, E=128, k=8, shared=False, T=512, layers=4, route="zipf1.1",
                    desc="configs[3]: prefill 512 tokens, 128 experts top-8, Q4_K, Zipf(1.1) skew"),
    "prefill_long": dict(gu=18, d=21, N=2048, FF=512, E=256, k=8, shared=True, T=4096, layers=4, route="zipf1.3",
                         outliers=True, desc="configs[4]: prefill 4096 tokens, 256 experts top-8 + shared, IQ3, "
                                              "Zipf(1.3) skew, 1% outlier channels x20"),
    # not a BASELINE configuration: the hybrid CPU/GPU split on configs[1]'s layer, half of the experts in HBM
    "hybrid": dict(gu=18, d=21, N=2048, FF=512, E=256, k=8, shared=True, T=1, layers=4, route="normal",
                   resident=128, desc="hybrid: configs[1]'s decode layer with 128 of 256 experts in HBM, the rest "
                                      "on the CPU pool"),
}


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def make_logits(rng, cfg, layers):
    T, E = cfg["T"], cfg["E"]
    if cfg["route"] == "correlated":
        z = rng.normal(0, 1, (layers, 1, E))
        return (z + 0.5 * rng.normal(0, 1, (layers, T, E))).astype(np.float32)
    if cfg["route"].startswith("zipf"):
        s = float(cfg["route"][4:])
        bias = np.stack([np.log(1.0 / (1 + rng.permutation(E)) ** s) for _ in range(layers)])[:, None, :]
        return (rng.normal(0, 1, (layers, T, E)) + bias).astype(np.float32)
    return rng.normal(0, 1, (layers, T, E)).astype(np.float32)


def parse_args(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="decode", choices=sorted(CONFIGS))
    ap.add_argument("--eager", action="store_true", help="launch each step eagerly instead of replaying a HIP graph")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--norm", action="store_true",
                    help="end every layer with the MoE block's norm epilogue (h = rms(x) * norm_w and its Q8_1 image)")
    ap.add_argument("--no-secondary", action="store_true",
                    help="skip the prompt-chunk configurations measured after the default decode line")
    ap.add_argument("--layers", type=int, default=0,
                    help="layers per step (default: the configuration's; the default line's prompt-chunk entries use 2)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--secondary-cpu-seconds", type=float, default=4.0,
                    help="CPU baseline sample of each secondary configuration")
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="before the timed region, run one plain fp32 copy kernel (out = in * 1) over this many MiB: "
                         "the known-size launch that scales rocprofv3's FETCH_SIZE / WRITE_SIZE to bytes")
    ap.add_argument("--trace-marks", action="store_true",
                    help="launch a tiny int16 fill just before and just after the timed steps, and an int8 fill "
                         "around the dominant-launch loop, outside both timed regions, so that --summarize-trace can "
                         "pick those regions' dispatches out of a rocprofv3 kernel trace")
    ap.add_argument("--summarize-trace", metavar="KERNEL_TRACE_CSV",
                    help="no GPU work: summarize a rocprofv3 kernel trace of a --trace-marks run (the dispatches "
                         "between the marks only) as markdown")
    ap.add_argument("--summarize-pmc", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                    help="no GPU work: HBM bytes per dominant launch from two rocprofv3 --pmc counter files "
                         "(FETCH_SIZE, WRITE_SIZE) of a --copy-probe-mib run; prints markdown and, with "
                         "--traffic-json, records the figure under --config's name")
    ap.add_argument("--traffic-json", help="with --summarize-pmc: the traffic record to update (profiles/traffic.json)")
    ap.add_argument("--pmc-source", default="", help="with --summarize-pmc: the commands that made the counter files")
    return ap.parse_args(argv)


def main() -> int:
    args = parse_args()
    if args.summarize_trace:
        print(summarize_trace(args.summarize_trace, args.steps))
        return 0
    if args.summarize_pmc:
        print(summarize_pmc(args, *args.summarize_pmc))
        return 0
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build runs on one GPU; --gpus N > 1 is not supported (the sharding plan is design only)",
              file=sys.stderr)
        return 2
    cfg = CONFIGS[args.config]
    if "resident" in cfg:
        return run_hybrid(args, cfg)
    res = run_config(args, args.config, cfg, args.steps, args.warmup, cpu=not args.no_cpu, layers=args.layers or None)
    line = {
        "metric": METRIC,
        "value": res["value"],
        "unit": "MoE-layer tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": res["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": res["config"],
        "roofline": res["roofline"],
        "cpu_baseline": res["cpu_baseline"],
    }
    if args.config == "decode" and not args.no_secondary:
        # every other BASELINE configuration, each measured the same way (not part of `value`): the metric's prefill
        # half (the prompt chunks, fewer layers and steps), the Q8_0 plumbing layer and the speculative verify step
        # (with the same tokens through the one-token layer one at a time beside it)
        sec = {}
        for name, kw in (("prefill_long", dict(steps=8, warmup=2, layers=2)),
                         ("prefill", dict(steps=8, warmup=2, layers=2)),
                         ("plumb", dict(steps=10, warmup=3)),
                         ("verify", dict(steps=10, warmup=3))):
            r = run_config(args, name, CONFIGS[name], cpu=not args.no_cpu, cpu_seconds=args.secondary_cpu_seconds,
                           **kw)
            c = r["config"]
            sec[name] = {"workload": c["workload"], "value": r["value"], "unit": "MoE-layer tokens/s",
                         "ms_per_step": r["ms_per_step"], "layers": c["layers"], "layer_us": c["layer_us"],
                         "layer_hbm_frac": c["layer_hbm_frac"], "layer_int8_mfma_frac": c["layer_int8_mfma_frac"],
                         "distinct_experts_per_layer": c["distinct_experts_per_layer"],
                         "roofline": r["roofline"], "cpu_baseline": r["cpu_baseline"]}
            for key in ("distinct_experts_min_max", "per_token"):
                if key in c:
                    sec[name][key] = c[key]
        line["secondary"] = sec
    print(json.dumps(line), flush=True)
    return 0


def run_config(args, name, cfg, steps, warmup, cpu, layers=None, cpu_seconds=None):
    """One configuration: synthetic weights and inputs in HBM, `steps` timed steps (graph replays unless --eager), the
    dominant launch timed alone, and (cpu) the reference CPU path on this host."""
    import torch

    from tinystrata_amd import _lib, moe, ops

    gu, d, N, FF, E, k, shared, T = (cfg[key] for key in ("gu", "d", "N", "FF", "E", "k", "shared", "T"))
    layers = layers or cfg["layers"]
    prefill = T > 8
    dev = torch.device("cuda:0")
    _lib.check(_lib.lib().tsx_moe_init(0), "tsx_moe_init")
    L = ops.native_expert_layout(gu, d, N, FF)
    stride = moe.blob_stride(L)

    # ---------------------------------------------------------------- synthetic weights, resident in HBM
    t0 = time.time()
    distinct = 24
    pool = moe.synthetic_pool(L, distinct, seed=1234)
    pool_dev = torch.from_numpy(pool).to(dev)
    log(f"bench {name}: {distinct} distinct experts quantized in {time.time() - t0:.1f}s; "
        f"{layers} layers x {E + int(shared)} blobs x {stride / 1e6:.3f} MB in HBM")
    rng = np.random.default_rng(7)
    Ws, orders, shared_idx = [], [], []
    for l in range(layers):
        order = (rng.permutation(E) + l) % distinct
        si = int(rng.integers(distinct)) if shared else None
        Ws.append(moe.weights_from_pool(L, pool_dev, E, order, si))
        orders.append(order)
        shared_idx.append(si)
    del pool_dev

    # ---------------------------------------------------------------- inputs
    x0 = rng.normal(0, 1, (T, N)).astype(np.float32)
    if cfg.get("outliers"):
        x0[:, rng.choice(N, N // 100, replace=False)] *= 20.0
    logits = make_logits(rng, cfg, layers)
    sg = rng.normal(0, 1, (layers, T)).astype(np.float32)
    x0_d = torch.from_numpy(x0).to(dev)
    x = torch.empty_like(x0_d)
    logits_d = torch.from_numpy(logits).to(dev)
    sg_d = torch.from_numpy(sg).to(dev)
    mls = [moe.MoELayer(Ws[l], k, T, dev) for l in range(layers)]
    # --norm: every layer ends as the reference's MoE block does (k_moe_out_small with the next layer's norm weights):
    # h = rms(x) * norm_w and its Q8_1 image, the next layer's input
    norm = {}
    if args.norm:
        norm = dict(norm_w=torch.from_numpy((1.0 + 0.1 * rng.normal(0, 1, N)).astype(np.float32)).to(dev), eps=1e-6,
                    h=torch.empty((T, N), device=dev), hq=torch.empty((T, N // 32 * 36), dtype=torch.uint8, device=dev))

    def step():
        x.copy_(x0_d)
        for l in range(layers):
            mls[l](x, logits_d[l], sg_d[l] if shared else None, x, **norm)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    graph = None
    if not args.eager:
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            step()
        torch.cuda.current_stream().wait_stream(s)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            step()
        for _ in range(warmup):
            graph.replay()
    torch.cuda.synchronize()

    if args.copy_probe_mib > 0:
        n = args.copy_probe_mib << 18  # fp32 elements
        src = torch.ones(n, device=dev)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        torch.mul(src, 1.0, out=dst)
        torch.cuda.synchronize()
        log(f"bench: copy probe read {4 * n} bytes and wrote {4 * n} bytes")
        del src, dst

    # ---------------------------------------------------------------- timed region
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    mark = (lambda dt: torch.full((3,), 7, dtype=dt, device=dev)) if args.trace_marks else (lambda dt: None)
    torch.cuda.synchronize()
    mark(torch.int16)
    start.record()
    for _ in range(steps):
        graph.replay() if graph is not None else step()
    end.record()
    mark(torch.int16)
    torch.cuda.synchronize()
    ms_step = start.elapsed_time(end) / steps
    value = layers * T / (ms_step / 1e3)
    log(f"bench {name}: {ms_step:.4f} ms per step of {layers} layers")

    # algorithmic work: each distinct expert's blob once per layer, the fp32 input and output rows; int8 ops
    ids_host = [ml.ids.cpu().numpy() for ml in mls]
    distinct_per_layer = [len(np.unique(i)) for i in ids_host]
    blob = L.bytes
    layer_bytes = [(n + int(shared)) * blob + 2 * T * N * 4 for n in distinct_per_layer]
    layer_ops = 2 * T * (k + int(shared)) * (3 * N * FF)
    layer_s = ms_step / layers / 1e3

    # ---------------------------------------------------------------- the dominant launch, timed alone
    reps = max(3, min(20, steps // 5))
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    if prefill and mls[0].fused_prefill:
        # the grouped gate/up product with SwiGLU and the Q8_1 of h fused in, every layer, on the current stream
        def dom():
            for ml in mls:
                W = ml.W
                ops.mmq_gate_up_swiglu(W.blobs, L.gu_type, FF, N, W.stride, W.n_expert, ml.txq, T, ml.sort[2],
                                       ml.sort[0], ml.n_ent, hq=ml.mhq)
        # the distinct experts' gate/up rows, each token's Q8_1 row once, h's Q8_1 rows out
        gu_bytes = 2 * FF * L.gu_row
        dom_bytes = float(np.mean([n * gu_bytes + T * (N + N // 32 * 8) + ml.n_ent * (FF + FF // 32 * 8)
                                   for n, ml in zip(distinct_per_layer, mls)]))
        dom_ops = 2.0 * T * k * 2 * FF * N
        kernel = ("mmq_f16_kernel<fused> (grouped gate/up product with SwiGLU and the Q8_1 of h, "
                  "v_mfma_f32_16x16x32_f16 on exact integer codes) per layer")
    elif prefill:
        # the grouped gate/up product (f16 MFMA on exact integer codes) of every layer, on the current stream
        def dom():
            for ml in mls:
                W = ml.W
                ops.mmq_run(W.blobs, L.gu_type, 2 * FF, N, W.stride, W.n_expert, ml.mxq, ml.sort[0], None, ml.n_ent,
                            ml.gu, 2 * FF)
        gu_bytes = 2 * FF * L.gu_row
        dom_bytes = float(np.mean([n * gu_bytes + ml.n_ent * (N + N // 32 * 8) + ml.n_ent * 2 * FF * 4
                                   for n, ml in zip(distinct_per_layer, mls)]))
        dom_ops = 2.0 * T * k * 2 * FF * N
        kernel = "mmq_f16_kernel (grouped gate/up product, v_mfma_f32_16x16x32_f16 on exact integer codes) per layer"
    else:
        # the whole expert work of a layer: tsx_moe_decode_layer's two launches, on the current stream
        def dom():
            for l, ml in enumerate(mls):
                ops.moe_decode_layer(L, ml.W.blobs, ml.W.stride, ml.W.n_expert, k, logits_d[l], x, x, ml.ids, ml.wts,
                                     ml.lscratch, shared=ml.W.shared, sgate=sg_d[l] if shared else None)
        dom_bytes = float(np.mean(layer_bytes))
        dom_ops = float(layer_ops)
        kernel = ("tsx_moe_decode_layer (" + ("layer_gu1s_kernel" if T == 1 else "layer_gut_kernel") +
                  " + layer_down_kernel) per layer")
    dom()
    torch.cuda.synchronize()
    # replayed from a HIP graph like the timed steps, so the figure is the kernels' time, not host launch gaps
    dom_graph = None
    if not args.eager:
        s2 = torch.cuda.Stream()
        s2.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s2):
            dom()
        torch.cuda.current_stream().wait_stream(s2)
        dom_graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(dom_graph):
            dom()
        dom_graph.replay()
    torch.cuda.synchronize()
    mark(torch.int8)
    ev0.record()
    for _ in range(reps):
        dom_graph.replay() if dom_graph is not None else dom()
    ev1.record()
    mark(torch.int8)
    torch.cuda.synchronize()
    dom_s = ev0.elapsed_time(ev1) / (reps * layers) / 1e3
    achieved_gbs = dom_bytes / dom_s / 1e9
    achieved_tops = dom_ops / dom_s / 1e12
    if prefill and name == "prefill_long":
        # the products are f16 MFMAs on exact integer codes (2 flops per multiply-add, as an int8 op count), so the
        # roofline is the f16 MFMA peak; the fraction of the int8 peak is reported beside it
        roof = {"bound": "mfma", "achieved": round(achieved_tops, 2), "peak": F16_PEAK_TFLOPS,
                "unit": "TFLOP/s (f16 MFMA on exact integer codes)", "frac": round(achieved_tops / F16_PEAK_TFLOPS, 4)}
    else:
        roof = {"bound": "hbm", "achieved": round(achieved_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved_gbs / HBM_PEAK_GBS, 4)}
    traffic = measured_traffic(name)
    roof.update({"traffic": traffic, "kernel": kernel, "launch_us": round(dom_s * 1e6, 3),
                 "bytes_per_launch": int(dom_bytes), "int8_ops_per_launch": int(dom_ops),
                 "traffic_over_algorithmic": round(traffic / dom_bytes, 3) if traffic else None,
                 "hbm_frac": round(achieved_gbs / HBM_PEAK_GBS, 4),
                 "int8_mfma_frac": round(achieved_tops / INT8_PEAK_TOPS, 4)})
    if prefill:
        roof["f16_mfma_frac"] = round(achieved_tops / F16_PEAK_TFLOPS, 4)

    # the verify step: the same tokens through the one-token layer, one token at a time, beside the grouped call
    per_token = None
    if name == "verify":
        per_token = one_token_layers(args, Ws, k, T, N, layers, x0_d, logits_d, sg_d, shared, steps, dev, ms_step)

    cpu_res = None
    if cpu:
        cpu_res = cpu_baseline(args, L, pool, orders, shared_idx, ids_host, mls, x0, sg, layers, T, k, shared,
                               seconds=cpu_seconds)
    config = {
        "workload": f"{name}: {cfg['desc']}",
        "tokens": T, "layers": layers, "hidden": N, "expert_ff": FF, "experts": E, "top_k": k,
        "shared_expert": shared, "graph": graph is not None,
        "layer_us": round(layer_s * 1e6, 3),
        "layer_hbm_GBps": round(float(np.mean(layer_bytes)) / layer_s / 1e9, 1),
        "layer_hbm_frac": round(float(np.mean(layer_bytes)) / layer_s / 1e9 / HBM_PEAK_GBS, 4),
        "layer_int8_TOPs": round(layer_ops / layer_s / 1e12, 3),
        "layer_int8_mfma_frac": round(layer_ops / layer_s / 1e12 / INT8_PEAK_TOPS, 5),
        "layer_bytes": int(np.mean(layer_bytes)),
        "distinct_experts_per_layer": float(np.mean(distinct_per_layer)),
        "distinct_experts_min_max": [int(np.min(distinct_per_layer)), int(np.max(distinct_per_layer))],
        "layer_int8_ops": layer_ops,
    }
    if per_token is not None:
        config["per_token"] = per_token
    del mls, Ws, graph, dom_graph
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return {"value": round(value, 2), "ms_per_step": round(ms_step, 4), "config": config, "roofline": roof,
            "cpu_baseline": cpu_res}


def one_token_layers(args, Ws, k, T, N, layers, x0_d, logits_d, sg_d, shared, steps, dev, grouped_ms):
    """The verify step's T tokens through the one-token decode layer one at a time (T launches of the one-token layer
    per layer, each token's row its own x), timed like the grouped step: what the grouped several-token call saves."""
    import torch

    from tinystrata_amd import moe

    mls1 = [[moe.MoELayer(Ws[l], k, 1, dev) for _ in range(T)] for l in range(layers)]
    x1 = torch.empty((T, N), device=dev)

    def step1():
        x1.copy_(x0_d)
        for l in range(layers):
            for t in range(T):
                row = x1[t:t + 1]
                mls1[l][t](row, logits_d[l, t:t + 1], sg_d[l, t:t + 1] if shared else None, row)

    step1()
    torch.cuda.synchronize()
    graph = None
    if not args.eager:
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            step1()
        torch.cuda.current_stream().wait_stream(s)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            step1()
        graph.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        graph.replay() if graph is not None else step1()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    del mls1, graph
    return {"what": f"the same {T} tokens through the one-token layer, one launch pair per token and layer",
            "layer_us": round(ms / layers * 1e3, 3), "ms_per_step": round(ms, 4),
            "grouped_over_per_token": round(grouped_ms / ms, 4)}


def run_hybrid(args, cfg) -> int:
    """The hybrid decode layer (tinystrata_amd.pool.HybridMoELayer): eager steps of `layers` layers with distinct
    weights, each with a host round trip (routing to the host, the CPU rows back), so no graph.  value = layer-tokens/s
    of the whole layer; "pool" = the CPU pool's expert bytes per second over its drain time."""
    import torch

    from tinystrata_amd import _lib, moe, ops
    from tinystrata_amd.pool import ExpertPool, HybridMoELayer

    gu, d, N, FF, E, k, T, layers, R = (cfg[key] for key in ("gu", "d", "N", "FF", "E", "k", "T", "layers",
                                                               "resident"))
    dev = torch.device("cuda:0")
    _lib.check(_lib.lib().tsx_moe_init(0), "tsx_moe_init")
    L = ops.native_expert_layout(gu, d, N, FF)
    distinct = 24
    pool = moe.synthetic_pool(L, distinct, seed=1234)
    pool_dev = torch.from_numpy(pool).to(dev)
    rng = np.random.default_rng(7)
    cpu = ExpertPool()
    hys = []
    for l in range(layers):
        order = (rng.permutation(E) + l) % distinct
        # the routed experts live in the host copy and the layer's slots only
        W = moe.MoEWeights(L=L, n_expert=E, stride=pool.shape[1], blobs=torch.empty(0, dtype=torch.uint8, device=dev),
                           shared=pool_dev[int(rng.integers(distinct))].clone())
        hys.append(HybridMoELayer(W, np.ascontiguousarray(pool[order]), np.sort(rng.permutation(E)[:R]), k, T, dev,
                                  cpu))
    del pool_dev
    x0 = torch.from_numpy(rng.normal(0, 1, (T, N)).astype(np.float32)).to(dev)
    logits = torch.from_numpy(make_logits(rng, cfg, layers)).to(dev)
    sg = torch.from_numpy(rng.normal(0, 1, (layers, T)).astype(np.float32)).to(dev)
    x = torch.empty_like(x0)

    def step():
        x.copy_(x0)
        for l in range(layers):
            hys[l](x, logits[l], sg[l], x)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    st0 = cpu.stats()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    st1 = cpu.stats()
    per_layer = dt / (args.steps * layers)
    drain_s = (st1["drain"] - st0["drain"]) / 1e3
    pool_gbs = (st1["bytes"] - st0["bytes"]) / drain_s / 1e9 if drain_s > 0 else None
    misses = sum(h.n_miss for h in hys) / layers
    print(json.dumps({
        "metric": METRIC, "value": round(T / per_layer, 1), "unit": "layer-tokens/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(dt / args.steps * 1e3, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int8 x int8 -> int32, fp32",
        "data": "synthetic: random-init quantized experts, N(0,1) activations and logits",
        "config": {"workload": cfg["desc"], "layer_us": round(per_layer * 1e6, 3), "n_tok": T,
                   "layers": layers, "resident_experts": R, "experts": E, "cpu_entries_per_layer": misses},
        "pool": {"workers": cpu.workers, "host_works": cpu.host_works, "expert_GBps": pool_gbs,
                 "drain_ms_per_layer": round((st1["drain"] - st0["drain"]) / (args.steps * layers), 4)},
        "roofline": None, "cpu_baseline": None,
    }))
    cpu.close()
    return 0


# ---------------------------------------------------------------- profile summaries (no GPU work)
MARK_STEP, MARK_DOM = "FillFunctor<short>", "FillFunctor<signed char>"


def _short_kernel(name: str) -> str:
    import re

    m = re.search(r"(\w+_kernel<[^>]*>|\w+_kernel\b|__amd_rocclr_\w+)", name)
    return m.group(1) if m else name[:60]


def summarize_trace(path: str, steps: int) -> str:
    """Markdown: per kernel and launch shape, the dispatches between each pair of --trace-marks marks (the timed steps,
    then the dominant-launch loop), with each region's span on the GPU clock."""
    import csv
    import statistics

    rows = sorted(csv.DictReader(open(path)), key=lambda r: int(r["Start_Timestamp"]))
    out = []
    for label, mark in (("timed steps", MARK_STEP), ("dominant-launch loop", MARK_DOM)):
        at = [i for i, r in enumerate(rows) if mark in r["Kernel_Name"]]
        if len(at) < 2:
            out.append(f"{label}: no marks in {path}")
            continue
        sel = rows[at[0] + 1: at[1]]
        span = (int(sel[-1]["End_Timestamp"]) - int(sel[0]["Start_Timestamp"])) / 1e3
        per = {}
        for r in sel:
            g = int(r["Grid_Size_X"]) * int(r["Grid_Size_Y"]) * int(r["Grid_Size_Z"])
            wg = int(r["Workgroup_Size_X"]) * int(r["Workgroup_Size_Y"]) * int(r["Workgroup_Size_Z"])
            key = (_short_kernel(r["Kernel_Name"]), g // max(wg, 1), wg)
            per.setdefault(key, []).append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
        busy = sum(sum(v) for v in per.values())
        out.append(f"**{label}**: {len(sel)} dispatches over {span:.1f} us of GPU time (first start to last end)"
                   + (f", {span / steps:.1f} us per step" if label == "timed steps" else "") + "; kernels busy "
                   f"{busy:.1f} us")
        out.append("")
        out.append("| kernel | blocks x threads | calls | avg us | median us | min us | max us | % of span |")
        out.append("|---|---|---|---|---|---|---|---|")
        for k, v in sorted(per.items(), key=lambda kv: -sum(kv[1])):
            out.append(f"| {k[0]} | {k[1]} x {k[2]} | {len(v)} | {statistics.mean(v):.2f} | "
                       f"{statistics.median(v):.2f} | {min(v):.2f} | {max(v):.2f} | {100 * sum(v) / span:.1f} |")
        out.append("")
    return "\n".join(out)


# the dominant launch of each configuration by kernel (per layer for the decode configurations: both launches); where
# one kernel runs at two grid sizes (the prompt products of the routed and the shared experts) the larger grid's
DOMINANT = {"decode": ("layer_gu1s_kernel<18>", "layer_down_kernel<21, 1, 3>"),
            "plumb": ("layer_gu1s_kernel<8>", "layer_down_kernel<8, 4, 3>"),
            "verify": ("layer_gut_kernel<18, 1>", "layer_down_kernel<21, 4, 5>"),
            "prefill": ("mmq_f16_kernel<12, 4, true, 1>",), "prefill_long": ("mmq_f16_kernel<18, 8, true, 1>",)}


def summarize_pmc(args, fetch_csv: str, write_csv: str) -> str:
    """HBM bytes per dominant launch: each counter's KiB per dispatch, averaged per kernel, scaled by what the same
    counter read for the copy probe (--copy-probe-mib: a known number of bytes in and out)."""
    import csv

    mib = args.copy_probe_mib or 1024
    vals = {}
    for ctr, path in (("FETCH_SIZE", fetch_csv), ("WRITE_SIZE", write_csv)):
        per = {}
        for r in csv.DictReader(open(path)):
            if r.get("Counter_Name", ctr) != ctr:
                continue
            name = r["Kernel_Name"]
            if "elementwise" in name and "Mul" not in name:
                continue  # torch's fills of the probe's buffers
            blocks = int(r["Grid_Size"]) // max(1, int(r["Workgroup_Size"]))
            key = ("copy probe", 0) if "elementwise" in name else (_short_kernel(name), blocks)
            per.setdefault(key, []).append(float(r["Counter_Value"]))
        vals[ctr] = per
    probe = {c: max(vals[c].get(("copy probe", 0), [0.0])) for c in vals}
    fac = {c: probe[c] / (mib * 1024.0) for c in probe}  # counter KiB per true KiB
    lines = [f"copy probe ({mib} MiB in, {mib} MiB out): FETCH_SIZE {probe['FETCH_SIZE']:.1f} KiB, WRITE_SIZE "
             f"{probe['WRITE_SIZE']:.1f} KiB -> factors {fac['FETCH_SIZE']:.3f} (fetch), {fac['WRITE_SIZE']:.3f} (write)",
             "", "| kernel | blocks | dispatches | FETCH_SIZE KiB / dispatch | WRITE_SIZE KiB / dispatch | bytes / dispatch |",
             "|---|---|---|---|---|---|"]
    dom = DOMINANT.get(args.config, ())
    per_bytes = {}
    for k in sorted(set(vals["FETCH_SIZE"]) | set(vals["WRITE_SIZE"])):
        if k[0] == "copy probe":
            continue
        f, w = vals["FETCH_SIZE"].get(k, [0.0]), vals["WRITE_SIZE"].get(k, [0.0])
        fa, wa = sum(f) / len(f), sum(w) / len(w)
        b = (fa / fac["FETCH_SIZE"] + wa / fac["WRITE_SIZE"]) * 1024
        lines.append(f"| {k[0]} | {k[1]} | {len(f)} | {fa:.1f} | {wa:.1f} | {b:,.0f} |")
        per_bytes[k] = b
    total = 0.0
    for d in dom:  # each dominant kernel at its largest grid
        grids = [k for k in per_bytes if k[0] == d]
        if grids:
            total += per_bytes[max(grids, key=lambda k: k[1])]
    lines += ["", f"dominant launch ({' + '.join(dom)}): {total:,.0f} bytes"]
    if args.traffic_json:
        f = Path(args.traffic_json)
        rec = json.loads(f.read_text()) if f.exists() else {}
        rec[args.config] = {"hbm_bytes_per_launch": int(round(total)), "launch": " + ".join(dom),
                            "fetch_factor": round(fac["FETCH_SIZE"], 4), "write_factor": round(fac["WRITE_SIZE"], 4),
                            "source": args.pmc_source}
        f.write_text(json.dumps(rec, indent=1) + "\n")
    return "\n".join(lines)


def measured_traffic(config: str):
    """HBM bytes per dominant launch from two rocprofv3 --pmc passes (FETCH_SIZE, WRITE_SIZE), each scaled by what the
    same counter read for a copy kernel of known size; recorded in profiles/traffic.json.  None when not measured."""
    f = ROOT / "profiles" / "traffic.json"
    if not f.exists():
        return None
    rec = json.loads(f.read_text()).get(config)
    return None if rec is None else rec.get("hbm_bytes_per_launch")


# the CPU share of one GPU on the GPU boxes this bench runs on (their harness limits a job to 16 host threads per GPU)
CPU_SHARE = 16


def cpu_topology():
    """This host's CPUs: model name, logical and physical counts (whole machine and this process's affinity mask), and
    one logical CPU per physical core of the mask (sysfs topology), in CPU order."""
    model = "unknown"
    try:
        for ln in open("/proc/cpuinfo"):
            if ln.startswith("model name"):
                model = ln.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    logical_all = os.cpu_count() or 1
    mask = sorted(os.sched_getaffinity(0))
    seen, cores = set(), []
    phys_all = set()
    for c in range(logical_all):
        try:
            core = int(open(f"/sys/devices/system/cpu/cpu{c}/topology/core_id").read())
            pkg = int(open(f"/sys/devices/system/cpu/cpu{c}/topology/physical_package_id").read())
        except (OSError, ValueError):
            continue
        phys_all.add((pkg, core))
        if c in mask and (pkg, core) not in seen:
            seen.add((pkg, core))
            cores.append(c)
    if not cores:
        cores = mask
    return {"model": model, "logical": logical_all, "physical": len(phys_all) or None,
            "mask_logical": len(mask), "mask_physical": len(cores), "cores": cores}


def cpu_baseline(args, L, pool, orders, shared_idx, ids_host, mls, x0, sg, layers, T, k, shared, seconds=None):
    """The reference CPU path (its own AVX-512/AVX2 expert rows, oracle/_ref: Q8_K activations) on this host, one
    pinned worker per physical core of the process's CPU mask (at most the GPU's host share), over the same routing
    and weights (each layer's used experts at distinct host addresses), timed for about cpu_seconds.  The reference's
    pool takes at most 8 tokens per expert call, so a prompt chunk is run as consecutive 8-token pieces (the first
    64 tokens)."""
    import oracle as O

    seconds = args.cpu_seconds if seconds is None else seconds
    topo = cpu_topology()
    threads = max(1, min(CPU_SHARE, topo["mask_physical"]))
    cpus = np.asarray(topo["cores"][:threads], np.int32)
    stride = pool.shape[1]
    Tc = min(T, 8)
    pieces = [(t0, min(T, t0 + Tc)) for t0 in range(0, min(T, 64), Tc)]
    if not O.ref_available():
        per = []
        for l in range(layers):
            used = np.unique(ids_host[l][:Tc])
            blobs = [pool[orders[l][e]] for e in used] + ([pool[shared_idx[l]]] if shared else [])
            per.append((np.stack(blobs), None))
        return cpu_port(L, per, Tc, k, shared, seconds)
    R = O.ref()
    wts_all = [ml.wts.cpu().numpy() for ml in mls]
    runs = []
    for a, b in pieces:
        nt = b - a
        per = []
        for l in range(layers):  # only the experts this piece uses, remapped to 0..u-1, plus the layer's shared blob
            ids_l = ids_host[l][a:b]
            used = np.unique(ids_l)
            remap = {int(e): i for i, e in enumerate(used)}
            blobs = [pool[orders[l][e]] for e in used] + ([pool[shared_idx[l]]] if shared else [])
            per.append((np.stack(blobs), np.vectorize(remap.get)(ids_l).astype(np.int32), len(used)))
        umax = max(p[0].shape[0] for p in per)
        host = np.zeros((layers, umax, stride), np.uint8)
        ids = np.zeros((layers, nt, k), np.int32)
        for l, (bl, i, _) in enumerate(per):
            host[l, : bl.shape[0]] = bl
            if shared:  # ref_moe_decode reads layer l's shared blob at shared + l * layer_stride: every layer's last slot
                host[l, umax - 1] = bl[-1]
            ids[l] = i
        wts = np.ascontiguousarray(np.stack([w[a:b] for w in wts_all]).astype(np.float32))
        sgs = np.ascontiguousarray((1 / (1 + np.exp(-sg[:, a:b].astype(np.float64)))).astype(np.float32))
        shared_ptr = host.ctypes.data + (umax - 1) * stride if shared else None
        x = np.ascontiguousarray(x0[a:b])
        # algorithmic bytes of one pass: every layer's distinct experts (and the shared one) once, x in and out
        nbytes = sum((u + int(shared)) * L.bytes + 2 * nt * L.n_embd * 4 for _, _, u in per)
        runs.append((nt, host, ids, wts, sgs, shared_ptr, x, nbytes))

    def one_pass(iters):
        tot = 0.0
        for nt, host, ids, wts, sgs, shared_ptr, x, _ in runs:
            tot += R.ref_moe_decode(L.gu_type, L.d_type, L.n_embd, L.n_ff, nt, k, layers, ids.ctypes.data,
                                    wts.ctypes.data, host.ctypes.data, stride, host.shape[1] * stride, shared_ptr,
                                    sgs.ctypes.data, x.ctypes.data, threads, iters, cpus.ctypes.data) * layers
        return tot  # seconds per pass over every piece, each the median of its iterations

    first = one_pass(2)
    iters = int(max(3, min(5000, seconds / max(first, 1e-6))))
    sec = one_pass(iters)
    toks = sum(r[0] for r in runs) * layers
    nbytes = sum(r[7] for r in runs)
    isa = R.ref_isa()
    return {"value": round(toks / sec, 2), "unit": "MoE-layer tokens/s", "cores": threads, "kind": "reference",
            "GBps": round(nbytes / sec / 1e9, 2),
            "layer_us": round(sec / (len(runs) * layers) * 1e6, 2),
            "cpu_model": topo["model"],
            "host_cpus": {"logical": topo["logical"], "physical": topo["physical"],
                          "mask_logical": topo["mask_logical"], "mask_physical": topo["mask_physical"]},
            "isa": {512: "AVX-512 VNNI (iq512 rows)", 256: "AVX2 (iq256 rows)"}.get(isa, "scalar") + ", kq256 rows",
            "threads_note": (f"one worker per physical core of the process mask, pinned, the caller working too; "
                             f"capped at {CPU_SHARE}, the host share of one GPU on the GPU box"
                             if topo["mask_physical"] > CPU_SHARE else
                             "one worker per physical core of the process mask, pinned, the caller working too"),
            "sample": f"{iters} passes x {layers} layers over {len(runs)} piece(s) of {Tc} token(s), median pass; "
                      f"reference CPU expert rows, " + ("Q8_0" if L.gu_type == 8 else "Q8_K") + " activations"
                      + (f" (the first {sum(r[0] for r in runs)} of the {T}-token chunk)" if T > Tc else "")}


def cpu_port(L, per, T, k, shared, seconds):
    """Fallback where oracle/_ref was not built: the oracle's own C layer (reference CPU arithmetic, ggml mode) over
    each layer's used experts, routed by its own synthetic logits; single-threaded loops with OpenMP rows."""
    import oracle as O

    Lo = O.layout(L.gu_type, L.d_type, L.n_embd, L.n_ff)
    rng = np.random.default_rng(0)
    x = rng.normal(0, 1, (T, L.n_embd)).astype(np.float32)
    n, t0 = 0, time.time()
    while time.time() - t0 < seconds or n < 3:
        blobs, _ = per[n % len(per)]
        used = blobs.shape[0] - int(shared)
        logits = rng.normal(0, 1, (T, max(used, k))).astype(np.float32)
        O.moe_layer(1, Lo, x, logits, k, blobs[:max(used, k)] if used >= k else np.resize(blobs, (k, blobs.shape[1])),
                    blobs.shape[1], blobs[-1] if shared else None, np.zeros(T, np.float32) if shared else None)
        n += 1
    per_layer = (time.time() - t0) / n
    return {"value": round(T / per_layer, 2), "unit": "MoE-layer tokens/s", "cores": O.orc().orc_threads(),
            "kind": "port", "sample": f"{n} layers of the oracle's C restatement (ggml activations)"}


if __name__ == "__main__":
    sys.exit(main())
