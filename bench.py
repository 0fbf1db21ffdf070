"""bench.py - TinyStrata's MoE expert matmul on one MI355X: the decode MoE layer stack.

    python bench.py [--steps K] [--warmup W] [--config decode|verify|plumb] [--eager] [--no-cpu]

A step is one token through 40 MoE layers with distinct weights (so the experts stream from HBM): per layer the
router, the grouping, the Q8_1 activations, the grouped IQ3_XXS/IQ3_S experts, the shared expert and the weighted
combine, each layer's output feeding the next (x <- x + moe(x)).  Inputs are synthetic (N(0,0.02) weights quantized
by this library, N(0,1) activations and router logits) and resident in HBM before the timed region.
Prints one JSON line (the driver's contract) with the roofline of the dominant launch and the reference CPU path
timed on this host beside it.
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

CONFIGS = {
    # name: (gu, d, N, FF, E, k, shared, T, layers, description)
    "decode": (18, 21, 2048, 512, 256, 8, True, 1, 40, "configs[1]: decode, 256 experts top-8 + shared, IQ3_XXS/IQ3_S"),
    "verify": (18, 21, 2048, 512, 256, 8, True, 4, 40, "configs[2]: speculative verify M=4, correlated routing"),
    "plumb": (8, 8, 2048, 768, 128, 8, False, 1, 40, "configs[0]: decode, 128 experts top-8, Q8_0"),
}


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="decode", choices=sorted(CONFIGS))
    ap.add_argument("--eager", action="store_true", help="launch each step eagerly instead of replaying a HIP graph")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build runs on one GPU; --gpus N > 1 is not supported (see DESIGN.md for the sharding plan)",
              file=sys.stderr)
        return 2

    import torch

    from tinystrata_amd import _lib, moe, ops

    gu, d, N, FF, E, k, shared, T, layers, desc = CONFIGS[args.config]
    dev = torch.device("cuda:0")
    _lib.check(_lib.lib().tsx_moe_init(0), "tsx_moe_init")
    L = ops.native_expert_layout(gu, d, N, FF)
    stride = moe.blob_stride(L)

    # ---------------------------------------------------------------- synthetic weights, resident in HBM
    t0 = time.time()
    distinct = 24
    pool = moe.synthetic_pool(L, distinct, seed=1234)
    pool_dev = torch.from_numpy(pool).to(dev)
    log(f"bench: {distinct} distinct experts quantized in {time.time() - t0:.1f}s; "
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
    if args.config == "verify":
        z = rng.normal(0, 1, (layers, 1, E))
        logits = (z + 0.5 * rng.normal(0, 1, (layers, T, E))).astype(np.float32)
    else:
        logits = rng.normal(0, 1, (layers, T, E)).astype(np.float32)
    sg = rng.normal(0, 1, (layers, T)).astype(np.float32)
    x0_d = torch.from_numpy(x0).to(dev)
    x = torch.empty_like(x0_d)
    logits_d = torch.from_numpy(logits).to(dev)
    sg_d = torch.from_numpy(sg).to(dev)
    mls = [moe.MoELayer(Ws[l], k, T, dev) for l in range(layers)]

    def step():
        x.copy_(x0_d)
        for l in range(layers):
            mls[l](x, logits_d[l], sg_d[l] if shared else None, x)

    for _ in range(args.warmup):
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
        for _ in range(args.warmup):
            graph.replay()
    torch.cuda.synchronize()

    # ---------------------------------------------------------------- timed region
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for _ in range(args.steps):
        graph.replay() if graph is not None else step()
    end.record()
    torch.cuda.synchronize()
    ms_step = start.elapsed_time(end) / args.steps
    value = layers * T / (ms_step / 1e3)

    # distinct experts per layer (the bytes the layer must read)
    ids_host = [ml.ids.cpu().numpy() for ml in mls]
    distinct_per_layer = [len(np.unique(i)) for i in ids_host]
    blob = L.bytes
    layer_bytes = [(n + int(shared)) * blob + 2 * T * N * 4 for n in distinct_per_layer]
    layer_ops = 2 * T * (k + int(shared)) * (3 * N * FF)

    # ---------------------------------------------------------------- the dominant launch: the grouped experts
    # back to back over the 40 layers' weights, HIP events on the stream they run on (torch's current stream)
    reps = max(3, args.steps // 10)
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    ev0.record()
    for _ in range(reps):
        for ml in mls:
            gp, gs, ng, ed, et = ml.grp
            ops.native_expert_grouped(L, gp, gs, ng, ed, et, ml.cap_groups, ml.n_ent, ml.xq, ml.scratch, ml.parts)
    ev1.record()
    torch.cuda.synchronize()
    dom_ms = ev0.elapsed_time(ev1) / (reps * layers)
    dom_bytes = float(np.mean([n * blob + T * N // 32 * 36 + T * k * N * 4 for n in distinct_per_layer]))
    achieved = dom_bytes / (dom_ms / 1e3) / 1e9

    # ---------------------------------------------------------------- the reference CPU path on this host
    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(args, L, pool, orders, shared_idx, ids_host, mls, x0, sg, layers, T, k, shared)

    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "MoE-layer tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": {
            "workload": f"{args.config}: {desc}",
            "tokens": T, "layers": layers, "hidden": N, "expert_ff": FF, "experts": E, "top_k": k,
            "shared_expert": shared, "graph": graph is not None,
            "layer_us": round(ms_step * 1e3 / layers, 3),
            "layer_hbm_GBps": round(float(np.mean(layer_bytes)) / (ms_step / layers / 1e3) / 1e9, 1),
            "layer_hbm_frac": round(float(np.mean(layer_bytes)) / (ms_step / layers / 1e3) / 1e9 / HBM_PEAK_GBS, 4),
            "layer_bytes": int(np.mean(layer_bytes)),
            "distinct_experts_per_layer": float(np.mean(distinct_per_layer)),
            "layer_int8_ops": layer_ops,
        },
        "roofline": {
            "kernel": "native_expert_grouped (gate/up, SwiGLU+Q8_1, down) per layer",
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": None,
            "launch_us": round(dom_ms * 1e3, 3),
            "bytes_per_launch": int(dom_bytes),
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


def cpu_baseline(args, L, pool, orders, shared_idx, ids_host, mls, x0, sg, layers, T, k, shared):
    """The reference CPU path (its own AVX-512/AVX2 expert rows, oracle/_ref) on this host's cores, over the same
    routing and weights (each layer's used experts at distinct host addresses), timed for about cpu_seconds."""
    import oracle as O

    threads = max(1, min(16, os.cpu_count() or 1))
    stride = pool.shape[1]
    # per layer: only the experts it uses, remapped to 0..u-1, plus its shared blob
    per = []
    for l in range(layers):
        used = np.unique(ids_host[l])
        remap = {int(e): i for i, e in enumerate(used)}
        blobs = [pool[orders[l][e]] for e in used]
        if shared:
            blobs.append(pool[shared_idx[l]])
        per.append((np.stack(blobs), np.vectorize(remap.get)(ids_host[l]).astype(np.int32)))
    umax = max(b.shape[0] for b, _ in per)
    layer_stride = umax * stride
    host = np.zeros((layers, umax, stride), np.uint8)
    ids = np.zeros((layers, T, k), np.int32)
    for l, (b, i) in enumerate(per):
        host[l, : b.shape[0]] = b
        ids[l] = i
    wts = np.stack([ml.wts.cpu().numpy() for ml in mls]).astype(np.float32)
    sgs = (1 / (1 + np.exp(-sg.astype(np.float64)))).astype(np.float32)
    if not O.ref_available():
        return cpu_port(L, per, T, k, shared, args.cpu_seconds)
    shared_ptr = None
    if shared:  # ref_moe_decode reads layer l's shared blob at shared + l * layer_stride: the last slot of every layer
        for l in range(layers):
            host[l, umax - 1] = per[l][0][-1]
        shared_ptr = host.ctypes.data + (umax - 1) * stride
    x = x0.copy()
    R = O.ref()
    one = R.ref_moe_decode(L.gu_type, L.d_type, L.n_embd, L.n_ff, T, k, layers, ids.ctypes.data, wts.ctypes.data,
                           host.ctypes.data, stride, layer_stride, shared_ptr, sgs.ctypes.data, x.ctypes.data,
                           threads, 2)
    iters = int(max(3, min(5000, args.cpu_seconds / max(one * layers, 1e-6))))
    x = x0.copy()
    per_layer = R.ref_moe_decode(L.gu_type, L.d_type, L.n_embd, L.n_ff, T, k, layers, ids.ctypes.data,
                                 wts.ctypes.data, host.ctypes.data, stride, layer_stride, shared_ptr, sgs.ctypes.data,
                                 x.ctypes.data, threads, iters)
    isa = R.ref_isa()
    return {"value": round(T / per_layer, 2), "unit": "MoE-layer tokens/s", "cores": threads, "kind": "reference",
            "sample": f"{iters} passes x {layers} layers, median pass; reference iq{isa}/kq256 rows, "
                      f"Q8_K activations, {threads} pinned threads, {T} token(s)",
            "layer_us": round(per_layer * 1e6, 2)}


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
