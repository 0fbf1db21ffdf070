"""The hybrid CPU/GPU decode layer (tinystrata_amd.pool.HybridMoELayer; reference moe_hybrid_gpu / moe_hybrid_cpu,
src/qwen35/q36_engine.cu:3052-3209) against the all-GPU layer and the oracle (marked gpu).

Bars: the expert ids identical; with every expert resident the output bit-identical to MoELayer's kernel-by-kernel
decode path (the same kernels); otherwise within 1e-3 relative L2 of the oracle's layer in Q8_1 mode (a CPU row and
a GPU row accumulate their floats in different orders, so an h code at a rounding boundary may differ) and of the
all-GPU layer; the resident grouping and the merge checked entry by entry."""
import numpy as np
import pytest
import torch

import oracle as O
from tinystrata_amd import moe, ops
from tinystrata_amd._lib import IQ3_S, IQ3_XXS, Q4_K, Q8_0
from tinystrata_amd.pool import ExpertPool, HybridMoELayer

from gpu_util import dev, host, pool, rel_l2

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("gu,d,T,every", [(IQ3_XXS, IQ3_S, 1, 2), (IQ3_XXS, IQ3_S, 4, 3), (IQ3_XXS, IQ3_S, 4, 0),
                                          (IQ3_XXS, IQ3_S, 1, 1), (Q8_0, Q8_0, 2, 2), (Q4_K, Q4_K, 8, 2)])
def test_hybrid_layer(gu, d, T, every):
    N, FF, E, k, distinct = 2048, 512, 64, 8, 6
    print(f"hybrid layer types {gu}/{d} T={T} resident every {every}", flush=True)
    L = ops.native_expert_layout(gu, d, N, FF)
    p = pool(gu, d, N, FF, distinct, 0)
    order = (np.arange(E) * 5 + 3) % (distinct - 1)
    host_blobs = np.ascontiguousarray(p[order])
    W = moe.weights_from_pool(L, dev(p), E, order, distinct - 1)
    resident = np.arange(0, E, every) if every else np.zeros(0, np.int64)
    rng = np.random.default_rng(T + every)
    x = rng.normal(0, 1, (T, N)).astype(np.float32)
    logits = rng.normal(0, 1, (T, E)).astype(np.float32)
    sgate = rng.normal(0, 1, T).astype(np.float32)
    y0 = rng.normal(0, 1, (T, N)).astype(np.float32)
    with ExpertPool(4, pin=False) as cpu:
        hy = HybridMoELayer(W, host_blobs, resident, k, T, torch.device("cuda"), cpu)
        ys = []
        for _ in range(2):  # the second call reuses every buffer
            y = dev(y0.copy())
            hy(dev(x), dev(logits), dev(sgate), y)
            torch.cuda.synchronize()
            ys.append(host(y))
        assert np.array_equal(ys[0], ys[1])
        ids = host(hy.ids)
        missed = ~np.isin(ids.ravel(), resident)
        assert hy.n_miss == int(missed.sum())
    gl = moe.MoELayer(W, k, T, torch.device("cuda"), fused=False)
    yg = dev(y0.copy())
    gl(dev(x), dev(logits), dev(sgate), yg)
    assert np.array_equal(host(gl.ids), ids)
    if every == 1:
        assert np.array_equal(ys[0], host(yg))
    else:
        assert rel_l2(ys[0] - y0, host(yg) - y0) < 1e-3
    yo, io, _ = O.moe_layer(0, O.layout(gu, d, N, FF), x, logits, k, host_blobs, W.stride, shared=p[distinct - 1],
                            sgate=sgate)
    assert np.array_equal(io, ids)
    assert rel_l2(ys[0] - y0, yo) < 1e-3


def test_group_resident_and_merge():
    E, k, T, n = 40, 8, 3, 96
    rng = np.random.default_rng(1)
    ids = np.stack([rng.permutation(E)[:k] for _ in range(T)]).astype(np.int32)
    slot_of = np.where(np.arange(E) % 2 == 1, np.arange(E) // 2, -1).astype(np.int32)
    base, stride = 1 << 20, 4096
    cap = min(T * k, E)
    bufs = (torch.zeros(cap, dtype=torch.int64, device="cuda"), torch.zeros(cap + 1, dtype=torch.int32, device="cuda"),
            torch.zeros(1, dtype=torch.int32, device="cuda"), torch.full((T * k,), -7, dtype=torch.int32, device="cuda"),
            torch.full((T * k,), -7, dtype=torch.int32, device="cuda"))
    gp, gs, ng, ed, et = ops.group_resident(dev(ids), k, E, dev(slot_of), base, stride, bufs)
    flat = ids.ravel()
    res = [e for e in range(T * k) if slot_of[flat[e]] >= 0]
    experts = sorted({int(flat[e]) for e in res})
    assert int(host(ng)[0]) == len(experts)
    assert list(host(gp)[: len(experts)]) == [base + int(slot_of[x]) * stride for x in experts]
    want = [e for x in experts for e in res if flat[e] == x]
    assert list(host(ed)[: len(want)]) == want and list(host(et)[: len(want)]) == [e // k for e in want]
    assert list(host(gs)[: len(experts) + 1]) == list(np.cumsum([0] + [int((flat[res] == x).sum()) for x in experts]))
    parts = rng.normal(0, 1, (T * k, n)).astype(np.float32)
    rows = rng.normal(0, 1, (T * k, n)).astype(np.float32)
    miss = np.full(T * k, -1, np.int32)
    miss[[0, 5, 9, 23]] = [3, 0, 2, 1]
    dp = dev(parts)
    ops.merge_rows(dp, dev(rows), dev(miss))
    want = parts.copy()
    for e in range(T * k):
        if miss[e] >= 0:
            want[e] = rows[miss[e]]
    assert np.array_equal(host(dp), want)
