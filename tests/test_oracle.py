"""Pins the CPU oracle (oracle/oracle.c) before it is trusted as the GPU's checker.

  * golden fixtures made by the reference's own compiled CPU kernels (tests/golden/make_golden.py): Q8_K bytes,
    row outputs in the reference CPU arithmetic (ggml mode), SwiGLU rows, and single-sub-block probes that expose
    the integer sub-block sums times the format's sub-block scale exactly;
  * oracle/_ref directly on fresh random inputs, where it was built;
  * what the mathematics fixes: the Q8_1 block (closed form, special blocks), integer sums against the dequantized
    values, the router's ties / NaN / renormalization floor, the stable sort against numpy's, the combine's order.
"""
from pathlib import Path

import numpy as np
import pytest

import oracle as O

GOLD = Path(__file__).resolve().parent / "golden"
TYPES = (O.IQ3_XXS, O.IQ3_S, O.Q4_K, O.Q8_0)
K_FACTOR = {O.IQ3_XXS: 0.25, O.IQ3_S: 1.0, O.Q4_K: 1.0, O.Q8_0: 1.0}


# ------------------------------------------------------------------ Q8_K and Q8_0 activations
def test_q8k_matches_reference_bytes():
    g = np.load(GOLD / "golden_q8k.npz")
    got, ref = O.quantize_q8_K(g["x"]).reshape(-1, 292), g["q"].reshape(-1, 292)
    zero = got[:, :4].view(np.float32)[:, 0] == 0
    assert zero.sum() == 1                                   # the fixture's all-zero block
    # an all-zero block: the reference writes d and qs but leaves bsums unwritten (here they are zeroed)
    assert (got[:, :260] == ref[:, :260]).all() and (got[~zero] == ref[~zero]).all()


def test_q8k_zero_and_outlier_blocks():
    x = np.zeros(512, np.float32)
    x[256 + 3] = -5.0
    q = O.quantize_q8_K(x).reshape(2, 292)
    assert np.frombuffer(q[0, :4].tobytes(), np.float32)[0] == 0.0 and (q[0, 4:260] == 0).all()
    codes = q[1, 4:260].view(np.int8)
    assert codes[3] == -127 and (np.delete(codes, 3) == 0).all()       # the max maps to -127 (iscale = -127/max)
    assert np.isclose(np.frombuffer(q[1, :4].tobytes(), np.float32)[0], 5.0 / 127.0)
    assert np.frombuffer(q[1, 260:262].tobytes(), np.int16)[0] == -127


def test_q8_0_closed_form():
    rng = np.random.default_rng(3)
    x = rng.normal(0, 1, 64).astype(np.float32)
    q = O.quantize_q8_0(x).reshape(2, 34)
    for b in range(2):
        d = np.abs(x[32 * b:32 * b + 32]).max() / 127
        assert q[b, :2].view(np.float16)[0] == np.float16(d)
        exp = np.round(x[32 * b:32 * b + 32].astype(np.float64) * np.float32(1.0 / np.float32(d)))
        assert (q[b, 2:].view(np.int8) == exp.astype(np.int8)).all()


# ------------------------------------------------------------------ Q8_1
def test_q8_1_closed_form():
    rng = np.random.default_rng(4)
    x = rng.normal(0, 2, (512, 2048)).astype(np.float32)
    d, s, codes = O.q8_1_split(O.quantize_q8_1(x))
    xb = x.reshape(-1, 32)
    amax = np.abs(xb).max(1)
    dd = (amax / np.float32(127)).astype(np.float32)
    assert (d == dd.astype(np.float16).astype(np.float32)).all()
    # roundf: half away from zero, on x / d in float
    r = xb / dd[:, None]
    exp = np.sign(r) * np.floor(np.abs(r) + 0.5)
    assert (codes == np.clip(exp, -127, 127)).all()
    # s, exactly: the fp16 of the 32 raw values' float sum in the warp's xor-tree order (q8_1_store,
    # src/kernels/cuda/iq_kernels.cu:1469-1474: sum += shfl_xor(sum, o) for o = 16 .. 1), clamped to the largest half
    v, lanes = xb.copy(), np.arange(32)
    for o in (16, 8, 4, 2, 1):
        v = (v + v[:, lanes ^ o]).astype(np.float32)
    assert (v == v[:, :1]).all()  # every lane of the tree ends with the same bits
    tree = np.clip(v[:, 0], -65504, 65504).astype(np.float16).astype(np.float32)
    assert (s == tree).all()
    # the check tells summation orders apart: a left-to-right float sum rounds to another half in some blocks
    seq = np.zeros(len(xb), np.float32)
    for j in range(32):
        seq = (seq + xb[:, j]).astype(np.float32)
    assert (seq.astype(np.float16).astype(np.float32) != tree).sum() > 0


def test_q8_1_special_blocks():
    x = np.zeros((1, 128), np.float32)
    x[0, 32:64] = 1.0                   # all equal: codes 127
    x[0, 64] = 1e9                      # amax / 127 beyond fp16: d and s held to 65504
    x[0, 96:128] = np.linspace(-1, 1, 32)
    d, s, codes = O.q8_1_split(O.quantize_q8_1(x))
    assert d[0] == 0 and (codes[0] == 0).all() and s[0] == 0          # zero block
    assert (codes[1] == 127).all() and d[1] == np.float16(1 / 127)
    assert d[2] == 65504.0 and s[2] == 65504.0 and codes[2][0] == 127
    assert codes[3][0] == -127 and codes[3][-1] == 127


# ------------------------------------------------------------------ rows against the reference kernels
@pytest.mark.parametrize("t", TYPES)
@pytest.mark.parametrize("n", [256, 2048])
@pytest.mark.parametrize("nt", [1, 4])
def test_ggml_rows_match_reference(t, n, nt):
    g = np.load(GOLD / "golden_rows.npz")
    key = f"t{t}_n{n}_nt{nt}"
    w, a, y = g[key + "_w"], g[key + "_a"], g[key + "_y"]
    rows = y.shape[1]
    got = O.mmvq_ggml(t, w[:rows], n, rows, a, nt)
    # same integer sums, same scales: only the order of the float additions differs
    np.testing.assert_allclose(got, y, rtol=2e-6, atol=2e-6 * np.abs(y).max())


@pytest.mark.parametrize("t", TYPES)
def test_swiglu_rows_match_reference(t):
    g = np.load(GOLD / "golden_rows.npz")
    key = f"t{t}_n2048_nt4"
    w, a, ff = g[key + "_w"], g[key + "_a"], g[key + "_ff"]
    rows = ff.shape[1]
    gate = O.mmvq_ggml(t, w[:rows], 2048, rows, a, 4)
    up = O.mmvq_ggml(t, w[rows:2 * rows], 2048, rows, a, 4)
    h = (gate / (1 + np.exp(-gate))) * up
    np.testing.assert_allclose(h, ff, rtol=1e-5, atol=1e-5 * np.abs(ff).max())


@pytest.mark.parametrize("t", TYPES)
def test_subblock_sums_match_reference_probes(t):
    """Reference output for a probe with only sub-block j non-zero = K * iscale_j * S_j (exact in float)."""
    g = np.load(GOLD / "golden_sums.npz")
    w, codes, out = g[f"t{t}_w"], g[f"t{t}_codes"], g[f"t{t}_out"]
    rows = w.shape[0]
    xq = np.zeros((8, 8, 36), np.uint8)          # 8 probes, 8 Q8_1 blocks each, d = 1
    for j in range(8):
        xq[j, :, 0:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
        xq[j, j, 4:] = codes[j].view(np.uint8)
    sums, qsums = O.subblock_sums(t, w, 256, rows, xq.reshape(8, -1), 8)
    deq = np.stack([O.dequantize(t, w[r], 256) for r in range(rows)])      # d = 1, dmin = 0: value = iscale * w_int
    for j in range(8):
        S = sums[:, j, j].astype(np.int64)
        assert (sums[:, j, np.arange(8) != j] == 0).all()
        # the oracle's decode of the sub-block scale times its integer sum equals the reference's output exactly
        w_int_scaled = deq[:, 32 * j:32 * j + 32].astype(np.float64)
        dot = (w_int_scaled * codes[j].astype(np.float64)).sum(1)
        assert (dot == out[j].astype(np.float64)).all(), (t, j)
        # S itself divides that: S = out / (K * iscale) with iscale = value / w_int on any non-zero weight
        iscale = np.round(np.abs(out[j]) / np.maximum(np.abs(S), 1) / K_FACTOR[t]).astype(np.int64)
        assert (np.abs(S) * iscale * K_FACTOR[t] == np.abs(out[j])).all()
        assert (qsums[:, j, j] == codes[j].astype(np.int32).sum()).all()


@pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built here")
@pytest.mark.parametrize("t", TYPES)
def test_ggml_rows_match_reference_live(t):
    rng = np.random.default_rng(11 + t)
    from tinystrata_amd import ops

    n, rows, nt = 1024, 9, 3
    w = ops.quantize_weights(t, rng.normal(0, 0.02, (rows, n)).astype(np.float32))
    x = rng.normal(0, 1, (nt, n)).astype(np.float32)
    if t == O.Q8_0:
        a = np.concatenate([O.quantize_q8_0(r) for r in x])
    else:
        a = O.quantize_q8_K(x)
        ra = np.empty_like(a)
        O.ref().ref_q8k_quant(x.ctypes.data, ra.ctypes.data, x.size)
        assert (ra == a).all()
    y = np.empty((nt, rows), np.float32)
    assert O.ref().ref_rows(t, w.ctypes.data, n, rows, a.ctypes.data, nt, y.ctypes.data) == 0
    np.testing.assert_allclose(O.mmvq_ggml(t, w, n, rows, a, nt), y, rtol=2e-6, atol=2e-6 * np.abs(y).max())


# ------------------------------------------------------------------ the Q8_1 contract against the dequantized values
@pytest.mark.parametrize("t", TYPES)
def test_q8_1_rows_equal_dequantized_dot(t):
    """Reference bound of tests/native-iq-packed-bytes.cu:153-166: |err| <= 2e-6 * max(1, sum |term|)."""
    rng = np.random.default_rng(5 + t)
    from tinystrata_amd import ops

    n, rows, nt = 512, 7, 3
    w = ops.quantize_weights(t, rng.normal(0, 0.02, (rows, n)).astype(np.float32))
    x = rng.normal(0, 1, (nt, n)).astype(np.float32)
    xq = O.quantize_q8_1(x)
    d, _, codes = O.q8_1_split(xq)
    xv = (codes.astype(np.float64) * d[:, None]).reshape(nt, n)
    deq = np.stack([O.dequantize(t, w[r], n) for r in range(rows)]).astype(np.float64)
    terms = xv[:, None, :] * deq[None, :, :]
    exp, bound = terms.sum(-1), np.abs(terms).sum(-1)
    got = O.mmvq_q8_1(t, w, n, rows, xq, nt)
    assert (np.abs(got - exp) <= 2e-6 * np.maximum(1.0, bound)).all()
    # integer sums: brute force over the dequantized integers
    sums, qsums = O.subblock_sums(t, w, n, rows, xq, nt)
    assert (qsums == codes.reshape(nt, n // 32, 32).sum(-1)[None, :, :]).all()


# ------------------------------------------------------------------ routing
def _np_router(logits, k):
    ids = np.argsort(-logits.astype(np.float64), axis=1, kind="stable")[:, :k]
    p = np.exp(logits.astype(np.float64) - logits.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    sel = np.take_along_axis(p, ids, 1)
    return ids, sel / np.maximum(sel.sum(1, keepdims=True), 6.103515625e-5)


@pytest.mark.parametrize("E,k", [(256, 8), (128, 8), (64, 4)])
def test_router_against_numpy(E, k):
    rng = np.random.default_rng(E)
    logits = rng.normal(0, 1, (16, E)).astype(np.float32)
    ids, w = O.router_topk(logits, k)
    eids, ew = _np_router(logits, k)
    assert (ids == eids).all()
    np.testing.assert_allclose(w, ew, rtol=1e-5)


def test_router_ties_nan_and_floor():
    logits = np.zeros((3, 64), np.float32)
    logits[0, [5, 9, 40]] = 3.0                  # ties resolve to the lower id
    logits[1, :] = -50.0
    logits[1, 7] = np.nan                        # NaN probability never wins
    logits[2, :] = 0.0
    ids, w = O.router_topk(logits, 4)
    assert list(ids[0][:3]) == [5, 9, 40]
    assert 7 not in ids[1]
    assert list(ids[2]) == [0, 1, 2, 3] and np.allclose(w[2], 0.25)
    # renormalization floor: picks summing below 6.1035e-5 are divided by the floor, not by their sum
    tiny = np.full((1, 64), -30.0, np.float32)
    tiny[0, 0] = 30.0
    ids, w = O.router_topk(tiny, 2)
    p = np.exp(np.float64(-60.0)) / (1 + 63 * np.exp(np.float64(-60.0)))
    assert ids[0, 0] == 0 and np.isclose(w[0, 1], p / 1.0, rtol=1e-3)


def test_group_and_sort_against_numpy():
    rng = np.random.default_rng(9)
    ids = rng.integers(0, 32, (12, 4)).astype(np.int32)
    gp, gs, g, ed, et = O.group(ids, 4, 32, blobs=1000, stride=10)
    flat = ids.ravel()
    order = np.argsort(flat, kind="stable")
    used = np.unique(flat)
    assert g == used.size and (gp == 1000 + 10 * used.astype(np.uint64)).all()
    assert (ed == order).all() and (et == order // 4).all()
    assert (np.diff(gs) == np.bincount(flat, minlength=32)[used]).all()
    bounds, ed2, et2, ri, mr = O.route_sort(ids, 4, 32)
    assert (ed2 == order).all() and (ri[order] == np.arange(flat.size)).all()
    assert (bounds == np.concatenate([[0], np.cumsum(np.bincount(flat, minlength=32))])).all()
    assert mr == np.bincount(flat).max()


def test_combine_order_and_shared():
    rng = np.random.default_rng(10)
    T, k, n = 3, 4, 64
    parts = rng.normal(0, 1, (T * k, n)).astype(np.float32)
    wts = rng.random((T, k)).astype(np.float32)
    x = rng.normal(0, 1, (T, n)).astype(np.float32)
    sh = rng.normal(0, 1, (T, n)).astype(np.float32)
    sg = rng.normal(0, 1, T).astype(np.float32)
    got = O.combine(x, parts, wts, k, shared=sh, sgate=sg)
    exp = x.astype(np.float64) + np.einsum("tk,tkn->tn", wts.astype(np.float64), parts.reshape(T, k, n).astype(np.float64))
    exp += (1 / (1 + np.exp(-sg.astype(np.float64))))[:, None] * sh
    np.testing.assert_allclose(got, exp, rtol=1e-5, atol=1e-5)
    prow = np.arange(T * k)[::-1].copy().astype(np.int32)  # rows read through prow
    got2 = O.combine(x, parts[::-1].copy(), wts, k, prow=prow)
    got3 = O.combine(x, parts, wts, k)
    assert (got2 == got3).all()


# ------------------------------------------------------------------ the layer
def test_layer_modes_agree_for_q8_0():
    """Q8_0 experts: Q8_1 and the reference's Q8_0 activations are both per-32 blocks (the same codes up to ties)."""
    from tinystrata_amd import moe, ops

    L = O.layout(O.Q8_0, O.Q8_0, 256, 96)
    Ll = ops.native_expert_layout(O.Q8_0, O.Q8_0, 256, 96)
    pool = moe.synthetic_pool(Ll, 8, seed=2)
    rng = np.random.default_rng(2)
    x = rng.normal(0, 1, (2, 256)).astype(np.float32)
    logits = rng.normal(0, 1, (2, 64)).astype(np.float32)
    blobs = np.tile(pool, (8, 1))
    y0, ids, _ = O.moe_layer(0, L, x, logits, 4, blobs, pool.shape[1])
    y1, ids1, _ = O.moe_layer(1, L, x, logits, 4, blobs, pool.shape[1])
    assert (ids == ids1).all()
    rel = np.linalg.norm(y0 - y1) / np.linalg.norm(y1)
    assert rel < 1e-3, rel


def _ref_act(t: int, v: np.ndarray) -> np.ndarray:
    """The reference CPU's activation for weight type t (IQ3 / Q4_K: Q8_K by q8k_quant_avx2 itself)."""
    v = np.ascontiguousarray(v, np.float32)
    a = np.empty(v.size // 256 * 292, np.uint8)
    O.ref().ref_q8k_quant(v.ctypes.data, a.ctypes.data, v.size)
    return a


def _ref_rows(t, w, n, rows, a):
    w = np.ascontiguousarray(w)
    y = np.empty(rows, np.float32)
    assert O.ref().ref_rows(t, w.ctypes.data, n, rows, a.ctypes.data, 1, y.ctypes.data) == 0
    return y


def _ref_layer(L, x, ids, wts, k, blobs, shared, sgate, plant=None):
    """A MoE layer assembled from the reference's own CPU kernels (oracle/_ref), in the structure of
    src/lfm2/cpu_experts.cpp:145-235: Q8_K of x, the gate/up rows with SwiGLU inside (iq512/kq256_gu_rows), Q8_K of h,
    the down rows, and the combine in pick order (w0 p0, then fma; + sigmoid(sgate) * shared).  `plant` swaps in one
    plausible mistake, to show the comparison catches it."""
    N, FF = int(L.n_embd), int(L.n_ff)
    up, down = int(L.up_off), int(L.down_off)

    def expert(blob, xt):
        a = _ref_act(L.gu_type, xt)
        if plant == "swiglu_order":  # silu(up) * gate, from the reference's plain rows
            g, u = _ref_rows(L.gu_type, blob[:up], N, FF, a), _ref_rows(L.gu_type, blob[up:down], N, FF, a)
            h = ((u / (1 + np.exp(-u.astype(np.float64)))) * g).astype(np.float32)
        else:
            h = np.empty(FF, np.float32)
            assert O.ref().ref_gu_rows(L.gu_type, np.ascontiguousarray(blob).ctypes.data, N, FF, a.ctypes.data, 1,
                                       h.ctypes.data) == 0
        if plant == "h_q8_1":  # the down rows on h's Q8_1 image (the GPU contract's), not the reference CPU's Q8_K
            return O.mmvq_q8_1(L.d_type, np.ascontiguousarray(blob[down:]), FF, N, O.quantize_q8_1(h[None]), 1).ravel()
        return _ref_rows(L.d_type, blob[down:], FF, N, _ref_act(L.d_type, h))

    T = x.shape[0]
    y = np.zeros((T, N), np.float32)
    for t in range(T):
        p = [expert(blobs[ids[t, j]], x[t]) for j in range(k)]
        acc = (wts[t, 0] * p[0]).astype(np.float32)
        for j in range(1, k):  # fmaf in float64: the product is exact, one rounding of the sum to float32
            acc = (wts[t, j].astype(np.float64) * p[j] + acc).astype(np.float32)
        if shared is not None:
            gs = np.float32(1.0) if plant == "shared_gate" else np.float32(1 / (1 + np.exp(-np.float64(sgate[t]))))
            acc = (acc + gs * expert(shared, x[t])).astype(np.float32)
        y[t] = acc
    return y


@pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built here")
@pytest.mark.parametrize("gu,dn,N,FF,shared", [(O.IQ3_XXS, O.IQ3_S, 1024, 512, True),
                                               (O.Q4_K, O.Q4_K, 1024, 256, False)])
def test_layer_composition_against_reference_rows(gu, dn, N, FF, shared):
    """orc_moe_layer in the reference CPU's activation mode against the same layer built from oracle/_ref's own
    kernels: pins the SwiGLU operand order, the quantization of h and the shared expert's gate directly, not only
    through their parts.  The two differ by float summation order alone (rows, SwiGLU), so the bound is 1e-5 relative
    L2; each planted mistake moves the layer by more than 1e-2."""
    from tinystrata_amd import moe, ops

    E, k, T = 16, 4, 3
    Lp = ops.native_expert_layout(gu, dn, N, FF)
    L = O.layout(gu, dn, N, FF)
    pool = moe.synthetic_pool(Lp, 6, seed=9)
    blobs = pool[(np.arange(E) * 5 + 1) % 5]
    sh = pool[5] if shared else None
    rng = np.random.default_rng(17)
    x = rng.normal(0, 1, (T, N)).astype(np.float32)
    logits = rng.normal(0, 1, (T, E)).astype(np.float32)
    sg = rng.normal(0, 1, T).astype(np.float32) if shared else None
    y, ids, w = O.moe_layer(1, L, x, logits, k, blobs, pool.shape[1], sh, sg)
    ref = _ref_layer(Lp, x, ids, w, k, blobs, sh, sg)
    rel = np.linalg.norm(y - ref) / np.linalg.norm(ref)
    assert rel < 1e-5, rel
    for plant in ("swiglu_order", "h_q8_1") + (("shared_gate",) if shared else ()):
        bad = _ref_layer(Lp, x, ids, w, k, blobs, sh, sg, plant=plant)
        assert np.linalg.norm(y - bad) / np.linalg.norm(ref) > 1e-2, plant
