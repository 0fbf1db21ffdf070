"""GPU parity of each kernel against the CPU oracle, through the C ABI (marked gpu).

Bars: bit-exact for the Q8_1 bytes, the integer sub-block sums, the routing ids, the grouping and sort tables and the
prefill activation planes; float outputs of a dot product within 1e-5 relative (the same integer sums, a different
float summation order); a whole layer within 1e-3 relative L2 of the oracle fed the same int8 activation codes.
"""
import numpy as np
import pytest
import torch

import oracle as O
from tinystrata_amd import ops
from tinystrata_amd._lib import IQ3_S, IQ3_XXS, Q4_K, Q8_0

from gpu_util import dev, experts, host, rel_l2

pytestmark = pytest.mark.gpu
TYPES = (IQ3_XXS, IQ3_S, Q4_K, Q8_0)


def test_quantize_q8_1_bytes_exact():
    rng = np.random.default_rng(0)
    x = rng.normal(0, 1, (9, 2048)).astype(np.float32)
    x[1] = 0.0
    x[2, ::97] *= 40.0                       # outliers
    x[3, :32] = 1e9                          # d and s clamped to the largest half
    x[4] = np.round(x[4] * 8) / 8            # many exact halves of d
    got = host(ops.quantize_q8_1_rows(dev(x)))
    assert (got == O.quantize_q8_1(x)).all()


def _halves_rows(rng, rows, nb):
    """Rows of nb Q8_1 blocks whose values sit on and a few ulps beside half-integer multiples of the block scale, with
    block scales log-uniform from subnormal-adjacent to the fp16 clamp (so about one block in five has d < 2^-100)."""
    amax = np.exp(rng.uniform(np.log(1e-36), np.log(1e7), (rows, nb))).astype(np.float32)
    d = np.minimum(amax / np.float32(127.0), np.float32(65504.0)).astype(np.float32)
    n = rng.integers(-127, 127, (rows, nb, 31)).astype(np.float32)
    half = (n + np.float32(0.5)) * d[..., None]
    nudge = rng.integers(-3, 4, (rows, nb, 31))                    # a few ulps either side of the half
    vals = np.nextafter(half, np.where(nudge > 0, np.inf, -np.inf)).astype(np.float32)
    for _ in range(2):
        vals = np.where(np.abs(nudge) > 1, np.nextafter(vals, np.where(nudge > 0, np.inf, -np.inf)), vals)
    vals = np.where(nudge == 0, half, vals).astype(np.float32)
    x = np.concatenate([amax[..., None], vals], axis=2)             # the block's amax first
    x = np.where(rng.random(x.shape) < 0.5, -x, x).astype(np.float32).reshape(rows, nb * 32)
    assert np.isfinite(x).all()
    return x


def test_quantize_q8_1_halves_exact():
    """Quotients on and next to half-integers, where a quotient one ulp off would change roundf's code: the GPU forms
    v / d as a corrected product of the reciprocal, which must give the reference's codes (IEEE division, roundf) for
    every one of them, across block scales from subnormal-adjacent to the fp16 clamp."""
    x = _halves_rows(np.random.default_rng(11), 4096, 8)
    got = host(ops.quantize_q8_1_rows(dev(x)))
    assert (got == O.quantize_q8_1(x)).all()


def test_mmq_quantize_halves_exact():
    """The prompt quantizer's four-values-per-lane path on the same quotients: waves whose blocks all have d in
    [2^-100, 2^100] take the straight corrected products, waves holding a smaller d take the per-value path; both
    must give the reference's codes and scales, and the sums of the codes.  Zero blocks sit among them."""
    rng = np.random.default_rng(12)
    x = _halves_rows(rng, 2048, 8)
    x[::7, 64:96] = 0.0
    rows, cols = x.shape
    xq = host(ops.mmq_quantize(dev(x), None, Q4_K, cols, cols, rows))
    rp = (rows + 63) // 64 * 64 + 64
    r256 = lambda v: (v + 255) // 256 * 256
    q = xq[: rows * cols].view(np.int8).reshape(-1, 32)
    d = xq[r256(rp * cols): r256(rp * cols) + rows * cols // 32 * 4].view(np.float32)
    m0 = r256(rp * cols) + r256(rp * cols // 32 * 4)
    m = xq[m0: m0 + rows * cols // 32 * 4].view(np.int32)
    ed, _, ecodes = O.q8_1_split(O.quantize_q8_1(x))
    assert (q == ecodes).all() and (d == ed).all() and (m == ecodes.astype(np.int32).sum(1)).all()


@pytest.mark.parametrize("t", TYPES)
@pytest.mark.parametrize("n", [256, 2048])
def test_subblock_sums_exact(t, n):
    rng = np.random.default_rng(t * 7 + n)
    rows, ncols = 33, 3
    w = ops.quantize_weights(t, rng.normal(0, 0.02, (rows, n)).astype(np.float32))
    xq = O.quantize_q8_1(rng.normal(0, 1, (ncols, n)).astype(np.float32))
    s, q = ops.subblock_sums(t, dev(w), n, rows, dev(xq), ncols)
    es, eq = O.subblock_sums(t, w, n, rows, xq, ncols)
    assert (host(s) == es).all() and (host(q) == eq).all()


def test_subblock_sums_random_bytes_exact():
    """Random block bytes exercise every grid index, sign pattern and sub-block scale (fixture weights)."""
    from pathlib import Path

    g = np.load(Path(__file__).resolve().parent / "golden" / "golden_rows.npz")
    rng = np.random.default_rng(5)
    for t in TYPES:
        w = g[f"t{t}_n2048_nt4_w"]
        rows = w.shape[0]
        xq = O.quantize_q8_1(rng.normal(0, 1, (2, 2048)).astype(np.float32))
        s, q = ops.subblock_sums(t, dev(w), 2048, rows, dev(xq), 2)
        es, eq = O.subblock_sums(t, w, 2048, rows, xq, 2)
        assert (host(s) == es).all(), t


@pytest.mark.parametrize("t", TYPES)
@pytest.mark.parametrize("n_in,n_out,ncols", [(2048, 96, 1), (2048, 40, 4), (512, 2048, 8), (768, 64, 3)])
def test_mmvq(t, n_in, n_out, ncols):
    if n_in % O.BLOCK[t][0]:
        pytest.skip("not whole blocks")
    rng = np.random.default_rng(n_in + n_out + t)
    w = ops.quantize_weights(t, rng.normal(0, 0.02, (n_out, n_in)).astype(np.float32))
    xq = O.quantize_q8_1(rng.normal(0, 1, (ncols, n_in)).astype(np.float32))
    got = host(ops.iq_mmvq(t, dev(w), dev(xq), n_in, n_out, ncols))
    exp = O.mmvq_q8_1(t, w, n_in, n_out, xq, ncols)
    np.testing.assert_allclose(got, exp, rtol=1e-5, atol=1e-5 * np.abs(exp).max())


@pytest.mark.parametrize("E,k,T", [(256, 8, 1), (256, 8, 4), (128, 8, 512), (64, 4, 7), (512, 16, 3)])
def test_router_topk(E, k, T):
    rng = np.random.default_rng(E + k + T)
    logits = rng.normal(0, 1, (T, E)).astype(np.float32)
    ids, w = ops.native_router_topk(dev(logits), k)
    eids, ew = O.router_topk(logits, k)
    assert (host(ids) == eids).all()
    np.testing.assert_allclose(host(w), ew, rtol=2e-6, atol=1e-7)


def test_router_ties_and_nan():
    logits = np.zeros((2, 64), np.float32)
    logits[0, [5, 9, 40]] = 3.0
    logits[1, :] = -50.0
    logits[1, 7] = np.nan
    ids, w = ops.native_router_topk(dev(logits), 4)
    eids, ew = O.router_topk(logits, 4)
    assert (host(ids) == eids).all()


@pytest.mark.parametrize("n_tok,k,E", [(1, 8, 256), (4, 8, 256), (8, 8, 128), (64, 8, 256)])
def test_group_tables_exact(n_tok, k, E):
    rng = np.random.default_rng(n_tok * 13 + E)
    ids = np.stack([rng.choice(E, k, replace=False) for _ in range(n_tok)]).astype(np.int32)
    base, stride = 1 << 20, 4096
    gp, gs, ng, ed, et = ops.group_entries(dev(ids), k, E, base, stride)
    egp, egs, eg, eed, eet = O.group(ids, k, E, base, stride)
    g = int(host(ng)[0])
    assert g == eg
    assert (host(gp)[:g].astype(np.uint64) == egp).all() and (host(gs)[:g + 1] == egs).all()
    assert (host(ed) == eed).all() and (host(et) == eet).all()


@pytest.mark.parametrize("n_tok,k,E", [(512, 8, 128), (4096, 8, 256), (3, 2, 64), (129, 8, 512)])
def test_route_sort_exact(n_tok, k, E):
    rng = np.random.default_rng(n_tok + E)
    bias = np.log(1.0 / (1 + rng.permutation(E)) ** 1.2)          # Zipf-skewed loads
    logits = rng.normal(0, 1, (n_tok, E)) + bias
    ids = np.argsort(-logits, axis=1)[:, :k].astype(np.int32)
    b, ed, et, ri, mr = ops.route_sort(dev(ids), k, E)
    eb, eed, eet, eri, emr = O.route_sort(ids, k, E)
    assert (host(b) == eb).all() and (host(ed) == eed).all() and (host(et) == eet).all()
    assert (host(ri) == eri).all() and int(host(mr)[0]) == emr


@pytest.mark.parametrize("n", [2048, 2046])   # four columns per thread, and the one-column form
@pytest.mark.parametrize("shared", [False, True])
def test_combine(shared, n):
    rng = np.random.default_rng(3)
    T, k = 4, 8
    parts = rng.normal(0, 1, (T * k, n)).astype(np.float32)
    wts = rng.random((T, k)).astype(np.float32)
    x = rng.normal(0, 1, (T, n)).astype(np.float32)
    prow = rng.permutation(T * k).astype(np.int32)
    sh = rng.normal(0, 1, (T, n)).astype(np.float32) if shared else None
    sg = rng.normal(0, 1, T).astype(np.float32) if shared else None
    xd = dev(x)
    ops.moe_combine(xd, dev(parts), dev(wts), k, prow=dev(prow), shared=None if sh is None else dev(sh),
                    sgate=None if sg is None else dev(sg))
    exp = O.combine(x, parts, wts, k, prow=prow, shared=sh, sgate=sg)
    got = host(xd)
    if shared:   # expf of the gate on the two sides may differ in the last bit
        np.testing.assert_allclose(got, exp, rtol=1e-6, atol=1e-6)
    else:        # the same products and FMAs in the same order
        assert (got == exp).all()


@pytest.mark.parametrize("pad", [0, 1])  # rows 16-byte aligned (four values per lane), and not (one per lane)
@pytest.mark.parametrize("rows", [70, 0])
def test_mmq_quantize_planes_exact(pad, rows):
    rng = np.random.default_rng(8)
    cols = 512
    xw = rng.normal(0, 1, (100, cols + pad)).astype(np.float32)
    xw[3, 32:64] = 0.0                               # an all-zero block
    x = xw[:, :cols]
    ids = rng.integers(0, 100, rows).astype(np.int32)
    # the planes start as garbage: the launch writes every row, the padding rows as zeros
    xq0 = torch.full((ops.mmq_q8_bytes(rows, cols),), 0xAB, dtype=torch.uint8, device="cuda")
    xq = host(ops.mmq_quantize(dev(xw), dev(ids), Q4_K, cols, cols + pad, rows, xq=xq0))
    rp = (rows + 63) // 64 * 64 + 64
    r256 = lambda v: (v + 255) // 256 * 256
    q = xq[: rp * cols].view(np.int8).reshape(rp, cols)
    d = xq[r256(rp * cols): r256(rp * cols) + rp * cols // 32 * 4].view(np.float32).reshape(rp, cols // 32)
    m0 = r256(rp * cols) + r256(rp * cols // 32 * 4)
    m = xq[m0: m0 + rp * cols // 32 * 4].view(np.int32).reshape(rp, cols // 32)
    if rows:
        ed, _, ecodes = O.q8_1_split(O.quantize_q8_1(x[ids]))
        assert (q[:rows].reshape(-1, 32) == ecodes).all()
        assert (d[:rows].ravel() == ed).all()
        assert (m[:rows].ravel() == ecodes.astype(np.int32).sum(1)).all()
    assert (q[rows:] == 0).all() and (d[rows:] == 0).all() and (m[rows:] == 0).all()


@pytest.mark.parametrize("rows,E,k", [(1, 64, 8), (37, 128, 8), (300, 256, 8), (513, 512, 16)])
def test_mmq_quantize_route_matches_the_two_calls(rows, E, k):
    """tsx_moe_mmq_quantize_route: the token planes byte for byte as tsx_moe_mmq_quantize (every row, the padding
    rows zeroed over garbage), and ids / weights bit for bit as tsx_moe_router_topk, with tied logits in some rows."""
    rng = np.random.default_rng(rows + E + k)
    cols = 512
    x = rng.normal(0, 1, (rows, cols)).astype(np.float32)
    if rows > 3:
        x[3, 32:64] = 0.0                            # an all-zero block
    logits = rng.normal(0, 1, (rows, E)).astype(np.float32)
    if rows > 5:
        logits[5, :] = 0.25                          # every expert tied
        logits[4, 7:19] = logits[4, 6]               # ties around a pick
    xd, ld = dev(x), dev(logits)
    sep = host(ops.mmq_quantize(xd, None, IQ3_XXS, cols, cols, rows))
    ids_s = torch.empty((rows, k), dtype=torch.int32, device="cuda")
    wts_s = torch.empty((rows, k), dtype=torch.float32, device="cuda")
    ops.native_router_topk(ld, k, ids_s, wts_s)
    xq0 = torch.full((ops.mmq_q8_bytes(rows, cols),), 0xAB, dtype=torch.uint8, device="cuda")
    xq, ids, wts = ops.mmq_quantize_route(xd, IQ3_XXS, ld, k, xq=xq0)
    assert (host(xq) == sep).all()
    assert (host(ids) == host(ids_s)).all()
    assert (host(wts).view(np.int32) == host(wts_s).view(np.int32)).all()


@pytest.mark.parametrize("shared,prow,n", [(False, False, 2048), (True, True, 2048), (True, False, 4096),
                                           (False, True, 96)])
def test_combine_norm(shared, prow, n):
    """tsx_moe_combine_norm: x is tsx_moe_combine's x bit for bit; h the closed-form norm of it (within float32
    rounding); hq the Q8_1 image of h byte for byte."""
    rng = np.random.default_rng(n + shared)
    T, k, eps = 37, 8, 1e-5
    parts = rng.normal(0, 1, (T * k, n)).astype(np.float32)
    wts = rng.random((T, k)).astype(np.float32)
    x = rng.normal(0, 1, (T, n)).astype(np.float32)
    x[3] = 0.0                                                   # a row whose only content is the combine
    pr = dev(rng.permutation(T * k).astype(np.int32)) if prow else None
    sh = dev(rng.normal(0, 1, (T, n)).astype(np.float32)) if shared else None
    sg = dev(rng.normal(0, 1, T).astype(np.float32)) if shared else None
    wn = (1.0 + 0.1 * rng.normal(0, 1, n)).astype(np.float32)
    pd, wd = dev(parts), dev(wts)
    x_plain = dev(x)
    ops.moe_combine(x_plain, pd, wd, k, prow=pr, shared=sh, sgate=sg)
    xd = dev(x)
    h = torch.full((T, n), float("nan"), device="cuda")
    hq = torch.zeros((T, n // 32 * 36), dtype=torch.uint8, device="cuda")
    ops.moe_combine_norm(xd, pd, wd, k, dev(wn), eps, h, hq, prow=pr, shared=sh, sgate=sg)
    xv, hv = host(xd), host(h)
    assert (xv == host(x_plain)).all()
    ref = O.rms_norm(xv, wn, eps)
    assert np.abs(hv - ref).max() / np.abs(ref).max() < 2e-6
    assert (host(hq) == O.quantize_q8_1(hv)).all()


# ------------------------------------------------------------------ grouped experts
CASES = {
    "iq3_2048x512": (IQ3_XXS, IQ3_S, 2048, 512),
    "q8_0_2048x768": (Q8_0, Q8_0, 2048, 768),
    "q4_k_2048x768": (Q4_K, Q4_K, 2048, 768),
    "iq3_small": (IQ3_XXS, IQ3_S, 256, 256),
}


@pytest.mark.parametrize("case", list(CASES))
@pytest.mark.parametrize("n_tok", [1, 4])
def test_expert_grouped(case, n_tok):
    gu, d, N, FF = CASES[case]
    E, k = 32, 8
    L, blobs, _ = experts(gu, d, N, FF, E)
    Lo = O.layout(gu, d, N, FF)
    stride = blobs.shape[1]
    rng = np.random.default_rng(N + FF + n_tok)
    x = rng.normal(0, 1, (n_tok, N)).astype(np.float32)
    z = rng.normal(0, 1, E)
    logits = (z[None, :] + 0.5 * rng.normal(0, 1, (n_tok, E))).astype(np.float32)   # overlapping experts
    ids, _ = O.router_topk(logits, k)
    blobs_d = dev(blobs.ravel())
    n_ent = n_tok * k
    gp, gs, ng, ed, et = ops.group_entries(dev(ids), k, E, blobs_d.data_ptr(), stride)
    xq = ops.quantize_q8_1_rows(dev(x))
    scratch = torch.zeros(ops.native_expert_scratch_bytes(n_ent, FF), dtype=torch.uint8, device="cuda")
    out = torch.full((n_ent, N), float("nan"), device="cuda")
    cap_groups = min(n_ent, E)
    ops.native_expert_grouped(L, gp, gs, ng, ed, et, cap_groups, n_ent, xq, scratch, out)
    got = host(out)
    # the oracle on the same tables
    _, egs, g, eed, eet = O.group(ids, k, E)
    used = np.unique(ids)
    hb = [blobs[x] for x in used]
    xq_h = host(xq)
    h, hq = O.expert_gu(Lo, hb, egs, eet, xq_h)
    sc = host(scratch)
    fa = (n_ent * FF * 4 + 255) // 256 * 256
    gate = sc[:n_ent * FF * 4].view(np.float32).reshape(n_ent, FF)
    up = sc[fa: fa + n_ent * FF * 4].view(np.float32).reshape(n_ent, FF)
    # gate/up rows: the same integer sums, float order only
    for e in range(n_ent):
        tok = eet[e]
        x_blob = blobs[ids.ravel()[eed[e]]]
        eg = O.mmvq_q8_1(gu, x_blob, N, FF, xq_h[tok], 1)[0]
        eu = O.mmvq_q8_1(gu, x_blob[Lo.up_off:], N, FF, xq_h[tok], 1)[0]
        np.testing.assert_allclose(gate[e], eg, rtol=1e-5, atol=1e-5 * np.abs(eg).max())
        np.testing.assert_allclose(up[e], eu, rtol=1e-5, atol=1e-5 * np.abs(eu).max())
    hq_gpu = sc[ops.scratch_hq_offset(n_ent, FF): ops.scratch_hq_offset(n_ent, FF) + n_ent * FF // 32 * 36]
    hq_gpu = hq_gpu.reshape(n_ent, -1)
    # Q8_1 of the GPU's own SwiGLU output equals the oracle's but for values on a rounding edge
    d_g, _, c_g = O.q8_1_split(hq_gpu)
    d_o, _, c_o = O.q8_1_split(hq)
    assert np.mean(c_g != c_o) < 1e-3 and np.mean(d_g != d_o) < 1e-2
    # the down rows fed the GPU's int8 codes: float order only
    down_same = O.expert_down(Lo, hb, egs, eed, hq_gpu, n_ent)
    np.testing.assert_allclose(got, down_same, rtol=1e-5, atol=1e-5 * np.abs(down_same).max())
    # end to end against the oracle's own codes
    down_own = O.expert_down(Lo, hb, egs, eed, hq, n_ent)
    assert rel_l2(got, down_own) < 1e-3


def test_expert_grouped_grid_groups_invariant():
    gu, d, N, FF = CASES["iq3_small"]
    E, k, n_tok = 16, 4, 4
    L, blobs, _ = experts(gu, d, N, FF, E)
    rng = np.random.default_rng(1)
    ids = np.stack([rng.choice(E, k, replace=False) for _ in range(n_tok)]).astype(np.int32)
    blobs_d = dev(blobs.ravel())
    gp, gs, ng, ed, et = ops.group_entries(dev(ids), k, E, blobs_d.data_ptr(), blobs.shape[1])
    xq = ops.quantize_q8_1_rows(dev(rng.normal(0, 1, (n_tok, N)).astype(np.float32)))
    n_ent = n_tok * k
    outs = []
    for gg in (0, 1, 3):
        scratch = torch.zeros(ops.native_expert_scratch_bytes(n_ent, FF), dtype=torch.uint8, device="cuda")
        out = torch.zeros((n_ent, N), device="cuda")
        ops.native_expert_grouped(L, gp, gs, ng, ed, et, min(n_ent, E), n_ent, xq, scratch, out, grid_groups=gg)
        outs.append(host(out))
    assert (outs[0] == outs[1]).all() and (outs[0] == outs[2]).all()


# ------------------------------------------------------------------ grouped prompt products
@pytest.mark.parametrize("t", TYPES)
@pytest.mark.parametrize("w_cols", [256, 512, 2048])
@pytest.mark.parametrize("w_rows", [64, 128, 256, 512, 96])
def test_mmq_run_skewed_groups(t, w_cols, w_rows):
    """One grouped product over experts with 0, 1, 17, 70, 130, 255, 256 and 530 rows (tile tails, empty experts,
    several tiles, whole tiles, an expert over 500 rows as configs[4]'s Zipf routing makes),
    rows scattered to dst through ids; against the oracle's per-row dot on the same Q8_1 codes.  64, 128 and 256
    weight rows take the MFMA tiles with 2, 4 and 8 waves (Q4_K: 4 waves for 128 and 256, two blocks per CU; 512 IQ3
    columns: rows that start off 16-byte alignment); 512 rows of at most 512 columns take two 256-row column blocks per
    block in turn (every type but Q4_K; 256 columns: one chunk per pass); 96 rows the row-dot kernel."""
    rng = np.random.default_rng(t + w_cols + w_rows)
    counts = [0, 70, 1, 130, 17, 530, 255, 256]
    n, total = len(counts), sum(counts)
    bounds = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    W = [ops.quantize_weights(t, rng.normal(0, 0.02, (w_rows, w_cols)).astype(np.float32)) for _ in range(n)]
    rb = W[0].shape[1]
    eb = (w_rows * rb + 255) // 256 * 256
    blob = np.zeros(n * eb, np.uint8)
    for i, m in enumerate(W):
        blob[i * eb: i * eb + m.size] = m.ravel()
    x = rng.normal(0, 1, (total, w_cols)).astype(np.float32)
    ids = rng.permutation(total).astype(np.int32)
    xq = ops.mmq_quantize(dev(x), None, t, w_cols, w_cols, total)
    dst = torch.full((total, w_rows), float("nan"), device="cuda")
    ops.mmq_run(dev(blob), t, w_rows, w_cols, eb, n, xq, dev(bounds), dev(ids), total, dst, w_rows)
    got = host(dst)
    xb = O.quantize_q8_1(x)
    exp = np.zeros((total, w_rows), np.float64)
    for i in range(n):
        r0, r1 = bounds[i], bounds[i + 1]
        if r1 > r0:
            exp[ids[r0:r1]] = O.mmvq_q8_1(t, W[i], w_cols, w_rows, xb[r0:r1], r1 - r0)
    assert np.isfinite(got).all()
    np.testing.assert_allclose(got, exp, rtol=1e-5, atol=1e-5 * np.abs(exp).max())


@pytest.mark.parametrize("t", [IQ3_XXS, Q4_K])
def test_mmq_run_tile_classes(t):
    """The block order's tile classes at their edges: partial last tiles of exactly kBN/4 and kBN/2 rows and one more
    (IQ3: 128-token tiles, Q4_K: 64), whole tiles, empty experts, and enough full tiles (two experts of 1500 and 2600
    rows) that whole rounds of them take the XCD order while the rest keep linear order; every sorted row once, against
    the oracle's per-row dot on the same Q8_1 codes."""
    w_cols, w_rows = 512, 256
    rng = np.random.default_rng(40 + t)
    counts = [16, 17, 32, 33, 0, 48, 64, 65, 2600, 96, 127, 128, 160, 161, 80, 1500, 1, 0, 31]
    n, total = len(counts), sum(counts)
    bounds = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    W = [ops.quantize_weights(t, rng.normal(0, 0.02, (w_rows, w_cols)).astype(np.float32)) for _ in range(n)]
    rb = W[0].shape[1]
    eb = (w_rows * rb + 255) // 256 * 256
    blob = np.zeros(n * eb, np.uint8)
    for i, m in enumerate(W):
        blob[i * eb: i * eb + m.size] = m.ravel()
    x = rng.normal(0, 1, (total, w_cols)).astype(np.float32)
    ids = rng.permutation(total).astype(np.int32)
    xq = ops.mmq_quantize(dev(x), None, t, w_cols, w_cols, total)
    dst = torch.full((total, w_rows), float("nan"), device="cuda")
    ops.mmq_run(dev(blob), t, w_rows, w_cols, eb, n, xq, dev(bounds), dev(ids), total, dst, w_rows)
    got = host(dst)
    xb = O.quantize_q8_1(x)
    exp = np.zeros((total, w_rows), np.float64)
    for i in range(n):
        r0, r1 = bounds[i], bounds[i + 1]
        if r1 > r0:
            exp[ids[r0:r1]] = O.mmvq_q8_1(t, W[i], w_cols, w_rows, xb[r0:r1], r1 - r0)
    assert np.isfinite(got).all()  # every row written (the NaN fill would survive a missed tile)
    np.testing.assert_allclose(got, exp, rtol=1e-5, atol=1e-5 * np.abs(exp).max())


def _planes(buf, rows: int, cols: int):
    """The Q8_1 planes of tsx_moe_mmq_q8_bytes: codes, block scales and code sums of the first `rows` rows."""
    b = host(buf)
    rp = (rows + 63) // 64 * 64 + 64
    a256 = lambda v: (v + 255) // 256 * 256
    q = b[: rp * cols].view(np.int8).reshape(rp, cols)[:rows]
    o = a256(rp * cols)
    d = b[o: o + rp * (cols // 32) * 4].view(np.float32).reshape(rp, cols // 32)[:rows]
    o += a256(rp * (cols // 32) * 4)
    m = b[o: o + rp * (cols // 32) * 4].view(np.int32).reshape(rp, cols // 32)[:rows]
    return q, d, m


@pytest.mark.parametrize("t", TYPES)
@pytest.mark.parametrize("N,FF", [(512, 128), (2048, 384)])
@pytest.mark.parametrize("gather", [False, True])
def test_mmq_gate_up_swiglu_matches_the_call_sequence(t, N, FF, gather):
    """The fused gate/up + SwiGLU + Q8_1 launch against the reference's sequence on the GPU (gather-quantize, gate/up
    product, swiglu, quantize of h): the same planes byte for byte, over experts with 0, 70, 1, 130 and 17 rows whose
    activation rows are token rows taken through a map (gather) or the sorted rows themselves; and h against the
    oracle's SwiGLU of its own dot products, to the Q8_1 rounding."""
    rng = np.random.default_rng(t * 11 + N + FF + gather)
    counts = [0, 70, 1, 130, 17, 530, 255, 256]
    n, total = len(counts), sum(counts)
    bounds = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    W = [ops.quantize_weights(t, rng.normal(0, 0.05, (2 * FF, N)).astype(np.float32)) for _ in range(n)]
    rb = W[0].shape[1]
    eb = (2 * FF * rb + 255) // 256 * 256
    blob = np.zeros(n * eb, np.uint8)
    for i, m in enumerate(W):
        blob[i * eb: i * eb + m.size] = m.ravel()
    n_tok = 150 if gather else total
    x = rng.normal(0, 1, (n_tok, N)).astype(np.float32)
    x[:, rng.choice(N, N // 50, replace=False)] *= 20.0  # outlier channels
    xids = rng.integers(0, n_tok, total).astype(np.int32) if gather else np.arange(total, dtype=np.int32)
    blob_d, bounds_d = dev(blob), dev(bounds)
    # the reference's sequence
    xq_rows = ops.mmq_quantize(dev(x), dev(xids), t, N, N, total)
    gu = torch.empty((total, 2 * FF), device="cuda")
    ops.mmq_run(blob_d, t, 2 * FF, N, eb, n, xq_rows, bounds_d, None, total, gu, 2 * FF)
    h = ops.mmq_swiglu(gu, total, FF)
    ref = ops.mmq_quantize(h, None, t, FF, FF, total)
    # fused
    xq_tok = ops.mmq_quantize(dev(x), None, t, N, N, n_tok)
    got = ops.mmq_gate_up_swiglu(blob_d, t, FF, N, eb, n, xq_tok, n_tok, dev(xids) if gather else None, bounds_d,
                                 total)
    gq, gd, gm = _planes(got, total, FF)
    rq, rd, rm = _planes(ref, total, FF)
    assert (gq == rq).all() and (gd.view(np.int32) == rd.view(np.int32)).all() and (gm == rm).all()
    # h against the oracle: SwiGLU of the oracle's gate / up dots on the same Q8_1 codes
    xb = O.quantize_q8_1(x[xids])
    hx = np.zeros((total, FF), np.float64)
    for i in range(n):
        r0, r1 = bounds[i], bounds[i + 1]
        if r1 > r0:
            o = O.mmvq_q8_1(t, W[i], N, 2 * FF, xb[r0:r1], r1 - r0)
            g, u = o[:, :FF], o[:, FF:]
            hx[r0:r1] = g / (1.0 + np.exp(-g)) * u
    hd = gq.reshape(total, FF // 32, 32).astype(np.float64) * gd[:, :, None]
    assert rel_l2(hd.reshape(total, FF), hx) < 2e-2
