"""The single-matrix product on Q4_0 and Q6_K, and several matrices per launch: picked on the device through a table
(tsx_moe_mmvq_ids, reference lfm_native_mmvq_ids) or given by the host (tsx_moe_mmvq_slots, lfm_native_mmvq_slots),
against the CPU oracle (marked gpu).

Bars: the integer sub-block sums bit-exact; float outputs within 1e-5 relative of the oracle (the same integer sums,
another float order); each matrix of a many-matrix launch bit-identical to the same matrix through tsx_moe_mmvq."""
import numpy as np
import pytest
import torch

import oracle as O
from tinystrata_amd import ops
from tinystrata_amd._lib import IQ3_S, IQ3_XXS, Q4_0, Q4_K, Q6_K, Q8_0

from gpu_util import dev, host

pytestmark = pytest.mark.gpu
ALL = (IQ3_XXS, IQ3_S, Q4_K, Q8_0, Q4_0, Q6_K)


def weights(t, rows, n, seed):
    """rows x n of type t: quantized N(0, 0.02) for the expert formats, random blocks with finite scales for Q4_0 and
    Q6_K (no ggml quantizer offline; every byte pattern is a valid code)."""
    rng = np.random.default_rng(seed)
    if t in (IQ3_XXS, IQ3_S, Q4_K, Q8_0):
        return ops.quantize_weights(t, rng.normal(0, 0.02, (rows, n)).astype(np.float32))
    if t == Q4_0:
        b = rng.integers(0, 256, (rows, n // 32, 18), dtype=np.uint8)
        b[..., 0:2] = rng.uniform(0.001, 0.05, (rows, n // 32)).astype(np.float16)[..., None].view(np.uint8)
    else:
        b = rng.integers(0, 256, (rows, n // 256, 210), dtype=np.uint8)
        b[..., 208:210] = rng.uniform(0.0001, 0.002, (rows, n // 256)).astype(np.float16)[..., None].view(np.uint8)
    return b.reshape(rows, -1)


@pytest.mark.parametrize("t", (Q4_0, Q6_K))
@pytest.mark.parametrize("n_in,n_out,ncols", [(2048, 96, 1), (512, 300, 4), (768, 64, 8)])
def test_small_formats(t, n_in, n_out, ncols):
    print(f"small format t={t} {n_out}x{n_in} ncols={ncols}", flush=True)
    w = weights(t, n_out, n_in, n_in + n_out)
    xq = O.quantize_q8_1(np.random.default_rng(t).normal(0, 1, (ncols, n_in)).astype(np.float32))
    got = host(ops.iq_mmvq(t, dev(w), dev(xq), n_in, n_out, ncols))
    exp = O.mmvq_q8_1(t, w, n_in, n_out, xq, ncols)
    np.testing.assert_allclose(got, exp, rtol=1e-5, atol=1e-5 * np.abs(exp).max())
    s, q = ops.subblock_sums(t, dev(w), n_in, n_out, dev(xq), ncols)
    es, eq = O.subblock_sums(t, w, n_in, n_out, xq, ncols)
    assert (host(s) == es).all() and (host(q) == eq).all()


@pytest.mark.parametrize("t", ALL)
@pytest.mark.parametrize("x_every", [1, 3])
def test_mmvq_ids(t, x_every):
    n_in, n_out, n_mat, count = 512, 80, 6, 11
    print(f"mmvq_ids t={t} x_every={x_every}", flush=True)
    rb = ops.iq_row_bytes(t, n_in)
    stride = (n_out * rb + 255) // 256 * 256 + 64        # matrices apart in one buffer, behind a 64-byte offset
    host_w = np.zeros((n_mat, stride), np.uint8)
    mats = []
    for m in range(n_mat):
        w = weights(t, n_out, n_in, 100 + m)
        host_w[m, 64:64 + w.size] = w.ravel()
        mats.append(w)
    buf = dev(host_w.ravel())
    table = torch.tensor([buf.data_ptr() + m * stride for m in range(n_mat)], dtype=torch.int64, device="cuda")
    ids = np.array([3, 0, 5, -1, 2, 2, 9, 1, 4, 0, 5], np.int32)  # -1 and 9 are outside the table: zeros
    nx = (count + x_every - 1) // x_every
    xq = O.quantize_q8_1(np.random.default_rng(7).normal(0, 1, (nx, n_in)).astype(np.float32)).reshape(-1)
    xs = n_in // 32 * 36
    y_stride = n_out + 5
    y = torch.full((count * y_stride,), 7.0, device="cuda")
    ops.mmvq_ids(t, table, dev(ids), 64, dev(xq), xs, x_every, y, y_stride, count, n_in, n_out)
    got = host(y).reshape(count, y_stride)
    for j in range(count):
        assert (got[j, n_out:] == 7.0).all()              # nothing past the matrix's rows
        if not 0 <= ids[j] < n_mat:
            assert (got[j, :n_out] == 0.0).all()
            continue
        xj = xq[(j // x_every) * xs:(j // x_every + 1) * xs]
        exp = O.mmvq_q8_1(t, mats[ids[j]], n_in, n_out, xj, 1)[0]
        np.testing.assert_allclose(got[j, :n_out], exp, rtol=1e-5, atol=1e-5 * np.abs(exp).max())
        one = host(ops.iq_mmvq(t, dev(mats[ids[j]]), dev(xj), n_in, n_out, 1))[0]
        assert np.array_equal(got[j, :n_out], one)


@pytest.mark.parametrize("t", (IQ3_XXS, Q4_0, Q6_K))
def test_mmvq_slots(t):
    n_in, n_out, count = 768, 48, 5
    ws = [dev(weights(t, n_out, n_in, 200 + j)) for j in range(count)]
    xqs = [O.quantize_q8_1(np.random.default_rng(j).normal(0, 1, (1, n_in)).astype(np.float32)) for j in range(count)]
    xs = [dev(x) for x in xqs]
    ys = [torch.zeros(n_out, device="cuda") for _ in range(count)]
    ops.mmvq_slots(t, ws, xs, ys, n_in, n_out)
    for j in range(count):
        one = host(ops.iq_mmvq(t, ws[j], xs[j], n_in, n_out, 1))[0]
        assert np.array_equal(host(ys[j]), one)
        exp = O.mmvq_q8_1(t, host(ws[j]), n_in, n_out, xqs[j], 1)[0]
        np.testing.assert_allclose(host(ys[j]), exp, rtol=1e-5, atol=1e-5 * np.abs(exp).max())
