"""The oracle's Q4_0 and Q6_K (the single-matrix and id-indexed products' extra formats) pinned against the
reference's own per-thread decomposition of the Q8_1 dot (src/lfm2/matvec.cu:762-794 for Q6_K, 838-851 for Q4_0),
restated here in numpy index for index: a different walk over the same bytes, so a wrong nibble, bit pair, scale
index or offset in the oracle's per-block decode fails it.  Random blocks (any byte pattern is a valid code; the
scales are set finite) stand in for quantized weights: no ggml quantizer is available offline."""
import numpy as np
import pytest

import oracle as O

Q4_0, Q6_K = 2, 14


def random_blocks(t, rows, n, seed):
    rng = np.random.default_rng(seed)
    if t == Q4_0:
        b = rng.integers(0, 256, (rows, n // 32, 18), dtype=np.uint8)
        b[..., 0:2] = rng.uniform(0.001, 0.05, (rows, n // 32)).astype(np.float16)[..., None].view(np.uint8)
    else:
        b = rng.integers(0, 256, (rows, n // 256, 210), dtype=np.uint8)
        b[..., 208:210] = rng.uniform(0.0001, 0.002, (rows, n // 256)).astype(np.float16)[..., None].view(np.uint8)
    return b.reshape(rows, -1)


def q8_1(x):
    q = O.quantize_q8_1(x)
    return q, O.q8_1_split(q)


def ref_q6k_row(row, d8, s8, codes, n):
    """sum over blocks and thread indices iqs of d * sum_i d8 * (dp4a(code bytes - 32, u) * scale), fp64."""
    acc = 0.0
    for kb in range(n // 256):
        blk = row[kb * 210:(kb + 1) * 210]
        ql, qh, sc = blk[:128], blk[128:192], blk[192:208].view(np.int8)
        d = float(blk[208:210].view(np.float16)[0])
        for iqs in range(32):
            bq8 = 4 * (iqs // 16) + (iqs % 16) // 8
            so = 8 * (iqs // 16) + (iqs % 16) // 4
            vh_shift = 2 * ((iqs % 16) // 8)
            vl = ql[4 * iqs:4 * iqs + 4].astype(np.int32)
            hb = 4 * (8 * (iqs // 16) + iqs % 8)
            vh = qh[hb:hb + 4].astype(np.int32) >> vh_shift
            tot = 0.0
            for i in range(2):
                vil = (vl >> (4 * i)) & 0x0F
                vih = ((vh >> (4 * i)) << 4) & 0x30
                vi = (vil | vih) - 32
                blk8 = kb * 8 + bq8 + 2 * i
                u = codes[blk8, 4 * (iqs % 8):4 * (iqs % 8) + 4].astype(np.int32)
                tot += float(d8[blk8]) * (int((vi * u).sum()) * int(sc[so + 4 * i]))
            acc += d * tot
    return acc


def ref_q4_0_row(row, d8, s8, codes, n):
    """per block, two calls of iqs = 0, 2: d * (sumi * d8 - 4 * s8), sumi over the low / high nibbles, fp64."""
    acc = 0.0
    for kb in range(n // 32):
        blk = row[kb * 18:(kb + 1) * 18]
        d = float(blk[0:2].view(np.float16)[0])
        qs = blk[2:18].astype(np.int32)
        for iqs in (0, 2):
            sumi = 0
            for i in range(2):
                v = qs[4 * (iqs + i):4 * (iqs + i) + 4]
                sumi += int(((v & 0x0F) * codes[kb, 4 * (iqs + i):4 * (iqs + i) + 4]).sum())
                sumi += int(((v >> 4) * codes[kb, 4 * (iqs + i + 4):4 * (iqs + i + 4) + 4]).sum())
            acc += d * (sumi * float(d8[kb]) - 4 * float(s8[kb]))
    return acc


@pytest.mark.parametrize("t,n", [(Q6_K, 256), (Q6_K, 512), (Q4_0, 64), (Q4_0, 256)])
def test_rows_match_the_reference_decomposition(t, n):
    rows = 6
    w = random_blocks(t, rows, n, seed=n + t)
    x = np.random.default_rng(t).normal(0, 1, (2, n)).astype(np.float32)
    xq, (d8, s8, codes) = q8_1(x)
    y = O.mmvq_q8_1(t, w, n, rows, xq, 2)
    ref = ref_q6k_row if t == Q6_K else ref_q4_0_row
    nb = n // 32
    for c in range(2):
        for r in range(rows):
            want = ref(w[r], d8[c * nb:(c + 1) * nb], s8[c * nb:(c + 1) * nb], codes[c * nb:(c + 1) * nb], n)
            assert abs(y[c, r] - want) <= 2e-6 * max(1.0, abs(want)), (c, r, y[c, r], want)


@pytest.mark.parametrize("t,n", [(Q6_K, 512), (Q4_0, 128)])
def test_integer_sums_and_dequantized_values(t, n):
    """The exact sums equal a brute-force sum over the dequantized values divided by their scales, and the
    dequantized row dotted with the dequantized activations gives the product up to Q4_0's stored-sum term."""
    rows = 3
    w = random_blocks(t, rows, n, seed=5)
    x = np.random.default_rng(9).normal(0, 1, (1, n)).astype(np.float32)
    xq, (d8, s8, codes) = q8_1(x)
    sums, qsums = O.subblock_sums(t, w, n, rows, xq, 1)
    assert (qsums[:, 0, :] == codes.astype(np.int32).sum(1)[None, :]).all()
    for r in range(rows):
        v = O.dequantize(t, w[r], n).astype(np.float64)
        if t == Q6_K:
            # value / d = scale(i) * (code - 32): the integer sum is sum of (value / d) * a
            d = np.repeat(w[r].reshape(-1, 210)[:, 208:210].copy().view(np.float16).astype(np.float64).ravel(), 256)
            k = np.rint(v / d).astype(np.int64).reshape(-1, 32)
            assert np.array_equal((k * codes.astype(np.int64)).sum(1), sums[r, 0])
        else:
            # value = d (code - 8): code = value / d + 8, and the sums are over the raw codes
            d = np.repeat(w[r].reshape(-1, 18)[:, 0:2].copy().view(np.float16).astype(np.float64).ravel(), 32)
            k = (np.rint(v / d) + 8).astype(np.int64).reshape(-1, 32)
            assert ((k >= 0) & (k <= 15)).all()
            assert np.array_equal((k * codes.astype(np.int64)).sum(1), sums[r, 0])
        xd = (codes.astype(np.float64) * d8[:, None]).ravel()
        dot = float(v @ xd)
        y = float(O.mmvq_q8_1(t, w[r:r + 1], n, 1, xq, 1)[0, 0])
        if t == Q4_0:
            # the product uses the stored float sum of each activation block where the dequantized dot has
            # d8 * (sum of codes): the difference is exactly 8 d (d8 sum(codes) - s8) per block
            dw = w[r].reshape(-1, 18)[:, 0:2].copy().view(np.float16).astype(np.float64).ravel()
            dot -= float((8 * dw * (s8 - d8 * codes.astype(np.float64).sum(1))).sum())
        assert abs(y - dot) <= 1e-5 * max(1.0, abs(dot)), (r, y, dot)
