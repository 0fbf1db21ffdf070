"""Write the golden fixtures of tests/golden/ with the reference's own CPU kernels.

Runs only where the reference sources exist (this container): `make -C oracle` compiles
/root/reference/src/kernels/cpu/{iq_avx512,iq_avx2,kq_avx2,cpu_features}.cpp into oracle/_ref/libref.so, and this
script calls them through oracle/ref_driver.cpp.  The fixtures are data only (inputs and the reference's outputs):

  golden_q8k.npz    x [6, 512] float32 and the reference's Q8_K bytes (q8k_quant_avx2, src/kernels/cpu/iq_avx2.cpp:387-454),
                    including an all-zero block, a single-outlier block and a negative-maximum block.
  golden_rows.npz   per case (type, n, nt): weight row bytes, activation bytes (Q8_K, or Q8_0 for Q8_0 rows) and the
                    reference's row outputs (iq512_rows / kq256_rows: src/kernels/cpu/iq_avx512.cpp:155-186,
                    src/kernels/cpu/kq_avx2.cpp:84-189) and SwiGLU gate/up outputs (iq512_gu_rows / kq256_gu_rows).
  golden_sums.npz   single-sub-block probes: block scale 1.0, activation scale 1.0 and only sub-block j non-zero, so
                    the reference's float output is K * iscale_j * S_j exactly (every value < 2^24): pins the integer
                    sub-block sums and the sub-block scales of each format against the reference decode.

    python tests/golden/make_golden.py
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

import oracle as O  # noqa: E402

OUT = Path(__file__).resolve().parent
TYPES = (O.IQ3_XXS, O.IQ3_S, O.Q4_K, O.Q8_0)


def f16(v: float) -> bytes:
    return np.float16(v).tobytes()


def random_weights(rng, t: int, rows: int, n: int) -> np.ndarray:
    """Random block bytes with a controlled fp16 scale (every grid index, sign and sub-scale is exercised)."""
    qk, bb = O.BLOCK[t]
    w = rng.integers(0, 256, (rows, n // qk, bb), dtype=np.uint8)
    for r in range(rows):
        for b in range(n // qk):
            w[r, b, 0:2] = np.frombuffer(f16(float(np.ldexp(1.0, -12 + (r + b) % 5)) * (1 if (r + b) % 3 else -1)), np.uint8)
            if t == O.Q4_K:
                w[r, b, 2:4] = np.frombuffer(f16(float(np.ldexp(1.0, -13 + (r + 2 * b) % 4))), np.uint8)
    return w.reshape(rows, -1)


def activations(rng, t: int, x: np.ndarray) -> np.ndarray:
    if t == O.Q8_0:
        return np.concatenate([O.quantize_q8_0(r) for r in x])
    out = np.empty(x.shape[0] * (x.shape[1] // 256) * 292, np.uint8)
    O.ref().ref_q8k_quant(np.ascontiguousarray(x).ctypes.data, out.ctypes.data, x.size)
    return out


def main() -> None:
    if not O.ref_available():
        O.build()
    assert O.ref_available(), "the reference CPU kernels did not build (is /root/reference present?)"
    R = O.ref()
    rng = np.random.default_rng(20261201)

    # Q8_K quantizer
    x = rng.normal(0, 1, (6, 512)).astype(np.float32)
    x[1, :256] = 0.0                                   # all-zero block
    x[2, :256] = 1e-3
    x[2, 77] = 40.0                                    # one outlier
    x[3, 256:] = -np.abs(x[3, 256:])
    x[3, 300] = -9.0                                   # the block maximum is negative
    x[4, :] *= 1e-30                                   # tiny values
    q = np.empty(x.size // 256 * 292, np.uint8)
    R.ref_q8k_quant(x.ctypes.data, q.ctypes.data, x.size)
    np.savez_compressed(OUT / "golden_q8k.npz", x=x, q=q)

    # rows and gate/up rows
    cases = {}
    for t in TYPES:
        for n in (256, 2048):
            for nt in (1, 4):
                rows = 5
                w = random_weights(rng, t, 2 * rows, n)
                xa = rng.normal(0, 1, (nt, n)).astype(np.float32)
                a = activations(rng, t, xa)
                y = np.empty((nt, rows), np.float32)
                assert R.ref_rows(t, w.ctypes.data, n, rows, a.ctypes.data, nt, y.ctypes.data) == 0
                ff = np.empty((nt, rows), np.float32)
                assert R.ref_gu_rows(t, w.ctypes.data, n, rows, a.ctypes.data, nt, ff.ctypes.data) == 0
                key = f"t{t}_n{n}_nt{nt}"
                cases[key + "_w"] = w
                cases[key + "_x"] = xa
                cases[key + "_a"] = a
                cases[key + "_y"] = y
                cases[key + "_ff"] = ff
    np.savez_compressed(OUT / "golden_rows.npz", **cases)

    # single-sub-block probes at n = 256 (Q8_0: 32-value blocks, n = 256 = 8 blocks)
    sums = {}
    for t in TYPES:
        qk, bb = O.BLOCK[t]
        rows = 6
        w = random_weights(rng, t, rows, 256)
        for r in range(rows):
            for b in range(256 // qk):
                w[r, b * bb: b * bb + 2] = np.frombuffer(f16(1.0), np.uint8)
                if t == O.Q4_K:
                    w[r, b * bb + 2: b * bb + 4] = np.frombuffer(f16(0.0), np.uint8)  # dmin 0: the min term drops out
        codes = rng.integers(-127, 128, (8, 32), dtype=np.int8)
        outs = np.empty((8, rows), np.float32)
        acts = []
        for j in range(8):
            if t == O.Q8_0:
                a = np.zeros((8, 34), np.uint8)
                for b in range(8):
                    a[b, 0:2] = np.frombuffer(f16(1.0), np.uint8)
                a[j, 2:] = codes[j].view(np.uint8)
                a = a.ravel()
            else:
                a = np.zeros(292, np.uint8)
                a[0:4] = np.frombuffer(np.float32(1.0).tobytes(), np.uint8)
                qs = np.zeros(256, np.int8)
                qs[32 * j: 32 * j + 32] = codes[j]
                a[4:260] = qs.view(np.uint8)
                bs = qs.astype(np.int32).reshape(16, 16).sum(1).astype(np.int16)
                a[260:292] = bs.view(np.uint8)
            acts.append(a)
            y = np.empty((1, rows), np.float32)
            assert R.ref_rows(t, w.ctypes.data, 256, rows, a.ctypes.data, 1, y.ctypes.data) == 0
            outs[j] = y[0]
        sums[f"t{t}_w"] = w
        sums[f"t{t}_codes"] = codes
        sums[f"t{t}_out"] = outs
    np.savez_compressed(OUT / "golden_sums.npz", **sums)
    print("wrote", *(p.name for p in sorted(OUT.glob("golden_*.npz"))), "isa", R.ref_isa())


if __name__ == "__main__":
    main()
