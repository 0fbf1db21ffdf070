"""TEST INFRASTRUCTURE ONLY: numpy bindings of the CPU oracle (oracle/liboracle.so) and, where it was built, of the
reference's own CPU kernels (oracle/_ref/libref.so).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this package; the product path
(tinystrata_amd/) never does.  Each function names the reference code it restates in oracle/oracle.c.

Parity pins (tests/test_oracle.py): the golden fixtures of tests/golden/ (made by the reference's compiled CPU
kernels), oracle/_ref directly where it builds, brute-force integer sums against the dequantized floats, and closed
forms (Q8_1 / Q8_K special blocks, router ties, NaN and the renormalization floor).
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ORACLE_SO = HERE / "liboracle.so"
REF_SO = HERE / "_ref" / "libref.so"

Q8_0, Q8_1, Q4_K, Q8_K, IQ3_XXS, IQ3_S = 8, 9, 12, 15, 18, 21
BLOCK = {Q8_0: (32, 34), Q8_1: (32, 36), Q4_K: (256, 144), Q8_K: (256, 292), IQ3_XXS: (256, 98), IQ3_S: (256, 110),
         2: (32, 18), 14: (256, 210)}  # Q4_0, Q6_K

P, I32, I64, U64 = C.c_void_p, C.c_int, C.c_int64, C.c_uint64


class Layout(C.Structure):
    _fields_ = [("gu_type", C.c_int32), ("d_type", C.c_int32), ("n_embd", C.c_int64), ("n_ff", C.c_int64),
                ("gu_row", C.c_uint64), ("d_row", C.c_uint64), ("up_off", C.c_uint64), ("down_off", C.c_uint64),
                ("bytes", C.c_uint64)]


def build() -> None:
    """Compile liboracle.so (and _ref/libref.so where /root/reference exists) with oracle/Makefile."""
    subprocess.run(["make", "-s", "-C", str(HERE), "all"], check=True)


_orc = None
_ref = None


def orc() -> C.CDLL:
    global _orc
    if _orc is None:
        if not ORACLE_SO.exists():
            build()
        h = C.CDLL(str(ORACLE_SO))
        sig = {
            "orc_f2h": (C.c_uint16, [C.c_float]),
            "orc_h2f": (C.c_float, [C.c_uint16]),
            "orc_quantize_q8_1": (None, [P, I64, I64, P]),
            "orc_quantize_q8_K": (None, [P, I64, P]),
            "orc_quantize_q8_0": (None, [P, I64, P]),
            "orc_dequantize": (I32, [I32, P, I64, P]),
            "orc_subblock_sums": (I32, [I32, P, I64, I64, P, I64, P, P]),
            "orc_mmvq_q8_1": (I32, [I32, P, I64, I64, P, I64, P]),
            "orc_mmvq_ggml": (I32, [I32, P, I64, I64, P, I64, P]),
            "orc_router_topk": (I32, [P, I32, I32, I32, P, P]),
            "orc_group": (I32, [P, I32, I32, I32, U64, U64, P, P, P, P, P]),
            "orc_route_sort": (I32, [P, I32, I32, I32, P, P, P, P, P]),
            "orc_combine": (None, [P, P, P, P, I32, P, P, I32, I32, I32]),
            "orc_expert_gu": (I32, [C.POINTER(Layout), P, P, I32, P, P, P, P]),
            "orc_expert_down": (I32, [C.POINTER(Layout), P, P, I32, P, P, P]),
            "orc_moe_layer": (I32, [I32, C.POINTER(Layout), I32, I32, I32, P, P, P, U64, P, P, P, P, P]),
            "orc_grid_hash": (C.c_uint64, []),
            "orc_threads": (I32, []),
        }
        for name, (res, args) in sig.items():
            f = getattr(h, name)
            f.restype = res
            f.argtypes = args
        _orc = h
    return _orc


def ref_available() -> bool:
    return REF_SO.exists()


def ref() -> C.CDLL:
    global _ref
    if _ref is None:
        h = C.CDLL(str(REF_SO))
        sig = {
            "ref_isa": (I32, []),
            "ref_q8k_quant": (None, [P, P, I64]),
            "ref_rows": (I32, [I32, P, I32, I32, P, I32, P]),
            "ref_gu_rows": (I32, [I32, P, I32, I32, P, I32, P]),
            "ref_moe_decode": (C.c_double, [I32, I32, I32, I32, I32, I32, I32, P, P, P, U64, U64, P, P, P, I32, I32, P]),
        }
        for name, (res, args) in sig.items():
            f = getattr(h, name)
            f.restype = res
            f.argtypes = args
        _ref = h
    return _ref


def _c(a: np.ndarray) -> int:
    assert a.flags.c_contiguous
    return a.ctypes.data


def row_bytes(t: int, n: int) -> int:
    qk, bb = BLOCK[t]
    assert n % qk == 0
    return n // qk * bb


def layout(gu_type: int, d_type: int, n_embd: int, n_ff: int) -> Layout:
    L = Layout()
    L.gu_type, L.d_type, L.n_embd, L.n_ff = gu_type, d_type, n_embd, n_ff
    L.gu_row, L.d_row = row_bytes(gu_type, n_embd), row_bytes(d_type, n_ff)
    L.up_off = n_ff * L.gu_row
    L.down_off = 2 * L.up_off
    L.bytes = L.down_off + n_embd * L.d_row
    return L


# ------------------------------------------------------------------ activations
def quantize_q8_1(x: np.ndarray) -> np.ndarray:
    """x [rows, cols] -> uint8 [rows, cols/32*36] (q8_1_store: iq_kernels.cu:1467-1487)."""
    x = np.ascontiguousarray(x, np.float32)
    rows, cols = x.reshape(-1, x.shape[-1]).shape
    y = np.empty((rows, cols // 32 * 36), np.uint8)
    orc().orc_quantize_q8_1(_c(x), rows, cols, _c(y))
    return y


def quantize_q8_K(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32).ravel()
    y = np.empty(x.size // 256 * 292, np.uint8)
    orc().orc_quantize_q8_K(_c(x), x.size, _c(y))
    return y


def quantize_q8_0(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32).ravel()
    y = np.empty(x.size // 32 * 34, np.uint8)
    orc().orc_quantize_q8_0(_c(x), x.size, _c(y))
    return y


def q8_1_split(q: np.ndarray):
    """Q8_1 bytes -> (d float32 [..., nb], s float32 [..., nb], codes int8 [..., nb, 32])."""
    b = q.reshape(-1, 36)
    d = b[:, 0:2].copy().view(np.float16).astype(np.float32).ravel()
    s = b[:, 2:4].copy().view(np.float16).astype(np.float32).ravel()
    codes = b[:, 4:].copy().view(np.int8)
    return d, s, codes


# ------------------------------------------------------------------ weights
def dequantize(t: int, w: np.ndarray, n: int) -> np.ndarray:
    w = np.ascontiguousarray(w, np.uint8)
    out = np.empty(n, np.float32)
    assert orc().orc_dequantize(t, _c(w), n, _c(out)) == 0
    return out


def subblock_sums(t: int, w: np.ndarray, n_in: int, n_rows: int, xq: np.ndarray, ncols: int):
    sums = np.empty((n_rows, ncols, n_in // 32), np.int32)
    qsums = np.empty_like(sums)
    assert orc().orc_subblock_sums(t, _c(np.ascontiguousarray(w)), n_in, n_rows, _c(np.ascontiguousarray(xq)), ncols,
                                   _c(sums), _c(qsums)) == 0
    return sums, qsums


def mmvq_q8_1(t: int, w: np.ndarray, n_in: int, n_rows: int, xq: np.ndarray, ncols: int) -> np.ndarray:
    y = np.empty((ncols, n_rows), np.float32)
    assert orc().orc_mmvq_q8_1(t, _c(np.ascontiguousarray(w)), n_in, n_rows, _c(np.ascontiguousarray(xq)), ncols, _c(y)) == 0
    return y


def mmvq_ggml(t: int, w: np.ndarray, n_in: int, n_rows: int, xq: np.ndarray, ncols: int) -> np.ndarray:
    y = np.empty((ncols, n_rows), np.float32)
    assert orc().orc_mmvq_ggml(t, _c(np.ascontiguousarray(w)), n_in, n_rows, _c(np.ascontiguousarray(xq)), ncols, _c(y)) == 0
    return y


# ------------------------------------------------------------------ routing and combine
def router_topk(logits: np.ndarray, k: int):
    logits = np.ascontiguousarray(logits, np.float32)
    n_tok, n_expert = logits.shape
    ids = np.empty((n_tok, k), np.int32)
    w = np.empty((n_tok, k), np.float32)
    assert orc().orc_router_topk(_c(logits), n_tok, n_expert, k, _c(ids), _c(w)) == 0
    return ids, w


def group(ids: np.ndarray, k: int, n_expert: int, blobs: int = 0, stride: int = 0):
    ids = np.ascontiguousarray(ids, np.int32).ravel()
    n_ent = ids.size
    gp = np.zeros(min(n_ent, n_expert), np.uint64)
    gs = np.zeros(min(n_ent, n_expert) + 1, np.int32)
    ng = np.zeros(1, np.int32)
    ed = np.zeros(n_ent, np.int32)
    et = np.zeros(n_ent, np.int32)
    assert orc().orc_group(_c(ids), n_ent, k, n_expert, blobs, stride, _c(gp), _c(gs), _c(ng), _c(ed), _c(et)) == 0
    g = int(ng[0])
    return gp[:g], gs[:g + 1], g, ed, et


def route_sort(ids: np.ndarray, k: int, n_expert: int):
    ids = np.ascontiguousarray(ids, np.int32).ravel()
    n_ent = ids.size
    bounds = np.zeros(n_expert + 1, np.int32)
    ed, et, ri = (np.zeros(n_ent, np.int32) for _ in range(3))
    mr = np.zeros(1, np.int32)
    assert orc().orc_route_sort(_c(ids), n_ent, k, n_expert, _c(bounds), _c(ed), _c(et), _c(ri), _c(mr)) == 0
    return bounds, ed, et, ri, int(mr[0])


def combine(x: np.ndarray, parts: np.ndarray, wts: np.ndarray, k: int, prow=None, shared=None, sgate=None,
            sg_stride: int = 1) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32).copy()
    n_tok, n = x.shape
    prow_c = None if prow is None else np.ascontiguousarray(prow, np.int32)
    sh = None if shared is None else np.ascontiguousarray(shared, np.float32)
    sg = None if sgate is None else np.ascontiguousarray(sgate, np.float32)
    orc().orc_combine(_c(x), _c(np.ascontiguousarray(parts, np.float32)), None if prow_c is None else _c(prow_c),
                      _c(np.ascontiguousarray(wts, np.float32)), k, None if sh is None else _c(sh),
                      None if sg is None else _c(sg), sg_stride, n, n_tok)
    return x


def rms_norm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    """The MoE block's norm in closed form (float64): h[t] = x[t] / sqrt(mean(x[t]^2) + eps) * w
    (src/qwen35/q36_kernels.cuh:276-289; src/qwen35/q36_engine.cu:326-331)."""
    x = np.asarray(x, np.float64)
    return x / np.sqrt((x * x).mean(axis=1, keepdims=True) + eps) * np.asarray(w, np.float64)[None, :]


# ------------------------------------------------------------------ grouped experts and the layer
def expert_gu(L: Layout, blobs: list, grp_start: np.ndarray, ent_tok: np.ndarray, xq: np.ndarray):
    """-> h float32 [n_ent, n_ff], hq uint8 [n_ent, n_ff/32*36] (the gate/up half of native_expert_grouped)."""
    n_groups = len(blobs)
    n_ent = int(grp_start[n_groups])
    arr = (C.c_void_p * max(1, n_groups))(*[b.ctypes.data for b in blobs])
    h = np.zeros((max(1, n_ent), L.n_ff), np.float32)
    hq = np.zeros((max(1, n_ent), L.n_ff // 32 * 36), np.uint8)
    gs = np.ascontiguousarray(grp_start, np.int32)
    et = np.ascontiguousarray(ent_tok, np.int32)
    assert orc().orc_expert_gu(C.byref(L), arr, _c(gs), n_groups, _c(et), _c(np.ascontiguousarray(xq)), _c(h), _c(hq)) == 0
    return h[:n_ent], hq[:n_ent]


def expert_down(L: Layout, blobs: list, grp_start: np.ndarray, ent_dst: np.ndarray, hq: np.ndarray, n_out_rows: int):
    n_groups = len(blobs)
    arr = (C.c_void_p * max(1, n_groups))(*[b.ctypes.data for b in blobs])
    out = np.zeros((n_out_rows, L.n_embd), np.float32)
    assert orc().orc_expert_down(C.byref(L), arr, _c(np.ascontiguousarray(grp_start, np.int32)), n_groups,
                                 _c(np.ascontiguousarray(ent_dst, np.int32)), _c(np.ascontiguousarray(hq)), _c(out)) == 0
    return out


def moe_layer(mode: int, L: Layout, x: np.ndarray, logits: np.ndarray, k: int, blobs: np.ndarray, stride: int,
              shared: np.ndarray | None = None, sgate: np.ndarray | None = None):
    """The whole decode/prefill MoE layer on the CPU: mode 0 Q8_1 activations, mode 1 the reference CPU's (ggml)."""
    x = np.ascontiguousarray(x, np.float32)
    logits = np.ascontiguousarray(logits, np.float32)
    n_tok, n_expert = logits.shape
    y = np.empty((n_tok, L.n_embd), np.float32)
    ids = np.empty((n_tok, k), np.int32)
    w = np.empty((n_tok, k), np.float32)
    sg = None if sgate is None else np.ascontiguousarray(sgate, np.float32)
    rc = orc().orc_moe_layer(mode, C.byref(L), n_tok, n_expert, k, _c(x), _c(logits), _c(np.ascontiguousarray(blobs)),
                             stride, None if shared is None else _c(np.ascontiguousarray(shared)),
                             None if sg is None else _c(sg), _c(y), _c(ids), _c(w))
    assert rc == 0
    return y, ids, w


def grid_hash() -> int:
    return int(orc().orc_grid_hash())
