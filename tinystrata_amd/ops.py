"""Python mirror of the reference's operator API for the MoE expert path, over libtsx_moe.so.

Names and argument meanings follow TinyStrata's C++ headers (include/strata/kernels/iq_kernels.hpp,
native_mmvq.hpp, native_router.hpp, include/strata/prefill/moe_mmq.hpp); buffers are torch tensors in device
memory (PyTorch is only the allocator and the stream here), and every call enqueues on the current stream.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import torch

from ._lib import IQ3_S, IQ3_XXS, Q4_K, Q8_0, ExpertLayout, MmqProduct, MmvqIds, MmvqSlots, check, lib

WEIGHT_TYPES = (Q8_0, Q4_K, IQ3_XXS, IQ3_S)
Q8_1_BLOCK_BYTES = 36


def _p(t: torch.Tensor | None) -> int | None:
    if t is None:
        return None
    if not t.is_cuda:
        raise ValueError("device tensors only")
    return t.data_ptr()


def _stream(stream=None) -> int:
    s = stream if stream is not None else torch.cuda.current_stream()
    return s.cuda_stream


# ------------------------------------------------------------------ formats
def iq_supported(ggml_type: int) -> bool:
    return ggml_type in WEIGHT_TYPES


def iq_row_bytes(ggml_type: int, n: int) -> int:
    return lib().tsx_moe_row_bytes(ggml_type, n)


def native_expert_supported(gu_type: int, d_type: int, n_embd: int, n_ff: int) -> bool:
    return bool(lib().tsx_moe_expert_supported(gu_type, d_type, n_embd, n_ff))


def native_expert_layout(gu_type: int, d_type: int, n_embd: int, n_ff: int) -> ExpertLayout:
    L = ExpertLayout()
    check(lib().tsx_moe_expert_layout(gu_type, d_type, n_embd, n_ff, C.byref(L)), "native_expert_layout")
    return L


def native_expert_scratch_bytes(cap_entries: int, n_ff: int) -> int:
    return lib().tsx_moe_expert_scratch_bytes(cap_entries, n_ff)


def scratch_hq_offset(cap_entries: int, n_ff: int) -> int:
    return lib().tsx_moe_expert_scratch_hq_offset(cap_entries, n_ff)


# ------------------------------------------------------------------ activations
def quantize_q8_1_rows(x: torch.Tensor, out: torch.Tensor | None = None, stream=None) -> torch.Tensor:
    """x [rows, cols] float32 -> Q8_1 blocks, uint8 [rows, cols/32*36]."""
    rows, cols = x.shape
    if out is None:
        out = torch.empty((rows, cols // 32 * Q8_1_BLOCK_BYTES), dtype=torch.uint8, device=x.device)
    check(lib().tsx_moe_quantize_q8_1(_p(x), rows, cols, _p(out), _stream(stream)), "quantize_q8_1_rows")
    return out


def native_swiglu_quantize_q8_1(gate: torch.Tensor, up: torch.Tensor, out: torch.Tensor | None = None, stream=None):
    n = gate.numel()
    if out is None:
        out = torch.empty(n // 32 * Q8_1_BLOCK_BYTES, dtype=torch.uint8, device=gate.device)
    check(lib().tsx_moe_swiglu_quantize_q8_1(_p(gate), _p(up), n, _p(out), _stream(stream)), "native_swiglu_quantize_q8_1")
    return out


# ------------------------------------------------------------------ decode
def native_expert_grouped(L: ExpertLayout, grp_ptr, grp_start, n_groups, ent_dst, ent_tok, cap_groups: int,
                          cap_entries: int, x_q8_1, scratch, out, grid_groups: int = 0, stream=None) -> None:
    check(lib().tsx_moe_expert_grouped(C.byref(L), _p(grp_ptr), _p(grp_start), _p(n_groups), _p(ent_dst), _p(ent_tok),
                                       cap_groups, cap_entries, _p(x_q8_1), _p(scratch), _p(out), _stream(stream),
                                       grid_groups), "native_expert_grouped")


def iq_mmvq(ggml_type: int, w, x_q8_1, n_in: int, n_out: int, ncols: int, y=None, stream=None) -> torch.Tensor:
    """y[c][r] = W[r] . x[c] (ncols 1..8)."""
    if y is None:
        y = torch.empty((ncols, n_out), dtype=torch.float32, device=w.device)
    check(lib().tsx_moe_mmvq(ggml_type, _p(w), _p(x_q8_1), _p(y), n_in, n_out, ncols, _stream(stream)), "iq_mmvq")
    return y


native_mmvq = iq_mmvq


def mmvq_ids_supported(ggml_type: int) -> bool:
    return bool(lib().tsx_moe_mmvq_ids_supported(ggml_type))


def mmvq_ids(ggml_type: int, table: torch.Tensor, ids: torch.Tensor, offset: int, x_q8_1, x_stride: int, x_every: int,
             y: torch.Tensor, y_stride: int, count: int, n_in: int, n_out: int, stream=None) -> torch.Tensor:
    """Matrix j = table[ids[j]] + offset bytes (table: int64 device addresses), times the Q8_1 column
    x + (j / x_every) * x_stride bytes, into y + j * y_stride floats (reference lfm_native_mmvq_ids)."""
    a = MmvqIds(table=_p(table), ids=_p(ids), n_table=table.numel(), offset=offset, x=_p(x_q8_1), x_stride=x_stride,
                x_every=x_every, y=_p(y), y_stride=y_stride)
    check(lib().tsx_moe_mmvq_ids(ggml_type, C.byref(a), count, n_in, n_out, _stream(stream)), "mmvq_ids")
    return y


def mmvq_slots(ggml_type: int, ws, xs, ys, n_in: int, n_out: int, stream=None) -> None:
    """Up to 8 matrices ws[j] times their own Q8_1 column xs[j] into ys[j] (reference lfm_native_mmvq_slots)."""
    a = MmvqSlots()
    for j, (w, x, y) in enumerate(zip(ws, xs, ys)):
        a.w[j], a.x[j], a.y[j] = _p(w), _p(x), _p(y)
    check(lib().tsx_moe_mmvq_slots(ggml_type, C.byref(a), len(ws), n_in, n_out, _stream(stream)), "mmvq_slots")


def decode_layer_scratch_bytes(n_tok: int, k: int, n_ff: int) -> int:
    return lib().tsx_moe_decode_layer_scratch_bytes(n_tok, k, n_ff)


def moe_decode_layer(L: ExpertLayout, blobs, stride: int, n_expert: int, k: int, logits, x, y, ids, wts, scratch,
                     shared=None, sgate=None, sg_stride: int = 1, stream=None, norm_w=None, eps: float = 1e-6,
                     h=None, hq=None) -> None:
    """y += the whole decode MoE layer of x (1..8 tokens) in two launches (tsx_moe_decode_layer); with norm_w, also
    h = rms(y) * norm_w and (hq given) its Q8_1 image (tsx_moe_decode_layer_norm)."""
    n_tok = x.shape[0]
    # the scratch size depends on the token count (h in fp32 for one to four tokens at n_ff <= 512, as Q8_1 planes
    # otherwise): a buffer sized for another count may be too small
    need = decode_layer_scratch_bytes(n_tok, k, int(L.n_ff))
    have = scratch.numel() * scratch.element_size() if hasattr(scratch, "numel") else None
    if have is not None and have < need:
        raise ValueError(f"moe_decode_layer: scratch of {have} bytes, {n_tok} tokens x top-{k} at n_ff {int(L.n_ff)} "
                         f"need {need} (decode_layer_scratch_bytes)")
    if norm_w is None:
        check(lib().tsx_moe_decode_layer(C.byref(L), _p(blobs), stride, n_expert, k, n_tok, _p(logits), _p(x),
                                         _p(shared), _p(sgate), sg_stride, _p(y), _p(ids), _p(wts), _p(scratch),
                                         _stream(stream)), "moe_decode_layer")
        return
    check(lib().tsx_moe_decode_layer_norm(C.byref(L), _p(blobs), stride, n_expert, k, n_tok, _p(logits), _p(x),
                                          _p(shared), _p(sgate), sg_stride, _p(y), _p(ids), _p(wts), _p(norm_w), eps,
                                          _p(h), _p(hq), _p(scratch), _stream(stream)), "moe_decode_layer_norm")


# ------------------------------------------------------------------ routing
def native_router_topk(logits: torch.Tensor, k: int, ids=None, weights=None, stream=None):
    n_tok, n_expert = logits.shape
    if ids is None:
        ids = torch.empty((n_tok, k), dtype=torch.int32, device=logits.device)
    if weights is None:
        weights = torch.empty((n_tok, k), dtype=torch.float32, device=logits.device)
    check(lib().tsx_moe_router_topk(_p(logits), _p(ids), _p(weights), n_expert, k, n_tok, _stream(stream)),
          "native_router_topk")
    return ids, weights


def group_entries(ids: torch.Tensor, k: int, n_expert: int, blobs_ptr: int, stride: int, bufs=None, stream=None):
    """Decode grouping (k_group): returns grp_ptr, grp_start, n_groups, ent_dst, ent_tok (device tensors)."""
    n_ent = ids.numel()
    cap = min(n_ent, n_expert)
    dev = ids.device
    if bufs is None:
        bufs = (torch.empty(cap, dtype=torch.int64, device=dev), torch.empty(cap + 1, dtype=torch.int32, device=dev),
                torch.empty(1, dtype=torch.int32, device=dev), torch.empty(n_ent, dtype=torch.int32, device=dev),
                torch.empty(n_ent, dtype=torch.int32, device=dev))
    gp, gs, ng, ed, et = bufs
    check(lib().tsx_moe_group(_p(ids), n_ent, k, n_expert, blobs_ptr, stride, _p(gp), _p(gs), _p(ng), _p(ed), _p(et),
                              _stream(stream)), "group_entries")
    return bufs


def group_resident(ids: torch.Tensor, k: int, n_expert: int, slot_of: torch.Tensor, slots_ptr: int, stride: int,
                   bufs, stream=None):
    """Decode grouping of a hybrid layer (k_group_hy): only entries whose expert has a slot; group blobs in slots."""
    gp, gs, ng, ed, et = bufs
    check(lib().tsx_moe_group_resident(_p(ids), ids.numel(), k, n_expert, _p(slot_of), slots_ptr, stride, _p(gp),
                                       _p(gs), _p(ng), _p(ed), _p(et), _stream(stream)), "group_resident")
    return bufs


def merge_rows(parts: torch.Tensor, rows: torch.Tensor, miss: torch.Tensor, stream=None) -> None:
    """parts[e] = rows[miss[e]] where miss[e] >= 0 (k_merge_cpu, compact rows)."""
    n_ent, n = parts.shape
    check(lib().tsx_moe_merge_rows(_p(parts), _p(rows), _p(miss), n_ent, n, _stream(stream)), "merge_rows")


def route_sort(ids: torch.Tensor, k: int, n_expert: int, bufs=None, stream=None):
    """The prompt's expert sort: bounds [E+1], ent_dst, ent_tok, rinv [n_ent], max_rows [1]."""
    n_ent = ids.numel()
    dev = ids.device
    if bufs is None:
        bufs = (torch.empty(n_expert + 1, dtype=torch.int32, device=dev), torch.empty(n_ent, dtype=torch.int32, device=dev),
                torch.empty(n_ent, dtype=torch.int32, device=dev), torch.empty(n_ent, dtype=torch.int32, device=dev),
                torch.empty(1, dtype=torch.int32, device=dev))
    b, ed, et, ri, mr = bufs
    check(lib().tsx_moe_route_sort(_p(ids), n_ent, k, n_expert, _p(b), _p(ed), _p(et), _p(ri), _p(mr), _stream(stream)),
          "route_sort")
    return bufs


def moe_combine(x, parts, wts, k: int, prow=None, shared=None, sgate=None, sg_stride: int = 1, stream=None) -> None:
    """x[t] += sum_j w[t][j] parts[p(t,j)] (+ sigmoid(sgate[t]) shared[t]), in place."""
    n_tok, n = x.shape
    check(lib().tsx_moe_combine(_p(x), _p(parts), _p(prow), _p(wts), k, _p(shared), _p(sgate), sg_stride, n, n_tok,
                                _stream(stream)), "moe_combine")


def moe_combine_norm(x, parts, wts, k: int, norm_w, eps: float, h, hq=None, prow=None, shared=None, sgate=None,
                     sg_stride: int = 1, stream=None) -> None:
    """moe_combine, then h = rms(x) * norm_w and (hq given) its Q8_1 image: the MoE block's end (k_moe_out)."""
    n_tok, n = x.shape
    check(lib().tsx_moe_combine_norm(_p(x), _p(parts), _p(prow), _p(wts), k, _p(shared), _p(sgate), sg_stride, n, n_tok,
                                     _p(norm_w), eps, _p(h), _p(hq), _stream(stream)), "moe_combine_norm")


# ------------------------------------------------------------------ prefill
def mmq_q8_bytes(rows: int, cols: int) -> int:
    return lib().tsx_moe_mmq_q8_bytes(rows, cols)


def mmq_quantize(x, ids, ggml_type: int, cols: int, ld: int, rows: int, xq=None, stream=None) -> torch.Tensor:
    if xq is None:
        xq = torch.empty(mmq_q8_bytes(rows, cols), dtype=torch.uint8, device=x.device)
    check(lib().tsx_moe_mmq_quantize(_p(x), _p(ids), _p(xq), ggml_type, cols, ld, rows, _stream(stream)), "mmq_quantize")
    return xq


def mmq_quantize_route(x, ggml_type: int, logits, k: int, xq=None, ids=None, wts=None, stream=None):
    """mmq_quantize of the token rows of x (ids None) and native_router_topk of logits in one launch; returns
    (xq, ids, wts)."""
    rows, cols = x.shape
    n_expert = logits.shape[1]
    if xq is None:
        xq = torch.empty(mmq_q8_bytes(rows, cols), dtype=torch.uint8, device=x.device)
    if ids is None:
        ids = torch.empty((rows, k), dtype=torch.int32, device=x.device)
    if wts is None:
        wts = torch.empty((rows, k), dtype=torch.float32, device=x.device)
    check(lib().tsx_moe_mmq_quantize_route(_p(x), _p(xq), ggml_type, cols, x.stride(0), rows, _p(logits), _p(ids),
                                           _p(wts), n_expert, k, _stream(stream)), "mmq_quantize_route")
    return xq, ids, wts


def mmq_run(w, ggml_type: int, w_rows: int, w_cols: int, expert_bytes: int, n: int, xq, bounds, ids, total_rows: int,
            dst, ld_dst: int, max_rows: int = 0, stream=None) -> None:
    p = MmqProduct(w=_p(w), type=ggml_type, n=n, w_rows=w_rows, w_cols=w_cols, expert_bytes=expert_bytes, xq=_p(xq),
                   bounds=_p(bounds), ids=_p(ids), total_rows=total_rows, max_rows=max_rows, dst=_p(dst), ld_dst=ld_dst)
    check(lib().tsx_moe_mmq_run(C.byref(p), _stream(stream)), "mmq_run")


def mmq_swiglu(gu, rows: int, n_ff: int, interleaved: bool = False, h=None, stream=None) -> torch.Tensor:
    if h is None:
        h = torch.empty((rows, n_ff), dtype=torch.float32, device=gu.device)
    check(lib().tsx_moe_mmq_swiglu(_p(gu), _p(h), rows, n_ff, int(interleaved), _stream(stream)), "mmq_swiglu")
    return h


def mmq_gate_up_swiglu(w, ggml_type: int, n_ff: int, n_embd: int, expert_bytes: int, n: int, xq, x_rows: int, xids,
                       bounds, n_rows: int, hq=None, stream=None) -> torch.Tensor:
    """h = silu(x . gate) * (x . up) of every expert's sorted rows (x rows through xids), quantized into Q8_1 planes
    of n_rows rows and n_ff columns (the layout mmq_quantize writes)."""
    if hq is None:
        hq = torch.empty(mmq_q8_bytes(n_rows, n_ff), dtype=torch.uint8, device=w.device)
    check(lib().tsx_moe_mmq_gate_up_swiglu(_p(w), ggml_type, n_ff, n_embd, expert_bytes, n, _p(xq), x_rows, _p(xids),
                                            _p(bounds), n_rows, _p(hq), _stream(stream)), "mmq_gate_up_swiglu")
    return hq


# ------------------------------------------------------------------ checks and data
def subblock_sums(ggml_type: int, w, n_in: int, n_rows: int, x_q8_1, ncols: int, stream=None):
    nsub = n_in // 32
    sums = torch.empty((n_rows, ncols, nsub), dtype=torch.int32, device=w.device)
    qsums = torch.empty((n_rows, ncols, nsub), dtype=torch.int32, device=w.device)
    check(lib().tsx_moe_subblock_sums(ggml_type, _p(w), n_in, n_rows, _p(x_q8_1), ncols, _p(sums), _p(qsums),
                                      _stream(stream)), "subblock_sums")
    return sums, qsums


def quantize_weights(ggml_type: int, x: np.ndarray) -> np.ndarray:
    """Host: float32 [rows, cols] -> GGUF blocks uint8 [rows, row_bytes]."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, cols = x.shape
    rb = iq_row_bytes(ggml_type, cols)
    out = np.empty((rows, rb), dtype=np.uint8)
    check(lib().tsx_moe_quantize_weights(ggml_type, x.ctypes.data, rows, cols, out.ctypes.data), "quantize_weights")
    return out
