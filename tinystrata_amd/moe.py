"""A whole MoE FFN layer on the GPU through libtsx_moe's C ABI: routing, grouping, Q8_1 activations, the grouped
expert products, the shared expert and the router-weighted combine.

This is the call sequence of the reference engine's MoE block (src/qwen35/q36_engine.cu:2821-2925):
  decode (T <= 8):  native_router_topk -> group -> quantize_q8_1 -> native_expert_grouped -> shared expert (mmvq,
                    SwiGLU + Q8_1, mmvq) -> combine (k_moe_out without the norm)
  prefill:          native_router_topk -> route sort (count/scan/scatter) -> mmq quantize (gathered rows) ->
                    grouped gate/up product -> SwiGLU -> mmq quantize -> grouped down product -> combine via rinv
Every step stays on the device: no host round trip (the reference reads max_rows back before its MMQ launch).
Buffers are allocated once per layer shape; a call only launches kernels, so it can be captured in a HIP graph.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

from . import ops
from ._lib import ExpertLayout


def blob_stride(L: ExpertLayout) -> int:
    """Bytes between consecutive expert blobs: the blob rounded up to 256 (16-byte loads stay aligned)."""
    return (L.bytes + 255) // 256 * 256


@dataclass
class MoEWeights:
    """One layer's experts: n_expert blobs `stride` bytes apart in one device buffer, plus an optional shared one."""

    L: ExpertLayout
    n_expert: int
    stride: int
    blobs: torch.Tensor            # uint8 [n_expert * stride] on the device
    shared: torch.Tensor | None    # uint8 [stride] on the device, or None

    @property
    def base(self) -> int:
        return self.blobs.data_ptr()


def make_expert_blob(L: ExpertLayout, gate: np.ndarray, up: np.ndarray, down: np.ndarray) -> np.ndarray:
    """fp32 gate [FF, N], up [FF, N], down [N, FF] -> one quantized blob (host bytes)."""
    out = np.zeros(blob_stride(L), np.uint8)
    g = ops.quantize_weights(L.gu_type, gate).ravel()
    u = ops.quantize_weights(L.gu_type, up).ravel()
    d = ops.quantize_weights(L.d_type, down).ravel()
    out[: g.size] = g
    out[L.up_off: L.up_off + u.size] = u
    out[L.down_off: L.down_off + d.size] = d
    return out


def synthetic_pool(L: ExpertLayout, count: int, seed: int, std: float = 0.02) -> np.ndarray:
    """`count` distinct experts with N(0, std) weights quantized by this library: uint8 [count, stride]."""
    rng = np.random.default_rng(seed)
    N, FF = L.n_embd, L.n_ff
    pool = np.zeros((count, blob_stride(L)), np.uint8)
    for i in range(count):
        gate = rng.normal(0, std, (FF, N)).astype(np.float32)
        up = rng.normal(0, std, (FF, N)).astype(np.float32)
        down = rng.normal(0, std, (N, FF)).astype(np.float32)
        pool[i] = make_expert_blob(L, gate, up, down)
    return pool


def weights_from_pool(L: ExpertLayout, pool_dev: torch.Tensor, n_expert: int, order: np.ndarray,
                      shared_index: int | None) -> MoEWeights:
    """A layer whose expert x is a device copy of pool[order[x]] (every expert at its own address)."""
    stride = pool_dev.shape[1]
    idx = torch.as_tensor(np.asarray(order, np.int64), device=pool_dev.device)
    blobs = pool_dev.index_select(0, idx).reshape(-1).contiguous()
    shared = pool_dev[shared_index].clone() if shared_index is not None else None
    return MoEWeights(L=L, n_expert=n_expert, stride=stride, blobs=blobs, shared=shared)


class MoELayer:
    """Runs one MoE layer for n_tok tokens with fixed buffers (decode path for n_tok <= decode_max)."""

    def __init__(self, W: MoEWeights, k: int, n_tok: int, device: torch.device, decode_max: int = 8,
                 fused: bool = True):
        self.W, self.k, self.n_tok = W, k, n_tok
        self.side = None  # the prompt path's second stream (the shared expert), made on first use
        L = W.L
        self.N, self.FF = int(L.n_embd), int(L.n_ff)
        self.decode = n_tok <= decode_max
        n_ent = n_tok * k
        self.n_ent = n_ent
        dev = device
        f32, i32 = torch.float32, torch.int32
        self.ids = torch.empty((n_tok, k), dtype=i32, device=dev)
        self.wts = torch.empty((n_tok, k), dtype=f32, device=dev)
        self.parts = torch.empty((n_ent, self.N), dtype=f32, device=dev)
        self.sh = torch.empty((n_tok, self.N), dtype=f32, device=dev) if W.shared is not None else None
        # the two-launch decode layer where its limits allow, else the reference's call sequence kernel by kernel
        self.fused = fused and self.decode and n_ent <= 64 and self.N <= 4096 and self.FF <= 1024 and self.FF % 128 == 0
        if self.fused:
            self.lscratch = torch.empty(ops.decode_layer_scratch_bytes(n_tok, k, self.FF), dtype=torch.uint8,
                                        device=dev)
        if self.decode:
            cap = min(n_ent, W.n_expert)
            self.cap_groups = cap
            self.grp = (torch.empty(cap, dtype=torch.int64, device=dev), torch.empty(cap + 1, dtype=i32, device=dev),
                        torch.empty(1, dtype=i32, device=dev), torch.empty(n_ent, dtype=i32, device=dev),
                        torch.empty(n_ent, dtype=i32, device=dev))
            self.xq = torch.empty((n_tok, self.N // 32 * 36), dtype=torch.uint8, device=dev)
            self.scratch = torch.empty(ops.native_expert_scratch_bytes(n_ent, self.FF), dtype=torch.uint8, device=dev)
            if W.shared is not None:
                self.sg = torch.empty((n_tok, self.FF), dtype=f32, device=dev)
                self.su = torch.empty((n_tok, self.FF), dtype=f32, device=dev)
                self.shq = torch.empty((n_tok, self.FF // 32 * 36), dtype=torch.uint8, device=dev)
        else:
            self.sort = (torch.empty(W.n_expert + 1, dtype=i32, device=dev), torch.empty(n_ent, dtype=i32, device=dev),
                         torch.empty(n_ent, dtype=i32, device=dev), torch.empty(n_ent, dtype=i32, device=dev),
                         torch.empty(1, dtype=i32, device=dev))
            # gate/up with SwiGLU and the Q8_1 of h in one launch, reading each token's activations quantized once,
            # where the shape allows; else the reference's call sequence
            self.fused_prefill = (fused and self.N % 256 == 0 and self.FF % 128 == 0 and W.n_expert <= 512 and
                                  int(L.up_off) == self.FF * int(L.gu_row))
            self.mhq = torch.empty(ops.mmq_q8_bytes(n_ent, self.FF), dtype=torch.uint8, device=dev)
            if self.fused_prefill:
                self.txq = torch.empty(ops.mmq_q8_bytes(n_tok, self.N), dtype=torch.uint8, device=dev)
            else:
                self.mxq = torch.empty(ops.mmq_q8_bytes(n_ent, self.N), dtype=torch.uint8, device=dev)
                self.gu = torch.empty((n_ent, 2 * self.FF), dtype=f32, device=dev)
                self.h = torch.empty((n_ent, self.FF), dtype=f32, device=dev)
            if W.shared is not None:
                self.sh_bounds = torch.tensor([0, n_tok], dtype=i32, device=dev)
                self.shq = torch.empty(ops.mmq_q8_bytes(n_tok, self.FF), dtype=torch.uint8, device=dev)
                if not self.fused_prefill:
                    self.sxq = torch.empty(ops.mmq_q8_bytes(n_tok, self.N), dtype=torch.uint8, device=dev)
                    self.sgu = torch.empty((n_tok, 2 * self.FF), dtype=f32, device=dev)
                    self.sh_h = torch.empty((n_tok, self.FF), dtype=f32, device=dev)

    def __call__(self, x: torch.Tensor, logits: torch.Tensor, sgate: torch.Tensor | None, y: torch.Tensor,
                 norm_w: torch.Tensor | None = None, eps: float = 1e-6, h: torch.Tensor | None = None,
                 hq: torch.Tensor | None = None) -> None:
        """y += MoE(x): x, y [n_tok, N] float32; logits [n_tok, E]; sgate [n_tok] (shared expert gate logit).  With
        norm_w [N], the MoE block's end as well: h [n_tok, N] = rms(y) * norm_w and, hq given, its Q8_1 image."""
        self._norm = (norm_w, eps, h, hq)
        (self._decode if self.decode else self._prefill)(x, logits, sgate, y)

    def _combine(self, y, sgate, prow=None):
        norm_w, eps, h, hq = self._norm
        if norm_w is None:
            ops.moe_combine(y, self.parts, self.wts, self.k, prow=prow, shared=self.sh, sgate=sgate)
        else:
            ops.moe_combine_norm(y, self.parts, self.wts, self.k, norm_w, eps, h, hq, prow=prow, shared=self.sh,
                                 sgate=sgate)

    def _decode(self, x, logits, sgate, y):
        W, L, k = self.W, self.W.L, self.k
        if self.fused:
            norm_w, eps, h, hq = self._norm
            ops.moe_decode_layer(L, W.blobs, W.stride, W.n_expert, k, logits, x, y, self.ids, self.wts, self.lscratch,
                                 shared=W.shared, sgate=sgate, norm_w=norm_w, eps=eps, h=h, hq=hq)
            return
        ops.native_router_topk(logits, k, self.ids, self.wts)
        gp, gs, ng, ed, et = ops.group_entries(self.ids, k, W.n_expert, W.base, W.stride, bufs=self.grp)
        ops.quantize_q8_1_rows(x, self.xq)
        ops.native_expert_grouped(L, gp, gs, ng, ed, et, self.cap_groups, self.n_ent, self.xq, self.scratch, self.parts)
        if W.shared is not None:
            sh = W.shared
            ops.iq_mmvq(L.gu_type, sh, self.xq, self.N, self.FF, self.n_tok, y=self.sg)
            ops.iq_mmvq(L.gu_type, sh[L.up_off:], self.xq, self.N, self.FF, self.n_tok, y=self.su)
            ops.native_swiglu_quantize_q8_1(self.sg, self.su, self.shq)
            ops.iq_mmvq(L.d_type, sh[L.down_off:], self.shq, self.FF, self.N, self.n_tok, y=self.sh)
        self._combine(y, sgate)

    def _prefill(self, x, logits, sgate, y):
        W, L, k, N, FF = self.W, self.W.L, self.k, self.N, self.FF
        if self.fused_prefill:
            self._prefill_fused(x, logits, sgate, y)
            return
        ops.native_router_topk(logits, k, self.ids, self.wts)
        bounds, ed, et, rinv, mr = ops.route_sort(self.ids, k, W.n_expert, bufs=self.sort)
        n_ent = self.n_ent
        ops.mmq_quantize(x, et, L.gu_type, N, N, n_ent, xq=self.mxq)
        ops.mmq_run(W.blobs, L.gu_type, 2 * FF, N, W.stride, W.n_expert, self.mxq, bounds, None, n_ent, self.gu, 2 * FF)
        ops.mmq_swiglu(self.gu, n_ent, FF, False, h=self.h)
        ops.mmq_quantize(self.h, None, L.d_type, FF, FF, n_ent, xq=self.mhq)
        ops.mmq_run(W.blobs[L.down_off:], L.d_type, N, FF, W.stride, W.n_expert, self.mhq, bounds, None, n_ent,
                    self.parts, N)
        if W.shared is not None:
            T = self.n_tok
            sh = W.shared
            ops.mmq_quantize(x, None, L.gu_type, N, N, T, xq=self.sxq)
            ops.mmq_run(sh, L.gu_type, 2 * FF, N, W.stride, 1, self.sxq, self.sh_bounds, None, T, self.sgu, 2 * FF)
            ops.mmq_swiglu(self.sgu, T, FF, False, h=self.sh_h)
            ops.mmq_quantize(self.sh_h, None, L.d_type, FF, FF, T, xq=self.shq)
            ops.mmq_run(sh[L.down_off:], L.d_type, N, FF, W.stride, 1, self.shq, self.sh_bounds, None, T, self.sh, N)
        self._combine(y, sgate, prow=rinv)

    def _prefill_fused(self, x, logits, sgate, y):
        W, L, k, N, FF, T = self.W, self.W.L, self.k, self.N, self.FF, self.n_tok
        main = torch.cuda.current_stream()
        # every token's Q8_1 row once (routed rows read it via et) and the router's picks, in one launch
        ops.mmq_quantize_route(x, L.gu_type, logits, k, xq=self.txq, ids=self.ids, wts=self.wts)
        if W.shared is not None:
            if self.side is None:
                self.side = torch.cuda.Stream(device=x.device)
                self.x_ready = torch.cuda.Event()
            self.x_ready.record(main)
        bounds, ed, et, rinv, mr = ops.route_sort(self.ids, k, W.n_expert, bufs=self.sort)
        ops.mmq_gate_up_swiglu(W.blobs, L.gu_type, FF, N, W.stride, W.n_expert, self.txq, T, et, bounds, self.n_ent,
                               hq=self.mhq)
        ops.mmq_run(W.blobs[L.down_off:], L.d_type, N, FF, W.stride, W.n_expert, self.mhq, bounds, None, self.n_ent,
                    self.parts, N)
        if W.shared is not None:
            # the shared expert's two products on a second stream: they need only the tokens' Q8_1, so they run
            # beside the router, the sort and the routed products, filling the CUs those launches leave idle.  They
            # are issued after the routed chain so that a captured graph keeps that chain and the combine on one queue
            # (a wait across queues left 6-10 us gaps on the critical path); the shared chain ends long before the
            # combine waits for it
            self.side.wait_event(self.x_ready)
            with torch.cuda.stream(self.side):
                sh = W.shared
                ops.mmq_gate_up_swiglu(sh, L.gu_type, FF, N, W.stride, 1, self.txq, T, None, self.sh_bounds, T,
                                       hq=self.shq)
                ops.mmq_run(sh[L.down_off:], L.d_type, N, FF, W.stride, 1, self.shq, self.sh_bounds, None, T, self.sh,
                            N)
            main.wait_stream(self.side)
        self._combine(y, sgate, prow=rinv)
