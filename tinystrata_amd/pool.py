"""The hybrid CPU/GPU expert split through libtsx_moe's C ABI (include/tsx_pool.h): the CPU expert rows, the worker
pool (two batch slots joined by attach-and-recheck, per-expert chunk cursors), and a decode MoE layer whose experts without an HBM slot run on
the pool while the GPU runs the resident ones.

Mirrors strata::kernels::cpu::ExpertPool (include/strata/kernels/cpu/pool.hpp:111-260), the native expert rows
(include/strata/kernels/cpu/native_expert.hpp:41-65) and the engine's hybrid MoE block (moe_hybrid_gpu /
moe_hybrid_cpu, src/qwen35/q36_engine.cu:3052-3209).  The arithmetic and the threads are the library's (C++); this
module holds handles, host buffers and the call order.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import torch

from . import ops
from ._lib import CPU_MAXT, TSX_ERR_STALLED, CpuFmt, CpuJob, HybridLayerArgs, check, lib
from .moe import MoEWeights


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def cpu_fmt(gu_type: int, d_type: int, n_embd: int, n_ff: int) -> CpuFmt:
    """The CPU geometry of a layer (reference native_fmt)."""
    f = CpuFmt()
    check(lib().tsx_cpu_fmt_init(gu_type, d_type, n_embd, n_ff, C.byref(f)), "cpu_fmt")
    return f


def cpu_quant_act(f: CpuFmt, x: np.ndarray) -> np.ndarray:
    """x [n_embd] float32 -> Q8_1 bytes (reference native_quant_act)."""
    x = np.ascontiguousarray(x, np.float32)
    out = np.zeros(f.act_bytes, np.uint8)
    check(lib().tsx_cpu_quant_act(C.byref(f), _ptr(x), _ptr(out)), "cpu_quant_act")
    return out


def cpu_quant_h(f: CpuFmt, h: np.ndarray) -> np.ndarray:
    """h [n_ff] float32 -> Q8_1 bytes (reference native_quant_h)."""
    h = np.ascontiguousarray(h, np.float32)
    out = np.zeros(f.h_bytes, np.uint8)
    check(lib().tsx_cpu_quant_h(C.byref(f), _ptr(h), _ptr(out)), "cpu_quant_h")
    return out


def _ptrs(arrs) -> C.Array:
    return (C.c_void_p * len(arrs))(*[_ptr(a) for a in arrs])


def cpu_gu_rows(f: CpuFmt, blob: np.ndarray, acts: list, r0: int = 0, r1: int | None = None) -> np.ndarray:
    """ff[t][r] = silu(gate_r . act_t) * (up_r . act_t), rows [r0, r1) (reference native_gu_rows)."""
    r1 = int(f.n_ff) if r1 is None else r1
    ff = [np.zeros(int(f.n_ff), np.float32) for _ in acts]
    check(lib().tsx_cpu_gu_rows(C.byref(f), _ptr(blob), _ptrs(acts), len(acts), _ptrs(ff), r0, r1), "cpu_gu_rows")
    return np.stack(ff)


def cpu_down_rows(f: CpuFmt, blob: np.ndarray, hqs: list, r0: int = 0, r1: int | None = None) -> np.ndarray:
    """out[t][r] = down_r . hq_t, rows [r0, r1) (reference native_down_rows)."""
    r1 = int(f.n_embd) if r1 is None else r1
    out = [np.zeros(int(f.n_embd), np.float32) for _ in hqs]
    check(lib().tsx_cpu_down_rows(C.byref(f), _ptr(blob), _ptrs(hqs), len(hqs), _ptrs(out), r0, r1),
          "cpu_down_rows")
    return np.stack(out)


class ExpertPool:
    """CPU worker threads evaluating native experts in row tasks (reference strata::kernels::cpu::ExpertPool)."""

    def __init__(self, n_workers: int = 0, pin: bool = True, host_works: bool = True, tasks: int = 0):
        h = C.c_void_p()
        check(lib().tsx_pool_create(n_workers, int(pin), int(host_works), tasks, C.byref(h)), "pool create")
        self._h = h
        self._stalled = []

    @property
    def handle(self) -> C.c_void_p:
        return self._h

    @property
    def workers(self) -> int:
        return lib().tsx_pool_workers(self._h)

    @property
    def host_works(self) -> bool:
        return bool(lib().tsx_pool_host_works(self._h))

    def diag(self) -> str:
        """One line: the batch counters and every worker's state (reference ExpertPool::diag)."""
        buf = C.create_string_buffer(4096)
        check(lib().tsx_pool_diag(self._h, buf, len(buf)), "pool diag")
        return buf.value.decode()

    def set_spin_us(self, us: int) -> None:
        check(lib().tsx_pool_set_spin_us(self._h, us), "pool set_spin_us")

    def set_stall_ms(self, ms: int) -> None:
        check(lib().tsx_pool_set_stall_ms(self._h, ms), "pool set_stall_ms")

    def run(self, f: CpuFmt, jobs: list) -> None:
        """jobs: (blob ndarray, [act ndarray per token], [out float32 ndarray per token]) with 1..8 tokens each;
        the outputs are written in place (reference run_split_multi_native)."""
        arr = (CpuJob * max(1, len(jobs)))()
        for i, (blob, acts, outs) in enumerate(jobs):
            assert 1 <= len(acts) == len(outs) <= CPU_MAXT
            arr[i].blob = _ptr(blob)
            arr[i].nt = len(acts)
            for t in range(len(acts)):
                assert outs[t].dtype == np.float32 and outs[t].flags.c_contiguous
                arr[i].act[t] = _ptr(acts[t])
                arr[i].out[t] = _ptr(outs[t])
        rc = lib().tsx_pool_run(self._h, C.byref(f), arr, len(jobs))
        if rc == TSX_ERR_STALLED:
            # the library copied the job table, but workers of the stalled batch may still read these tokens' rows
            # and write their outputs: every array of such a run stays alive until close() has joined the workers
            self._stalled.append(jobs)
        check(rc, "pool run")

    def stats(self) -> dict:
        ms = (C.c_double * 6)()
        b = C.c_int64()
        check(lib().tsx_pool_stats(self._h, ms, C.byref(b)), "pool stats")
        keys = ("wait_slot", "drain", "gate_up", "quant_h", "down", "wait_h")
        return {**{k: ms[i] for i, k in enumerate(keys)}, "bytes": b.value}

    def close(self) -> None:
        if self._h:
            lib().tsx_pool_destroy(self._h)  # joins the workers
            self._h = C.c_void_p()
        self._stalled = []

    def __enter__(self) -> "ExpertPool":
        return self

    def __exit__(self, *exc) -> None:
        self.close()

    def __del__(self) -> None:
        try:
            self.close()
        except Exception:
            pass


def hybrid_cpu(pool: ExpertPool, f: CpuFmt, host_blobs: np.ndarray, stride: int, slot_of: np.ndarray, k: int,
               ids: np.ndarray, x: np.ndarray, cpu_out: np.ndarray, miss: np.ndarray) -> int:
    """The CPU half of a hybrid layer (tsx_moe_hybrid_cpu): rows of the missed entries into cpu_out (compact, entry
    order), miss[e] = row or -1; returns the number of misses."""
    n_tok = ids.shape[0]
    slot_of = np.ascontiguousarray(slot_of, np.int32)
    ids = np.ascontiguousarray(ids, np.int32)
    x = np.ascontiguousarray(x, np.float32)
    nm = C.c_int32()
    rc = lib().tsx_moe_hybrid_cpu(pool.handle, C.byref(f), _ptr(host_blobs), stride, _ptr(slot_of), len(slot_of), k,
                                  n_tok, _ptr(ids), _ptr(x), _ptr(cpu_out), _ptr(miss), C.byref(nm))
    if rc == TSX_ERR_STALLED:
        # workers of the stalled batch may still read the blobs and the activations and write cpu_out: they stay
        # alive until the pool's close() has joined the workers, as ExpertPool.run keeps its arrays
        pool._stalled.append((host_blobs, x, cpu_out, miss, ids, slot_of))
    check(rc, "hybrid_cpu")
    return nm.value


class HybridMoELayer:
    """A decode MoE layer (n_tok <= 8) whose experts live in host memory, `slots` of them also in HBM.

    GPU half: routing, the routing and the tokens' x to the host, the resident entries grouped into their slots and
    run by the grouped expert kernels, the shared expert.  CPU half, while the GPU works: the missed entries on the
    pool.  Then the CPU rows are uploaded, merged into the entries' rows, and the combine runs on the GPU."""

    def __init__(self, W: MoEWeights, host_blobs: np.ndarray, resident: np.ndarray, k: int, n_tok: int,
                 device: torch.device, pool: ExpertPool):
        L = W.L
        self.W, self.k, self.n_tok, self.pool = W, k, n_tok, pool
        self.N, self.FF = int(L.n_embd), int(L.n_ff)
        self.n_expert = int(host_blobs.shape[0]) if host_blobs.ndim == 2 else W.n_expert
        self.host_blobs = np.ascontiguousarray(host_blobs).reshape(-1)
        self.stride = W.stride
        slot_of = np.full(self.n_expert, -1, np.int32)
        resident = np.asarray(resident, np.int64)
        slot_of[resident] = np.arange(len(resident), dtype=np.int32)
        self.slot_of = slot_of
        self.f = cpu_fmt(L.gu_type, L.d_type, self.N, self.FF)
        dev = device
        n_ent = n_tok * k
        self.n_ent = n_ent
        f32, i32 = torch.float32, torch.int32
        self.d_slot_of = torch.as_tensor(slot_of, device=dev)
        # the resident experts' blobs, slot s = expert resident[s]
        self.slots = torch.empty(max(1, len(resident)) * W.stride, dtype=torch.uint8, device=dev)
        if len(resident):
            src = torch.as_tensor(host_blobs.reshape(self.n_expert, -1)[resident].reshape(-1))
            self.slots[: src.numel()].copy_(src)
        self.ids = torch.empty((n_tok, k), dtype=i32, device=dev)
        self.wts = torch.empty((n_tok, k), dtype=f32, device=dev)
        self.parts = torch.empty((n_ent, self.N), dtype=f32, device=dev)
        cap = min(n_ent, self.n_expert)
        self.cap_groups = cap
        self.grp = (torch.empty(cap, dtype=torch.int64, device=dev), torch.empty(cap + 1, dtype=i32, device=dev),
                    torch.empty(1, dtype=i32, device=dev), torch.empty(n_ent, dtype=i32, device=dev),
                    torch.empty(n_ent, dtype=i32, device=dev))
        self.xq = torch.empty((n_tok, self.N // 32 * 36), dtype=torch.uint8, device=dev)
        self.scratch = torch.empty(ops.native_expert_scratch_bytes(n_ent, self.FF), dtype=torch.uint8, device=dev)
        self.sh = torch.empty((n_tok, self.N), dtype=f32, device=dev) if W.shared is not None else None
        if W.shared is not None:
            self.sg = torch.empty((n_tok, self.FF), dtype=f32, device=dev)
            self.su = torch.empty((n_tok, self.FF), dtype=f32, device=dev)
            self.shq = torch.empty((n_tok, self.FF // 32 * 36), dtype=torch.uint8, device=dev)
        # pinned host buffers of the round trip
        self.h_ids = torch.empty((n_tok, k), dtype=i32, pin_memory=True)
        self.h_x = torch.empty((n_tok, self.N), dtype=f32, pin_memory=True)
        self.h_rows = torch.empty((n_ent, self.N), dtype=f32, pin_memory=True)
        self.h_miss = torch.empty(n_ent, dtype=i32, pin_memory=True)
        self.d_rows = torch.empty((n_ent, self.N), dtype=f32, device=dev)
        self.d_miss = torch.empty(n_ent, dtype=i32, device=dev)
        self.n_miss = 0

        A = HybridLayerArgs()
        A.L = L
        A.n_expert, A.k, A.n_tok, A.sg_stride = self.n_expert, k, n_tok, 1
        A.host_blobs, A.stride, A.slot_of = self.host_blobs.ctypes.data, self.stride, self.slot_of.ctypes.data
        A.d_slot_of, A.slots = self.d_slot_of.data_ptr(), self.slots.data_ptr()
        A.shared = W.shared.data_ptr() if W.shared is not None else None
        for name in ("ids", "wts", "xq", "scratch", "parts", "h_ids", "h_x", "h_rows", "h_miss", "d_rows", "d_miss"):
            setattr(A, name, getattr(self, name).data_ptr())
        A.grp_ptr, A.grp_start, A.n_groups, A.ent_dst, A.ent_tok = (t.data_ptr() for t in self.grp)
        if W.shared is not None:
            A.sh_gate, A.sh_up, A.sh_hq, A.sh_out = (t.data_ptr() for t in (self.sg, self.su, self.shq, self.sh))
        self.args = A

    def __call__(self, x: torch.Tensor, logits: torch.Tensor, sgate: torch.Tensor | None, y: torch.Tensor) -> None:
        """y += MoE(x) as MoELayer does, with the non-resident experts computed on the CPU pool: one library call
        (tsx_moe_hybrid_decode_layer) enqueues the GPU half, runs the CPU half while the GPU works, and enqueues the
        merge and the combine."""
        A = self.args
        A.x, A.logits, A.y = x.data_ptr(), logits.data_ptr(), y.data_ptr()
        A.sgate = sgate.data_ptr() if sgate is not None else None
        rc = lib().tsx_moe_hybrid_decode_layer(self.pool.handle, C.byref(self.f), C.byref(A),
                                               torch.cuda.current_stream(y.device).cuda_stream)
        if rc == TSX_ERR_STALLED:
            # the stalled batch's workers may still read the host blobs and x and write the CPU rows
            self.pool._stalled.append((self.host_blobs, self.h_x, self.h_rows))
        check(rc, "hybrid layer")
        self.n_miss = A.n_miss
