"""ctypes binding of libtsx_moe.so (the C ABI declared in include/tsx_moe.h).

The library is built in-tree by tinystrata_amd.build; nothing here falls back to another implementation: a missing
library raises, so a GPU run can never pass on a silent host or PyTorch path.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libtsx_moe.so"

ABI_VERSION = 1
TSX_OK, TSX_ERR_UNSUPPORTED, TSX_ERR_ARG, TSX_ERR_FORMAT, TSX_ERR_NOT_FOUND, TSX_ERR_STALLED = 0, -1, -2, -3, -4, -5
CPU_MAXT, POOL_MAX_SPLIT = 8, 96  # tokens per CPU job, experts per pool batch (include/tsx_pool.h)

# type ids (ggml's)
Q4_0, Q8_0, Q8_1, Q4_K, Q6_K, Q8_K, IQ3_XXS, IQ3_S = 2, 8, 9, 12, 14, 15, 18, 21


class ExpertLayout(C.Structure):
    """tsx_expert_layout: the [gate | up | down] blob of one expert (reference NativeExpertLayout)."""

    _fields_ = [
        ("gu_type", C.c_int32),
        ("d_type", C.c_int32),
        ("n_embd", C.c_int64),
        ("n_ff", C.c_int64),
        ("gu_row", C.c_uint64),
        ("d_row", C.c_uint64),
        ("up_off", C.c_uint64),
        ("down_off", C.c_uint64),
        ("bytes", C.c_uint64),
    ]


class MmqProduct(C.Structure):
    """tsx_mmq_product: one grouped prompt product (reference prefill::mmq::Product)."""

    _fields_ = [
        ("w", C.c_void_p),
        ("type", C.c_int32),
        ("n", C.c_int32),
        ("w_rows", C.c_int64),
        ("w_cols", C.c_int64),
        ("expert_bytes", C.c_uint64),
        ("xq", C.c_void_p),
        ("bounds", C.c_void_p),
        ("ids", C.c_void_p),
        ("total_rows", C.c_int64),
        ("max_rows", C.c_int64),
        ("dst", C.c_void_p),
        ("ld_dst", C.c_int64),
    ]


class MmvqIds(C.Structure):
    """tsx_mmvq_ids: matrices picked on the device through a table (reference MmvqIds)."""

    _fields_ = [
        ("table", C.c_void_p),
        ("ids", C.c_void_p),
        ("n_table", C.c_int32),
        ("offset", C.c_uint64),
        ("x", C.c_void_p),
        ("x_stride", C.c_uint64),
        ("x_every", C.c_int32),
        ("y", C.c_void_p),
        ("y_stride", C.c_uint64),
    ]


class MmvqSlots(C.Structure):
    """tsx_mmvq_slots: up to 8 matrices given by the host (reference MmvqSlots)."""

    _fields_ = [("w", C.c_void_p * 8), ("x", C.c_void_p * 8), ("y", C.c_void_p * 8)]


class GgufTensor(C.Structure):
    """tsx_gguf_tensor: one entry of a GGUF tensor directory (reference TensorInfo)."""

    _fields_ = [
        ("name", C.c_char_p),
        ("type", C.c_int32),
        ("n_dims", C.c_int32),
        ("ne", C.c_int64 * 4),
        ("offset", C.c_uint64),
        ("bytes", C.c_uint64),
        ("data", C.c_void_p),
        ("shard", C.c_int32),
    ]


class GgufExperts(C.Structure):
    """tsx_gguf_experts: one layer's routed (or shared) experts inside the mapped model."""

    _fields_ = [
        ("L", ExpertLayout),
        ("stride", C.c_uint64),
        ("n_expert", C.c_int64),
        ("gate", C.c_void_p),
        ("up", C.c_void_p),
        ("down", C.c_void_p),
    ]


P, I32, I64, U64, SZ = C.c_void_p, C.c_int, C.c_int64, C.c_uint64, C.c_size_t

class CpuFmt(C.Structure):
    """tsx_cpu_fmt: one layer's expert geometry on the CPU (reference NativeFmt)."""

    _fields_ = [
        ("gu_type", C.c_int32),
        ("d_type", C.c_int32),
        ("gu_act", C.c_int32),
        ("d_act", C.c_int32),
        ("n_embd", C.c_int64),
        ("n_ff", C.c_int64),
        ("gu_row", C.c_uint64),
        ("d_row", C.c_uint64),
        ("up_off", C.c_uint64),
        ("down_off", C.c_uint64),
        ("bytes", C.c_uint64),
        ("act_bytes", C.c_uint64),
        ("h_bytes", C.c_uint64),
    ]


class CpuJob(C.Structure):
    """tsx_cpu_job: one expert applied to up to 8 tokens (reference ExpertJobMulti)."""

    _fields_ = [
        ("blob", C.c_void_p),
        ("nt", C.c_int32),
        ("pad", C.c_int32),
        ("out", C.c_void_p * CPU_MAXT),
        ("act", C.c_void_p * CPU_MAXT),
    ]


class HybridLayerArgs(C.Structure):
    """tsx_hybrid_layer: the buffers of one hybrid decode layer call."""

    _fields_ = [("L", ExpertLayout), ("n_expert", C.c_int32), ("k", C.c_int32), ("n_tok", C.c_int32),
                ("sg_stride", C.c_int32)] + [(n, C.c_void_p) for n in (
                    "host_blobs", "stride", "slot_of", "d_slot_of", "slots", "shared", "sgate", "x", "logits", "y",
                    "ids", "wts", "grp_ptr", "grp_start", "n_groups", "ent_dst", "ent_tok", "xq", "scratch", "parts",
                    "sh_gate", "sh_up", "sh_hq", "sh_out", "h_ids", "h_x", "h_rows", "h_miss", "d_rows",
                    "d_miss")] + [("n_miss", C.c_int32), ("pad", C.c_int32)]


# name -> (restype, argtypes); the list is the whole C ABI, checked against include/tsx_moe.h by the tests
SIGNATURES = {
    "tsx_moe_abi": (I32, []),
    "tsx_moe_init": (I32, [I32]),
    "tsx_moe_last_error": (C.c_char_p, []),
    "tsx_moe_row_bytes": (SZ, [I32, I64]),
    "tsx_moe_expert_layout": (I32, [I32, I32, I64, I64, C.POINTER(ExpertLayout)]),
    "tsx_moe_expert_supported": (I32, [I32, I32, I64, I64]),
    "tsx_moe_expert_scratch_bytes": (SZ, [I64, I64]),
    "tsx_moe_expert_scratch_hq_offset": (SZ, [I64, I64]),
    "tsx_moe_quantize_q8_1": (I32, [P, I64, I64, P, P]),
    "tsx_moe_swiglu_quantize_q8_1": (I32, [P, P, I64, P, P]),
    "tsx_moe_expert_grouped": (I32, [C.POINTER(ExpertLayout), P, P, P, P, P, I64, I64, P, P, P, P, I64]),
    "tsx_moe_mmvq": (I32, [I32, P, P, P, I32, I32, I32, P]),
    "tsx_moe_mmvq_ids_supported": (I32, [I32]),
    "tsx_moe_mmvq_ids": (I32, [I32, C.POINTER(MmvqIds), I32, I32, I32, P]),
    "tsx_moe_mmvq_slots": (I32, [I32, C.POINTER(MmvqSlots), I32, I32, I32, P]),
    "tsx_moe_decode_layer_scratch_bytes": (SZ, [I32, I32, I64]),
    "tsx_moe_decode_layer": (I32, [C.POINTER(ExpertLayout), P, U64, I32, I32, I32, P, P, P, P, I32, P, P, P, P, P]),
    "tsx_moe_decode_layer_norm": (I32, [C.POINTER(ExpertLayout), P, U64, I32, I32, I32, P, P, P, P, I32, P, P, P, P,
                                        C.c_float, P, P, P, P]),
    "tsx_moe_decode_layer_noalloc_max_bytes": (SZ, []),
    "tsx_moe_decode_layer_noalloc": (I32, [C.POINTER(ExpertLayout), P, U64, I32, I32, I32, P, P, P, P, I32, P, P, P, P]),
    "tsx_moe_router_topk": (I32, [P, P, P, I32, I32, I32, P]),
    "tsx_moe_group": (I32, [P, I32, I32, I32, P, U64, P, P, P, P, P, P]),
    "tsx_moe_group_resident": (I32, [P, I32, I32, I32, P, P, U64, P, P, P, P, P, P]),
    "tsx_moe_merge_rows": (I32, [P, P, P, I32, I64, P]),
    "tsx_moe_route_sort": (I32, [P, I32, I32, I32, P, P, P, P, P, P]),
    "tsx_moe_combine": (I32, [P, P, P, P, I32, P, P, I32, I32, I32, P]),
    "tsx_moe_combine_norm": (I32, [P, P, P, P, I32, P, P, I32, I32, I32, P, C.c_float, P, P, P]),
    "tsx_moe_mmq_q8_bytes": (SZ, [I64, I64]),
    "tsx_moe_mmq_quantize": (I32, [P, P, P, I32, I64, I64, I64, P]),
    "tsx_moe_mmq_quantize_route": (I32, [P, P, I32, I64, I64, I64, P, P, P, I32, I32, P]),
    "tsx_moe_mmq_run": (I32, [C.POINTER(MmqProduct), P]),
    "tsx_moe_mmq_swiglu": (I32, [P, P, I64, I64, I32, P]),
    "tsx_moe_mmq_gate_up_swiglu": (I32, [P, I32, I64, I64, U64, I32, P, I64, P, P, I64, P, P]),
    "tsx_moe_subblock_sums": (I32, [I32, P, I64, I64, P, I64, P, P, P]),
    "tsx_moe_quantize_weights": (I32, [I32, P, I64, I64, P]),
}

# the GGUF reader of include/tsx_gguf.h
GGUF_SIGNATURES = {
    "tsx_gguf_block_geometry": (I32, [I32, C.POINTER(C.c_int), C.POINTER(C.c_int)]),
    "tsx_gguf_split_paths": (I32, [C.c_char_p, P, SZ, C.POINTER(C.c_int), C.POINTER(C.c_size_t)]),
    "tsx_gguf_open": (I32, [C.POINTER(C.c_char_p), I32, C.POINTER(P)]),
    "tsx_gguf_open_model": (I32, [C.c_char_p, C.POINTER(P)]),
    "tsx_gguf_close": (None, [P]),
    "tsx_gguf_shard_count": (I32, [P]),
    "tsx_gguf_shard_info": (I32, [P, I32, C.POINTER(C.c_uint32), C.POINTER(U64), C.POINTER(U64), C.POINTER(U64)]),
    "tsx_gguf_tensor_count": (I64, [P]),
    "tsx_gguf_tensor_at": (I32, [P, I64, C.POINTER(GgufTensor)]),
    "tsx_gguf_find": (I32, [P, C.c_char_p, C.POINTER(GgufTensor)]),
    "tsx_gguf_meta_count": (I32, [P]),
    "tsx_gguf_meta_key": (C.c_char_p, [P, I32]),
    "tsx_gguf_meta": (I32, [P, C.c_char_p, C.POINTER(C.c_int), C.POINTER(U64), C.POINTER(I64), C.POINTER(C.c_double),
                            C.POINTER(C.c_char_p), C.POINTER(C.c_int), C.POINTER(U64)]),
    "tsx_gguf_meta_item": (I32, [P, C.c_char_p, U64, C.POINTER(U64), C.POINTER(C.c_double), C.POINTER(C.c_char_p)]),
    "tsx_gguf_layer_experts": (I32, [P, I32, I32, C.POINTER(GgufExperts)]),
    "tsx_gguf_expert_blob": (I32, [C.POINTER(GgufExperts), I64, P]),
    "tsx_gguf_upload_experts": (I32, [C.POINTER(GgufExperts), I64, I64, P, U64, P]),
}

# the CPU expert rows, the pool and the hybrid split of include/tsx_pool.h
POOL_SIGNATURES = {
    "tsx_cpu_fmt_init": (I32, [I32, I32, I64, I64, C.POINTER(CpuFmt)]),
    "tsx_cpu_quant_act": (I32, [C.POINTER(CpuFmt), P, P]),
    "tsx_cpu_quant_h": (I32, [C.POINTER(CpuFmt), P, P]),
    "tsx_cpu_gu_rows": (I32, [C.POINTER(CpuFmt), P, C.POINTER(P), I32, C.POINTER(P), I32, I32]),
    "tsx_cpu_down_rows": (I32, [C.POINTER(CpuFmt), P, C.POINTER(P), I32, C.POINTER(P), I32, I32]),
    "tsx_pool_create": (I32, [I32, I32, I32, I32, C.POINTER(P)]),
    "tsx_pool_destroy": (None, [P]),
    "tsx_pool_workers": (I32, [P]),
    "tsx_pool_host_works": (I32, [P]),
    "tsx_pool_run": (I32, [P, C.POINTER(CpuFmt), C.POINTER(CpuJob), I32]),
    "tsx_pool_stats": (I32, [P, C.POINTER(C.c_double), C.POINTER(I64)]),
    "tsx_pool_diag": (I32, [P, P, SZ]),
    "tsx_pool_set_spin_us": (I32, [P, I64]),
    "tsx_pool_set_stall_ms": (I32, [P, I64]),
    "tsx_moe_hybrid_cpu": (I32, [P, C.POINTER(CpuFmt), P, U64, P, I32, I32, I32, P, P, P, P, P]),
    "tsx_moe_hybrid_decode_layer": (I32, [P, C.POINTER(CpuFmt), C.POINTER(HybridLayerArgs), P]),
}

_lib: C.CDLL | None = None


class TsxError(RuntimeError):
    def __init__(self, what: str, rc: int, msg: str):
        super().__init__(f"{what} failed ({rc}): {msg}")
        self.rc = rc


def lib() -> C.CDLL:
    """The loaded library; raises FileNotFoundError when it has not been built (no fallback exists)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise FileNotFoundError(
                f"{LIB_PATH} is missing: build it with `python -m tinystrata_amd.build` (hipcc, gfx950)"
            )
        h = C.CDLL(str(LIB_PATH))
        for name, (res, args) in {**SIGNATURES, **GGUF_SIGNATURES, **POOL_SIGNATURES}.items():
            f = getattr(h, name)
            f.restype = res
            f.argtypes = args
        abi = h.tsx_moe_abi()
        if abi // 100000 != ABI_VERSION or abi % 100000 != C.sizeof(MmqProduct):
            raise RuntimeError(f"{LIB_PATH}: ABI {abi} does not match this binding")
        _lib = h
    return _lib


def check(rc: int, what: str) -> None:
    if rc != TSX_OK:
        raise TsxError(what, rc, lib().tsx_moe_last_error().decode(errors="replace"))
