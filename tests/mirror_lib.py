"""ctypes view of tinystrata_amd/libtsx_mirror_check.so: the test library that calls the C++ operator API
(strata_kernels.hpp) from C++ (source: tests/mirror/mirror_check.cpp)."""
from __future__ import annotations

import ctypes as C
import functools
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
LIB = ROOT / "tinystrata_amd" / "libtsx_mirror_check.so"

P, I, I64, U64 = C.c_void_p, C.c_int, C.c_int64, C.c_uint64

SIGNATURES = {
    "smc_expert_layout": (I, [I, I, I64, I64, P]),
    "smc_expert_scratch_bytes": (U64, [I64, I64]),
    "smc_expert_grouped": (I, [I, I, I64, I64, P, P, P, P, P, I64, I64, P, P, P, P, I64]),
    "smc_quantize_q8_1_rows": (I, [P, I64, I64, P, P]),
    "smc_router_topk": (I, [P, P, P, I, I, I, P, C.c_char_p, I]),
    "smc_router_topk_supported": (I, [I, I]),
    "smc_mmvq": (I, [I, P, P, P, I, I, I, P, C.c_char_p, I]),
    "smc_mmvq_weight_bytes": (I, [I, I, I, P, C.c_char_p, I]),
    "smc_mmq_q8_bytes": (U64, [I64, I64]),
    "smc_mmq_supported": (I, [I, I64]),
    "smc_mmq_quantize": (I, [P, P, P, I, I64, I64, I64, P]),
    "smc_mmq_run": (I, [P, I, I64, I64, U64, I, P, P, P, I64, I64, P, I64, P]),
    "smc_mmq_swiglu": (I, [P, P, I64, I64, I, P]),
    "smc_mmq_iota": (I, [P, I64, P]),
    "smc_margin_rows": (I, [I64, I, P]),
    "smc_margin_rows_null": (I, [I64, I]),
    "smc_table_rows": (U64, [U64, U64, I]),
    "smc_table_rows_default": (U64, [U64, U64]),
    "smc_ids_layout": (I, [U64, U64, P]),
    "smc_packed_ids_layout": (I, [U64, U64, U64, U64, P]),
    "smc_tile_cols": (I, [P]),
}


@functools.lru_cache(maxsize=None)
def lib() -> C.CDLL:
    if not LIB.exists():
        raise RuntimeError(f"{LIB} is not built (run __graft_entry__.build())")
    L = C.CDLL(str(LIB))
    for name, (res, args) in SIGNATURES.items():
        f = getattr(L, name)
        f.restype, f.argtypes = res, args
    return L


def msg_buf() -> C.Array:
    return C.create_string_buffer(512)
