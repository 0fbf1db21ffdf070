"""The C ABI boundary without a GPU: the library loads, exports exactly what include/tsx_moe.h declares, and its host
logic (layouts, sizes, argument checks, error codes and messages) behaves as documented."""
import ctypes as C
import re
import shutil
import subprocess
from pathlib import Path

import numpy as np
import pytest

from tinystrata_amd import _lib, ops

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "tsx_moe.h"


def declared():
    return sorted(set(re.findall(r"TSX_API\s+[\w\s\*]+?\b(tsx_moe_\w+)\s*\(", HEADER.read_text())))


def test_every_declared_symbol_is_exported_and_bound():
    names = declared()
    assert len(names) >= 20
    lib = _lib.lib()
    for n in names:
        assert hasattr(lib, n), n
    assert sorted(_lib.SIGNATURES) == names


def test_every_gguf_symbol_is_exported_and_bound():
    names = sorted(set(re.findall(r"TSX_API\s+[\w\s\*]+?\b(tsx_gguf_\w+)\s*\(",
                                  (ROOT / "include" / "tsx_gguf.h").read_text())))
    assert len(names) >= 15
    lib = _lib.lib()
    for n in names:
        assert hasattr(lib, n), n
    assert sorted(_lib.GGUF_SIGNATURES) == names


def test_every_pool_symbol_is_exported_and_bound():
    names = sorted(set(re.findall(r"TSX_API\s+[\w\s\*]+?\b(tsx_(?:cpu|pool|moe)_\w+)\s*\(",
                                  (ROOT / "include" / "tsx_pool.h").read_text())))
    assert len(names) >= 14
    lib = _lib.lib()
    for n in names:
        assert hasattr(lib, n), n
    assert sorted(_lib.POOL_SIGNATURES) == names


def test_abi_handshake():
    lib = _lib.lib()
    v = lib.tsx_moe_abi()
    assert v // 100000 == _lib.ABI_VERSION and v % 100000 == C.sizeof(_lib.MmqProduct)


def test_scratch_bytes_reference_formula():
    # src/kernels/cuda/iq_kernels.cu:2140-2143: 3 x round256(cap*FF*4) + round256(cap*FF/32*36)
    for cap, ff in [(8, 512), (9, 768), (1, 32), (4096, 512)]:
        f = cap * ff * 4
        r = lambda v: (v + 255) // 256 * 256
        assert ops.native_expert_scratch_bytes(cap, ff) == 3 * r(f) + r(cap * ff // 32 * 36)
        assert ops.scratch_hq_offset(cap, ff) == 3 * r(f)


def test_decode_layer_scratch_covers_fp32_h():
    """The decode layer's scratch holds the tables and h as Q8_1 planes, or in fp32 (4 bytes per value, every routed
    position and every token's shared one) wherever a slot-by-slot launch A may take the call: one token, or up to four
    tokens at n_ff <= 512.  The multi-token launch A once wrote fp32 h into a scratch sized for the planes."""
    r = lambda v: (v + 255) // 256 * 256
    for T, k, ff in [(1, 8, 512), (2, 8, 512), (3, 8, 512), (4, 8, 512), (4, 11, 256), (1, 16, 1024)]:
        need = (T * k + T) * ff * 4
        got = ops.decode_layer_scratch_bytes(T, k, ff)
        assert got >= need + 256, (T, k, ff, got, need)    # the tables come first (at least 256 bytes)
    for T, k, ff in [(5, 8, 512), (8, 8, 512), (4, 8, 1024), (2, 8, 768)]:
        planes = (T * k + T) * (ff + ff // 32 * 4)         # codes and a float scale per 32
        got = ops.decode_layer_scratch_bytes(T, k, ff)
        assert got >= planes and got < (T * k + T) * ff * 4, (T, k, ff, got)


def test_decode_layer_refuses_a_short_scratch():
    """The Python wrapper checks the scratch against the call's token count before any launch (a layer built for eight
    tokens would hold Q8_1 planes only, too little for four tokens' fp32 h)."""
    import torch
    L = ops.native_expert_layout(_lib.IQ3_XXS, _lib.IQ3_S, 2048, 512)
    x = torch.zeros(4, 2048)
    short = torch.empty(ops.decode_layer_scratch_bytes(8, 8, 512) // 2, dtype=torch.uint8)
    assert ops.decode_layer_scratch_bytes(4, 8, 512) > short.numel()
    with pytest.raises(ValueError, match="scratch"):
        ops.moe_decode_layer(L, None, 0, 256, 8, None, x, x, None, None, short)


def test_supported_shapes():
    assert ops.native_expert_supported(_lib.IQ3_XXS, _lib.IQ3_S, 2048, 512)
    assert ops.native_expert_supported(_lib.Q4_K, _lib.Q4_K, 2048, 768)
    assert ops.native_expert_supported(_lib.Q8_0, _lib.Q8_0, 2048, 768)
    assert not ops.native_expert_supported(_lib.IQ3_XXS, _lib.IQ3_S, 2048, 640)   # IQ3_S down needs FF % 256 == 0
    assert not ops.native_expert_supported(16, _lib.IQ3_S, 2048, 512)            # IQ2_XXS: not on this path
    with pytest.raises(_lib.TsxError) as e:
        ops.native_expert_layout(_lib.IQ3_XXS, _lib.IQ3_S, 2048, 640)
    assert e.value.rc == _lib.TSX_ERR_UNSUPPORTED and "not supported" in str(e.value)


def test_argument_errors_need_no_gpu():
    lib = _lib.lib()
    assert lib.tsx_moe_quantize_q8_1(None, 1, 32, None, None) == _lib.TSX_ERR_ARG
    assert b"tsx_moe_quantize_q8_1" in lib.tsx_moe_last_error()
    assert lib.tsx_moe_router_topk(None, None, None, 100, 8, 1, None) == _lib.TSX_ERR_UNSUPPORTED
    assert lib.tsx_moe_mmvq(16, None, None, None, 256, 1, 1, None) == _lib.TSX_ERR_UNSUPPORTED
    assert lib.tsx_moe_mmq_q8_bytes(10, 33) == 0
    assert lib.tsx_moe_expert_layout(18, 21, 2048, 512, None) == _lib.TSX_ERR_ARG
    p = _lib.MmqProduct(type=18, n=1, w_rows=8, w_cols=2048, expert_bytes=8 * 784)
    assert lib.tsx_moe_mmq_run(C.byref(p), None) == _lib.TSX_ERR_ARG


def test_mmq_q8_bytes_planes():
    # q plane rows_pad x cols, then two f32 planes of rows_pad x cols/32, each 256-aligned; rows padded to 64 (+64)
    rp = (100 + 63) // 64 * 64 + 64
    r = lambda v: (v + 255) // 256 * 256
    assert ops.mmq_q8_bytes(100, 2048) == r(rp * 2048) + 2 * r(rp * 64 * 4)


@pytest.mark.skipif(shutil.which("g++") is None, reason="no g++")
def test_cpp_operator_api_header_compiles():
    """The C++ mirror of the reference operator API is a self-contained header."""
    src = '#include "strata_kernels.hpp"\nint main(){ strata::prefill::mmq::Product p; (void)p; return 0; }\n'
    res = subprocess.run(["g++", "-std=c++17", "-fsyntax-only", "-I", str(ROOT / "tinystrata_amd" / "csrc"), "-x", "c++", "-"],
                         input=src, text=True, capture_output=True)
    assert res.returncode == 0, res.stderr
