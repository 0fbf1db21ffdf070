"""tsx_moe_decode_layer_noalloc (the decode layer on a fixed per-GPU scratch array) against tsx_moe_decode_layer with
a caller-provided scratch, through the C ABI: two calls in a row, the second with fewer tokens, each bit-identical to
the allocating entry point (the same kernels on the same inputs).  Marked gpu."""
import ctypes as C

import numpy as np
import pytest
import torch

from tinystrata_amd import moe, ops
from tinystrata_amd._lib import IQ3_S, IQ3_XXS, TSX_ERR_UNSUPPORTED, check, lib

from gpu_util import dev, host, pool

pytestmark = pytest.mark.gpu


def _p(t):
    return None if t is None else t.data_ptr()


def _both(L, W, k, x, logits, sgate):
    """The layer through both entry points on the same inputs: (y, ids, wts) of each."""
    T, N = x.shape
    s = torch.cuda.current_stream().cuda_stream
    out = []
    for noalloc in (False, True):
        y = torch.zeros((T, N), device="cuda")
        ids = torch.full((T, k), -1, dtype=torch.int32, device="cuda")
        wts = torch.full((T, k), float("nan"), device="cuda")
        args = [C.byref(L), W.blobs.data_ptr(), W.stride, W.n_expert, k, T, logits.data_ptr(), x.data_ptr(),
                _p(W.shared), _p(sgate), 1, y.data_ptr(), ids.data_ptr(), wts.data_ptr()]
        if noalloc:
            check(lib().tsx_moe_decode_layer_noalloc(*args, s), "decode_layer_noalloc")
        else:
            scratch = torch.empty(ops.decode_layer_scratch_bytes(T, k, int(L.n_ff)), dtype=torch.uint8, device="cuda")
            check(lib().tsx_moe_decode_layer(*args, scratch.data_ptr(), s), "decode_layer")
        out.append((host(y), host(ids), host(wts)))
    return out


def test_noalloc_matches_allocating_entry_point():
    N, FF, E, k = 2048, 512, 256, 8
    L = ops.native_expert_layout(IQ3_XXS, IQ3_S, N, FF)
    p = pool(IQ3_XXS, IQ3_S, N, FF, 8, 0)
    order = (np.arange(E) * 5 + 3) % 8
    W = moe.weights_from_pool(L, dev(p), E, order, 7)
    rng = np.random.default_rng(21)
    assert lib().tsx_moe_decode_layer_noalloc_max_bytes() >= ops.decode_layer_scratch_bytes(8, 8, 1024)
    W0 = moe.MoEWeights(L=W.L, n_expert=W.n_expert, stride=W.stride, blobs=W.blobs, shared=None)
    # each call smaller than the one before it, so the array holds an earlier call's bytes: T = 1 is the one-token
    # launch A (fp32 h quantized by launch B, tables written by its last block) over what the 8-token call left, with
    # and without the shared expert
    for T, Wt in ((8, W), (1, W), (3, W), (1, W0)):
        x = dev(rng.normal(0, 1, (T, N)).astype(np.float32))
        logits = dev(rng.normal(0, 1, (T, E)).astype(np.float32))
        sg = dev(rng.normal(0, 1, T).astype(np.float32)) if Wt.shared is not None else None
        (ya, ia, wa), (yb, ib, wb) = _both(L, Wt, k, x, logits, sg)
        tag = (T, Wt.shared is not None)
        assert np.isfinite(ya).all() and (ia >= 0).all()
        assert (ia == ib).all() and (wa.view(np.uint32) == wb.view(np.uint32)).all(), tag
        assert (ya.view(np.uint32) == yb.view(np.uint32)).all(), tag
        print(f"noalloc T={T} shared={tag[1]}: bit-identical to the allocating entry point", flush=True)


def test_noalloc_refuses_what_does_not_fit():
    # 8 tokens top-8 at n_ff 2048 need ~166 KB of scratch, more than the array holds: refused before any launch
    L = ops.native_expert_layout(IQ3_XXS, IQ3_S, 2048, 2048)
    assert ops.decode_layer_scratch_bytes(8, 8, 2048) > lib().tsx_moe_decode_layer_noalloc_max_bytes()
    z = torch.zeros(16, device="cuda")
    rc = lib().tsx_moe_decode_layer_noalloc(C.byref(L), z.data_ptr(), 256, 256, 8, 8, z.data_ptr(), z.data_ptr(),
                                            None, None, 1, z.data_ptr(), z.data_ptr(), z.data_ptr(),
                                            torch.cuda.current_stream().cuda_stream)
    assert rc == TSX_ERR_UNSUPPORTED and b"more than" in lib().tsx_moe_last_error()
