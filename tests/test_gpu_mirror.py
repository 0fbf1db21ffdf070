"""The C++ operator API driven from C++ on the GPU: tinystrata_amd/libtsx_mirror_check.so calls
strata::kernels::native_expert_layout / native_expert_grouped / quantize_q8_1_rows / native_router_topk /
native_mmvq and strata::prefill::mmq::quantize / iota / Context::run (tinystrata_amd/csrc/strata_kernels.hpp, the
reference's include/strata/kernels/iq_kernels.hpp:44-78, native_router.hpp:5-6, native_mmvq.hpp:125-131 and
include/strata/prefill/moe_mmq.hpp:37-85), in the reference caller's order; the results are checked against the
oracle, and the thrown exceptions (caught in the library and returned with their messages) against the reference's
error convention (src/kernels/cuda/native_router.cu:103-110)."""
import ctypes as C

import numpy as np
import pytest
import torch

import mirror_lib as ML
import oracle as O
from tinystrata_amd import ops
from tinystrata_amd._lib import IQ3_S, IQ3_XXS, Q4_K, Q8_0

from gpu_util import dev, experts, host, rel_l2

pytestmark = pytest.mark.gpu


def stream() -> int:
    return torch.cuda.current_stream().cuda_stream


@pytest.mark.parametrize("gu,d,N,FF,n_tok", [(IQ3_XXS, IQ3_S, 2048, 512, 1), (IQ3_XXS, IQ3_S, 2048, 512, 4),
                                             (Q4_K, Q4_K, 2048, 768, 3), (Q8_0, Q8_0, 256, 256, 2)])
def test_expert_grouped_through_the_mirror(gu, d, N, FF, n_tok):
    lib = ML.lib()
    E, k = 32, 8
    L, blobs, _ = experts(gu, d, N, FF, E)
    Lo = O.layout(gu, d, N, FF)
    lay = (C.c_uint64 * 6)()
    assert lib.smc_expert_layout(gu, d, N, FF, lay) == 1
    assert list(lay) == [Lo.gu_row, Lo.d_row, Lo.up_off, Lo.down_off, Lo.bytes, 0]
    rng = np.random.default_rng(N + FF + n_tok)
    x = rng.normal(0, 1, (n_tok, N)).astype(np.float32)
    logits = rng.normal(0, 1, (n_tok, E)).astype(np.float32)
    ids, _ = O.router_topk(logits, k)
    blobs_d = dev(blobs.ravel())
    n_ent = n_tok * k
    gp, gs, ng, ed, et = ops.group_entries(dev(ids), k, E, blobs_d.data_ptr(), blobs.shape[1])
    xd = dev(x)
    xq = torch.empty(n_tok * N // 32 * 36, dtype=torch.uint8, device="cuda")
    assert lib.smc_quantize_q8_1_rows(xd.data_ptr(), n_tok, N, xq.data_ptr(), stream()) == 0
    assert (host(xq).reshape(n_tok, -1) == O.quantize_q8_1(x)).all()
    nb = lib.smc_expert_scratch_bytes(n_ent, FF)
    assert nb == ops.native_expert_scratch_bytes(n_ent, FF)
    scratch = torch.zeros(nb, dtype=torch.uint8, device="cuda")
    out = torch.full((n_ent, N), float("nan"), device="cuda")
    rc = lib.smc_expert_grouped(gu, d, N, FF, gp.data_ptr(), gs.data_ptr(), ng.data_ptr(), ed.data_ptr(),
                                et.data_ptr(), min(n_ent, E), n_ent, xq.data_ptr(), scratch.data_ptr(),
                                out.data_ptr(), stream(), 0)
    assert rc == 0
    got = host(out)
    # the C ABI call on the same tables gives the same bits
    ref_out = torch.full((n_ent, N), float("nan"), device="cuda")
    ops.native_expert_grouped(L, gp, gs, ng, ed, et, min(n_ent, E), n_ent, xq.view(torch.uint8),
                              torch.zeros_like(scratch), ref_out)
    assert (host(ref_out) == got).all()
    # and the oracle fed the same activation codes
    _, egs, _, eed, eet = O.group(ids, k, E)
    hb = [blobs[e] for e in np.unique(ids)]
    _, hq = O.expert_gu(Lo, hb, egs, eet, host(xq).reshape(n_tok, -1))
    assert rel_l2(got, O.expert_down(Lo, hb, egs, eed, hq, n_ent)) < 1e-3


@pytest.mark.parametrize("t", [IQ3_XXS, IQ3_S, Q4_K, Q8_0])
def test_mmq_context_run_through_the_mirror(t):
    """quantize (rows gathered through a map), iota, Context::run over experts with 0, 70, 1, 130 and 17 rows,
    writing through the identity map iota filled, sized by ids_layout (the margin included)."""
    lib = ML.lib()
    rng = np.random.default_rng(t)
    w_rows, w_cols = 128, 512
    assert lib.smc_mmq_supported(t, w_rows) == 1
    counts = [0, 70, 1, 130, 17]
    n, total = len(counts), sum(counts)
    bounds = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    W = [ops.quantize_weights(t, rng.normal(0, 0.02, (w_rows, w_cols)).astype(np.float32)) for _ in range(n)]
    eb = (w_rows * W[0].shape[1] + 255) // 256 * 256
    blob = np.zeros(n * eb, np.uint8)
    for i, m in enumerate(W):
        blob[i * eb: i * eb + m.size] = m.ravel()
    tokens = rng.normal(0, 1, (64, w_cols)).astype(np.float32)
    tok_of_row = rng.integers(0, 64, total).astype(np.int32)
    io = (C.c_uint64 * 3)()
    assert lib.smc_ids_layout(total, max(counts), io) == 1
    storage = io[1]
    ident = torch.full((storage,), -1, dtype=torch.int32, device="cuda")
    assert lib.smc_mmq_iota(ident.data_ptr(), storage, stream()) == 0
    assert (host(ident) == np.arange(storage)).all()
    xq = torch.zeros(lib.smc_mmq_q8_bytes(total, w_cols), dtype=torch.uint8, device="cuda")
    xt, rows_d = dev(tokens), dev(tok_of_row)
    assert lib.smc_mmq_quantize(xt.data_ptr(), rows_d.data_ptr(), xq.data_ptr(), t, w_cols, w_cols, total,
                                stream()) == 0
    dst = torch.full((total, w_rows), float("nan"), device="cuda")
    wb, bd = dev(blob), dev(bounds)
    assert lib.smc_mmq_run(wb.data_ptr(), t, w_rows, w_cols, eb, n, xq.data_ptr(), bd.data_ptr(), ident.data_ptr(),
                           total, max(counts), dst.data_ptr(), w_rows, stream()) == 0
    got = host(dst)
    xb = O.quantize_q8_1(tokens[tok_of_row])
    exp = np.zeros((total, w_rows), np.float64)
    for i in range(n):
        r0, r1 = bounds[i], bounds[i + 1]
        if r1 > r0:
            exp[r0:r1] = O.mmvq_q8_1(t, W[i], w_cols, w_rows, xb[r0:r1], r1 - r0)
    assert np.isfinite(got).all()
    np.testing.assert_allclose(got, exp, rtol=1e-5, atol=1e-5 * np.abs(exp).max())


@pytest.mark.parametrize("E,k,T", [(256, 8, 1), (256, 8, 4), (128, 8, 33)])
def test_router_topk_through_the_mirror(E, k, T):
    lib = ML.lib()
    assert lib.smc_router_topk_supported(E, k) == 1
    rng = np.random.default_rng(E + T)
    logits = rng.normal(0, 1, (T, E)).astype(np.float32)
    lg = dev(logits)
    ids = torch.empty((T, k), dtype=torch.int32, device="cuda")
    w = torch.empty((T, k), dtype=torch.float32, device="cuda")
    msg = ML.msg_buf()
    s = torch.cuda.Stream()   # the reference's router takes a stream of the caller's: a null one throws
    s.wait_stream(torch.cuda.current_stream())
    rc = lib.smc_router_topk(lg.data_ptr(), ids.data_ptr(), w.data_ptr(), E, k, T, s.cuda_stream, msg, 512)
    assert rc == 0, msg.value
    s.synchronize()
    eids, ew = O.router_topk(logits, k)
    assert (host(ids) == eids).all()
    np.testing.assert_allclose(host(w), ew, rtol=2e-6, atol=1e-7)


def test_router_and_mmvq_exceptions():
    """Unsupported expert counts and a missing stream throw std::invalid_argument (nothing launched: the outputs
    keep their contents); an unsupported mmvq type throws std::invalid_argument from both the launch and the byte
    helper."""
    lib = ML.lib()
    logits = dev(np.zeros((2, 100), np.float32))
    ids = torch.full((2, 8), -5, dtype=torch.int32, device="cuda")
    w = torch.zeros((2, 8), dtype=torch.float32, device="cuda")
    msg = ML.msg_buf()
    assert lib.smc_router_topk_supported(100, 8) == 0
    assert lib.smc_router_topk(logits.data_ptr(), ids.data_ptr(), w.data_ptr(), 100, 8, 2, stream(), msg, 512) == 1
    assert b"native_router_topk" in msg.value
    lg = dev(np.zeros((2, 256), np.float32))
    assert lib.smc_router_topk(lg.data_ptr(), ids.data_ptr(), w.data_ptr(), 256, 8, 2, None, msg, 512) == 1
    assert lib.smc_router_topk(lg.data_ptr(), ids.data_ptr(), w.data_ptr(), 256, 17, 2, stream(), msg, 512) == 1
    assert (host(ids) == -5).all()
    y = torch.zeros(8, device="cuda")
    assert lib.smc_mmvq(99, y.data_ptr(), y.data_ptr(), y.data_ptr(), 256, 8, 1, stream(), msg, 512) == 1
    assert b"unsupported" in msg.value
    nb = C.c_uint64(0)
    assert lib.smc_mmvq_weight_bytes(99, 256, 8, C.byref(nb), msg, 512) == 1
    assert lib.smc_mmvq_weight_bytes(Q8_0, 256, 8, C.byref(nb), msg, 512) == 0 and nb.value == 8 * 8 * 34
