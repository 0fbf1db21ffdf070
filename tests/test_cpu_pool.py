"""The hybrid split's CPU side (include/tsx_pool.h), on the CPU: the expert rows against the oracle, the pool against
the rows run serially, and the CPU half of a hybrid layer.

Bars: the rows are bit-identical to the oracle (oracle/oracle.c orc_expert_gu / orc_expert_down: the same integer
sub-block sums and the same double accumulation order), the Q8_1 bytes identical; every pool configuration writes
the same bits as the serial rows (the reference's own pool test proves pool == serial,
tests/native-expert-pool.cpp); the hybrid CPU half numbers the misses in entry order (compact rows, reference
moe_hybrid_cpu, src/qwen35/q36_engine.cu:3140-3160)."""
import time

import numpy as np
import pytest

import oracle as O
from tinystrata_amd import _lib, ops
from tinystrata_amd._lib import IQ3_S, IQ3_XXS, Q4_K, Q8_0
from tinystrata_amd.moe import synthetic_pool
from tinystrata_amd.pool import (ExpertPool, cpu_down_rows, cpu_fmt, cpu_gu_rows, cpu_quant_act, cpu_quant_h,
                                 hybrid_cpu)

PAIRS = [(IQ3_XXS, IQ3_S), (Q4_K, Q4_K), (Q8_0, Q8_0), (IQ3_S, IQ3_XXS)]
_POOLS = {}


def experts(gu, d, N, FF, count, seed=0):
    key = (gu, d, N, FF, count, seed)
    if key not in _POOLS:
        _POOLS[key] = synthetic_pool(ops.native_expert_layout(gu, d, N, FF), count, seed)
    return _POOLS[key]


def serial(f, blob, xs):
    """One expert on the rows alone: gate/up rows, Q8_1 of h, down rows."""
    acts = [cpu_quant_act(f, x) for x in xs]
    h = cpu_gu_rows(f, blob, acts)
    return cpu_down_rows(f, blob, [cpu_quant_h(f, r) for r in h])


@pytest.mark.parametrize("gu,d", PAIRS)
@pytest.mark.parametrize("nt", [1, 3, 8])
def test_rows_match_the_oracle(gu, d, nt):
    N, FF = 512, 256
    f = cpu_fmt(gu, d, N, FF)
    blob = experts(gu, d, N, FF, 1)[0]
    x = np.random.default_rng(nt).normal(0, 1, (nt, N)).astype(np.float32)
    xq = O.quantize_q8_1(x)
    acts = [cpu_quant_act(f, x[t]) for t in range(nt)]
    assert all(np.array_equal(acts[t], xq[t]) for t in range(nt))
    OL = O.layout(gu, d, N, FF)
    h_o, hq_o = O.expert_gu(OL, [blob], np.array([0, nt]), np.arange(nt), xq)
    h = cpu_gu_rows(f, blob, acts)
    assert np.array_equal(h.view(np.uint32), h_o.view(np.uint32))
    hq = [cpu_quant_h(f, h[t]) for t in range(nt)]
    assert all(np.array_equal(hq[t], hq_o[t]) for t in range(nt))
    out_o = O.expert_down(OL, [blob], np.array([0, nt]), np.arange(nt), hq_o, nt)
    out = cpu_down_rows(f, blob, hq)
    assert np.array_equal(out.view(np.uint32), out_o.view(np.uint32))
    # a row range writes only its rows
    part = cpu_down_rows(f, blob, hq, 100, 140)
    assert np.array_equal(part[:, 100:140], out[:, 100:140]) and not part[:, :100].any() and not part[:, 140:].any()


def test_rows_reject_bad_arguments():
    with pytest.raises(_lib.TsxError) as e:
        cpu_fmt(IQ3_XXS, IQ3_S, 2048, 100)
    assert e.value.rc == _lib.TSX_ERR_UNSUPPORTED
    with pytest.raises(_lib.TsxError) as e:
        cpu_fmt(Q4_K, 2, 2048, 512)  # Q4_0 is no expert type
    assert e.value.rc == _lib.TSX_ERR_UNSUPPORTED
    f = cpu_fmt(Q8_0, Q8_0, 256, 256)
    blob = experts(Q8_0, Q8_0, 256, 256, 1)[0]
    act = cpu_quant_act(f, np.ones(256, np.float32))
    with pytest.raises(_lib.TsxError):
        cpu_gu_rows(f, blob, [act] * 9)  # more than 8 tokens
    with pytest.raises(_lib.TsxError):
        cpu_gu_rows(f, blob, [act], 0, 257)  # past n_ff


def make_jobs(f, blobs, rng, n_jobs, N):
    jobs, want = [], []
    for j in range(n_jobs):
        nt = int(rng.integers(1, 9))
        xs = rng.normal(0, 1, (nt, N)).astype(np.float32)
        b = blobs[j % len(blobs)]
        jobs.append((b, [cpu_quant_act(f, x) for x in xs], [np.full(N, np.nan, np.float32) for _ in range(nt)]))
        want.append(serial(f, b, xs))
    return jobs, want


@pytest.mark.parametrize("workers,host_works,tasks", [(1, True, 0), (3, False, 0), (4, True, 7), (6, True, 1000)])
def test_pool_equals_serial(workers, host_works, tasks):
    N, FF = 256, 256
    f = cpu_fmt(IQ3_XXS, IQ3_S, N, FF)
    blobs = experts(IQ3_XXS, IQ3_S, N, FF, 6, seed=1)
    rng = np.random.default_rng(workers * 10 + tasks)
    with ExpertPool(workers, pin=False, host_works=host_works, tasks=tasks) as p:
        assert p.workers == workers and p.host_works == host_works
        for n_jobs in (1, 2, 13, 100):  # one expert (phases), several (dependent tasks), more than one batch of 96
            jobs, want = make_jobs(f, blobs, rng, n_jobs, N)
            p.run(f, jobs)
            for (_, _, outs), w in zip(jobs, want):
                assert np.array_equal(np.stack(outs).view(np.uint32), w.view(np.uint32))
        st = p.stats()
        assert st["bytes"] == (1 + 2 + 13 + 100) * f.bytes and st["drain"] > 0 and st["gate_up"] > 0
        assert st["down"] > 0 and st["quant_h"] > 0
        # run() returns once every chunk is finished; workers still scanning the batch leave it right after
        d = p.diag()
        for _ in range(2000):
            if f"idle {workers}/{workers}" in d and "attached 0|0" in d:
                break
            time.sleep(0.001)
            d = p.diag()
        assert f"idle {workers}/{workers}" in d and "attached 0|0" in d and "FAILED" not in d, d
        assert "0 unclaimed" in d and d.count("idle") + d.count("sleeping") == workers + 1, d


def test_pool_sleeping_workers():
    """Workers that sleep between every batch (no spin): each run still completes with every job done once."""
    N, FF = 256, 256
    f = cpu_fmt(Q4_K, Q4_K, N, FF)
    blobs = experts(Q4_K, Q4_K, N, FF, 3, seed=2)
    rng = np.random.default_rng(5)
    with ExpertPool(5, pin=False, host_works=True) as p:
        p.set_spin_us(0)
        p.set_stall_ms(20000)
        for it in range(40):
            jobs, want = make_jobs(f, blobs, rng, 1 + it % 4, N)
            p.run(f, jobs)
            for (_, _, outs), w in zip(jobs, want):
                assert np.array_equal(np.stack(outs).view(np.uint32), w.view(np.uint32)), it


def test_pool_default_size_and_pinning():
    with ExpertPool() as p:
        assert p.workers >= 1
        f = cpu_fmt(Q8_0, Q8_0, 256, 256)
        blobs = experts(Q8_0, Q8_0, 256, 256, 2, seed=3)
        jobs, want = make_jobs(f, blobs, np.random.default_rng(0), 4, 256)
        p.run(f, jobs)
        for (_, _, outs), w in zip(jobs, want):
            assert np.array_equal(np.stack(outs), w)


@pytest.mark.parametrize("T", [1, 4, 12])  # 12 tokens: experts with more than 8 misses take two jobs
def test_hybrid_cpu_half(T):
    N, FF, E, k = 512, 256, 24, 8
    f = cpu_fmt(IQ3_XXS, IQ3_S, N, FF)
    pool = experts(IQ3_XXS, IQ3_S, N, FF, 6, seed=4)
    blobs = np.stack([pool[e % 6] for e in range(E)])
    rng = np.random.default_rng(T)
    ids = np.stack([rng.permutation(E)[:k] for _ in range(T)]).astype(np.int32)
    x = rng.normal(0, 1, (T, N)).astype(np.float32)
    slot_of = np.where(np.arange(E) % 3 == 0, np.arange(E) // 3, -1).astype(np.int32)  # every third expert resident
    rows = np.full((T * k, N), np.nan, np.float32)
    miss = np.zeros(T * k, np.int32)
    with ExpertPool(3, pin=False) as p:
        nm = hybrid_cpu(p, f, blobs, blobs.shape[1], slot_of, k, ids, x, rows, miss)
    flat = ids.ravel()
    want_miss = np.full(T * k, -1, np.int32)
    want_miss[slot_of[flat] < 0] = np.arange(int((slot_of[flat] < 0).sum()))
    assert nm == int((slot_of[flat] < 0).sum()) and np.array_equal(miss, want_miss)
    for e in range(T * k):
        if miss[e] >= 0:
            want = serial(f, blobs[flat[e]], x[e // k: e // k + 1])[0]
            assert np.array_equal(rows[miss[e]], want), e
    assert np.isnan(rows[nm:]).all()  # nothing past the misses
    with ExpertPool(1, pin=False) as p, pytest.raises(_lib.TsxError):
        hybrid_cpu(p, f, blobs, blobs.shape[1], slot_of, k, np.full((T, k), E, np.int32), x, rows, miss)


def test_pool_stall_is_an_error_not_a_hang():
    """A run that makes no progress for the stall limit returns TSX_ERR_STALLED (the reference aborts the engine
    there, src/kernels/cpu/pool.cpp:655-677), and the pool takes no more work.  The stall is forced from the host:
    a 1 ms limit, one worker and the host not draining, against jobs that take far longer."""
    N, FF = 2048, 512
    f = cpu_fmt(IQ3_XXS, IQ3_S, N, FF)
    blobs = experts(IQ3_XXS, IQ3_S, N, FF, 2, seed=6)
    act = cpu_quant_act(f, np.ones(N, np.float32))
    p = ExpertPool(1, pin=False, host_works=False, tasks=1)
    p.set_stall_ms(1)
    jobs = [(blobs[j % 2], [act] * 8, [np.zeros(N, np.float32) for _ in range(8)]) for j in range(1)]
    with pytest.raises(_lib.TsxError) as e:
        for _ in range(50):  # a single slow task: the host sees no completion for 1 ms
            p.run(f, jobs)
    assert e.value.rc == _lib.TSX_ERR_STALLED
    with pytest.raises(_lib.TsxError) as e:
        p.run(f, jobs)
    assert e.value.rc == _lib.TSX_ERR_STALLED
    p.close()  # joins the worker once its task ends


def test_hybrid_cpu_stall_then_destroy():
    """A stall inside tsx_moe_hybrid_cpu: the call returns TSX_ERR_STALLED, the next call is refused before it touches
    the pool's token rows (which the stalled batch's worker may still read), the caller's blobs and output rows stay
    referenced by the pool (the stalled worker may still read and write them), and destroying the pool joins that
    worker and only then lets them go."""
    N, FF, E, k, T = 2048, 512, 4, 4, 8
    f = cpu_fmt(Q8_0, Q8_0, N, FF)
    blobs = experts(Q8_0, Q8_0, N, FF, E, seed=7)
    ids = (np.arange(T * k) % E).reshape(T, k).astype(np.int32)
    x = np.random.default_rng(1).normal(0, 1, (T, N)).astype(np.float32)
    slot_of = np.full(E, -1, np.int32)
    rows = np.zeros((T * k, N), np.float32)
    miss = np.zeros(T * k, np.int32)
    p = ExpertPool(1, pin=False, host_works=False, tasks=1)
    p.set_stall_ms(1)
    with pytest.raises(_lib.TsxError) as e:
        for _ in range(50):
            hybrid_cpu(p, f, blobs, blobs.shape[1], slot_of, k, ids, x, rows, miss)
    assert e.value.rc == _lib.TSX_ERR_STALLED
    with pytest.raises(_lib.TsxError) as e:
        hybrid_cpu(p, f, blobs, blobs.shape[1], slot_of, k, ids, x, rows, miss)
    assert e.value.rc == _lib.TSX_ERR_STALLED and "takes no more work" in str(e.value)
    assert "FAILED" in p.diag()
    # the stalled call's arrays are held until close(): its worker may still be reading blobs and writing rows
    assert any(held[0] is blobs and held[2] is rows for held in p._stalled)
    p.close()
    assert p._stalled == []
