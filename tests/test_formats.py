"""Formats: block sizes, expert blob layouts at the benchmark shapes, and the IQ3 codebooks.

The codebooks are checked against ggml-common.h where the reference is mounted (this container) and, everywhere,
against an FNV-1a hash of the 768 expanded words taken from it.
"""
import re
from pathlib import Path

import numpy as np
import pytest

import oracle as O
from tinystrata_amd import ops
from tinystrata_amd._lib import IQ3_S, IQ3_XXS, Q4_K, Q8_0

REF_COMMON = Path("/root/reference/third_party/ggml/ggml-common.h")
GRID_HASH_PINNED = 0xA88D7B1B95407E6F


def test_block_bytes():
    assert O.BLOCK[O.Q8_0] == (32, 34) and O.BLOCK[O.Q8_1] == (32, 36)
    assert O.BLOCK[O.Q4_K] == (256, 144) and O.BLOCK[O.Q8_K] == (256, 292)
    assert O.BLOCK[O.IQ3_XXS] == (256, 98) and O.BLOCK[O.IQ3_S] == (256, 110)
    for t in (Q8_0, Q4_K, IQ3_XXS, IQ3_S):
        assert ops.iq_row_bytes(t, 2048) == O.row_bytes(t, 2048)
    assert ops.iq_row_bytes(IQ3_S, 100) == 0


@pytest.mark.parametrize("gu,d,n,ff,expect", [
    (IQ3_XXS, IQ3_S, 2048, 512, 1_253_376),   # configs 2, 3, 5
    (Q8_0, Q8_0, 2048, 768, 5_013_504),       # config 1
    (Q4_K, Q4_K, 2048, 768, 2_654_208),       # config 4
])
def test_expert_layout_bytes(gu, d, n, ff, expect):
    L = ops.native_expert_layout(gu, d, n, ff)
    assert L.bytes == expect
    assert L.up_off == ff * L.gu_row and L.down_off == 2 * L.up_off
    Lo = O.layout(gu, d, n, ff)
    assert (Lo.bytes, Lo.up_off, Lo.down_off) == (L.bytes, L.up_off, L.down_off)


def _ref_table(name):
    src = REF_COMMON.read_text()
    m = re.search(r"GGML_TABLE_BEGIN\(uint32_t, %s, (\d+)\)(.*?)GGML_TABLE_END" % name, src, re.S)
    return [int(v, 16) for v in re.findall(r"0x[0-9a-f]+", m.group(2))]


def _fnv(words):
    h = 1469598103934665603
    for w in words:
        for b in range(4):
            h = ((h ^ ((w >> (8 * b)) & 255)) * 1099511628211) & 0xFFFFFFFFFFFFFFFF
    return h


def test_grid_hash_pinned():
    assert O.grid_hash() == GRID_HASH_PINNED


@pytest.mark.skipif(not REF_COMMON.exists(), reason="reference not mounted")
def test_grids_match_ggml_common():
    xxs, s = _ref_table("iq3xxs_grid"), _ref_table("iq3s_grid")
    assert len(xxs) == 256 and len(s) == 512
    assert _fnv(xxs + s) == O.grid_hash() == GRID_HASH_PINNED


@pytest.mark.skipif(not REF_COMMON.exists(), reason="reference not mounted")
def test_ksigns_parity_rule_matches_table():
    # ksigns_iq2xs[i] = i | parity(i) << 7 (the rule the kernels use instead of the table)
    src = REF_COMMON.read_text()
    m = re.search(r"GGML_TABLE_BEGIN\(uint8_t, ksigns_iq2xs, 128\)(.*?)GGML_TABLE_END", src, re.S)
    table = [int(v) for v in re.findall(r"\d+", m.group(1))]
    assert table == [i | ((bin(i).count("1") & 1) << 7) for i in range(128)]


def test_weight_quantizers_valid_blocks():
    rng = np.random.default_rng(1)
    x = rng.normal(0, 0.02, (8, 512)).astype(np.float32)
    limits = {Q8_0: 0.01, Q4_K: 0.1, IQ3_S: 0.22, IQ3_XXS: 0.28}
    for t, lim in limits.items():
        w = ops.quantize_weights(t, x)
        deq = np.stack([O.dequantize(t, w[r], 512) for r in range(8)])
        rel = np.linalg.norm(deq - x) / np.linalg.norm(x)
        assert rel < lim, (t, rel)
        if t == IQ3_XXS:  # every 8-value sign group has an even count of negatives, as the format requires
            negs = (deq.reshape(-1, 8) < 0).sum(1)
            assert (negs % 2 == 0).all()
