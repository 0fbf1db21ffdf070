"""The C++ operator API (tinystrata_amd/csrc/strata_kernels.hpp) on the CPU, through the test library
tinystrata_amd/libtsx_mirror_check.so: it loads and exports its entry points; the row-map storage helpers
(include/strata/prefill/mmq_ids_margin.hpp:13-47) agree with their closed form, refuse what cannot be represented
without touching their output, and cover every tile a row-map reader may touch (the property the reference's
tests/mmq-ids-margin.cpp checks: whole tiles of ids, up to the widest expert's row count, for tile widths 8..128).
Where the reference's headers are present (this container, not the GPU box), tests/mirror/api_shape.cpp is built
against them and against strata_kernels.hpp, both linked to libtsx_moe.so: the link resolves every API function
with the reference's exact signature, and the two builds print the same struct layouts and helper values."""
import ctypes as C
import subprocess
from pathlib import Path

import numpy as np
import pytest

import mirror_lib as ML

ROOT = Path(__file__).resolve().parent.parent
REF_INCLUDE = Path("/root/reference/include")
I64MAX, U64MAX, I32MAX = 2**63 - 1, 2**64 - 1, 2**31 - 1


def test_library_exports_every_entry_point():
    lib = ML.lib()
    for name in ML.SIGNATURES:
        assert hasattr(lib, name), name
    t = (C.c_int * 2)()
    lib.smc_tile_cols(t)
    assert (t[0], t[1]) == (128, 8)


def margin(r: int, j: int):
    out = C.c_int64(-7)
    ok = ML.lib().smc_margin_rows(r, j, C.byref(out))
    return bool(ok), out.value


@pytest.mark.parametrize("j", [1, 8, 64, 120, 128])
def test_margin_closed_form(j):
    for r in [0, 1, j - 1, j, j + 1, 3 * j, 4096, 32768, 10**12]:
        ok, m = margin(r, j)
        assert ok and m == -(-r // j) * j + j, (r, j)
        assert ML.lib().smc_table_rows(1000, r, j) == 1000 + m


def test_margin_refusals_leave_the_output():
    for r, j in [(-1, 128), (10, 0), (10, -8), (I64MAX, 128), (I64MAX - 100, 128)]:
        assert margin(r, j) == (False, -7), (r, j)
    assert ML.lib().smc_margin_rows_null(5, 128) == 0
    assert ML.lib().smc_table_rows_default(U64MAX, 1) == 0
    assert ML.lib().smc_table_rows_default(1, U64MAX) == 0
    assert ML.lib().smc_table_rows_default(1, I64MAX + 1) == 0
    io = (C.c_uint64 * 3)(11, 22, 88)
    assert ML.lib().smc_ids_layout(I32MAX, 1, io) == 0
    assert list(io) == [11, 22, 88]
    out = (C.c_uint64 * 10)()
    for e, c in [(U64MAX, 3), (256, U64MAX), (I32MAX + 1, 3)]:
        assert ML.lib().smc_packed_ids_layout(32, 32, e, c, out) == 0


def ids_layout(logical: int, max_rows: int):
    io = (C.c_uint64 * 3)(0, 0, 0)
    ok = ML.lib().smc_ids_layout(logical, max_rows, io)
    return bool(ok), list(io)


def test_ids_layout_and_packed_offsets():
    ok, (lr, sr, sb) = ids_layout(4096 * 8, 4096)
    assert ok and lr == 32768 and sr == 32768 + 4096 + 128 and sb == 4 * sr
    out = (C.c_uint64 * 10)()
    E, classes, L = 128, 3, 512 * 8
    assert ML.lib().smc_packed_ids_layout(L, 512, E, classes, out) == 1
    _, _, _, place, bounds, rel, wts, cls, words, nbytes = list(out)
    sr = L + 512 + 128
    assert (place, bounds, rel, wts, cls) == (L, L + sr, L + sr + E + 1, L + sr + 3 * E + 3, 2 * L + sr + 3 * E + 3)
    assert words == cls + classes * (E + 1) and nbytes == 4 * words


def fixture_reads_fit(counts, t, k) -> tuple[bool, bool]:
    """Every whole tile a reader may touch (each expert reads tiles up to the widest expert's rows, from its own
    first row) inside the stored map, for tile widths 8..128; also whether the map without margin would have held."""
    ok, (_, storage, _) = ids_layout(t * k, t)
    assert ok
    widest = max(counts)
    fits, fits_exact = True, True
    for j in range(8, 129, 8):
        base = 0
        for c in counts:
            reach = max(c, widest)
            if reach:
                last = base + (-(-reach // j)) * j - 1      # the last index of the last tile
                fits &= last < storage
                fits_exact &= last < t * k
            base += c
    return fits, fits_exact


def test_row_map_covers_every_tile_read():
    # an empty expert after full ones (the case an exactly-sized map gets wrong), then full, empty and ragged routing
    fits, exact = fixture_reads_fit([100, 100, 0, 0], 100, 2)
    assert fits and not exact
    for t in [1, 7, 31, 127, 128, 129, 255, 512, 1120, 4096, 32768]:
        for k in [1, 2, 8, 10]:
            full = [t] * k + [0, 0, 0]
            assert fixture_reads_fit(full, t, k)[0], (t, k)
            assert fixture_reads_fit([0] * (k + 3), t, k)[0], (t, k)
            ragged = [(t + 3 * e) % (t + 1) for e in range(k)] + [0, 0, 0]
            assert fixture_reads_fit(ragged, t, k)[0], (t, k)


@pytest.mark.skipif(not (REF_INCLUDE / "strata" / "prefill" / "moe_mmq.hpp").exists(),
                    reason="the reference's headers are not present here")
def test_reference_signatures_link_and_layouts_agree(tmp_path):
    src = ROOT / "tests" / "mirror" / "api_shape.cpp"
    pkg = ROOT / "tinystrata_amd"
    outs = {}
    for name, flags in [("reference", ["-DAPI_SHAPE_REFERENCE", f"-I{REF_INCLUDE}"]),
                        ("mirror", [f"-I{pkg / 'csrc'}"])]:
        exe = tmp_path / f"api_{name}"
        subprocess.run(["g++", "-std=c++17", "-O1", *flags, str(src), "-o", str(exe), f"-L{pkg}", "-ltsx_moe",
                        f"-Wl,-rpath,{pkg}"], check=True, capture_output=True, text=True)
        outs[name] = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.splitlines()
    assert outs["reference"] == outs["mirror"]
    assert outs["mirror"][0] == "functions 27" and len(outs["mirror"]) > 300
