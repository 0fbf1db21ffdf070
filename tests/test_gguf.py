"""The GGUF reader (include/tsx_gguf.h) on synthetic model files: directory, metadata, payload offsets and alignment,
split models, the refusals of the reference reader (include/strata/artifact/gguf_reader.hpp:447-501,579-607), and
the expert repack into [gate | up | down] blobs (src/qwen35/q36_engine.cu:1144-1168,1196-1201)."""
import math

import numpy as np
import pytest

from tinystrata_amd import _lib, ops
from tinystrata_amd.gguf import GgufModel, block_geometry, split_paths

from gguf_writer import ARRAY, BOOL, F32, F64, I8, I16, I32, I64, STRING, U8, U16, U32, U64, GgufFile

IQ3_XXS, IQ3_S, Q4_K, Q8_0, F32_T = 18, 21, 12, 8, 0


def rnd(n, seed):
    return np.random.default_rng(seed).integers(0, 256, n, dtype=np.uint8)


def test_block_geometry_from_the_block_fields():
    # bytes per block as the sum of each format's fields (ggml-common.h), values per block
    fields = {
        0: (1, 4), 1: (1, 2), 30: (1, 2),
        2: (32, 2 + 16), 3: (32, 2 + 2 + 16), 6: (32, 2 + 4 + 16), 7: (32, 2 + 2 + 4 + 16), 8: (32, 2 + 32),
        9: (32, 2 + 2 + 32), 10: (256, 16 + 64 + 2 + 2), 11: (256, 32 + 64 + 12 + 2), 12: (256, 2 + 2 + 12 + 128),
        13: (256, 2 + 2 + 12 + 32 + 128), 14: (256, 128 + 64 + 16 + 2), 16: (256, 2 + 64), 17: (256, 2 + 64 + 8),
        18: (256, 2 + 96), 20: (32, 2 + 16), 21: (256, 2 + 64 + 8 + 32 + 4), 22: (256, 2 + 64 + 8 + 8),
        23: (256, 2 + 2 + 4 + 128), 29: (256, 32 + 16 + 8), 39: (32, 1 + 16), 24: (1, 1),
    }
    for t, ge in fields.items():
        assert block_geometry(t) == ge, t
    with pytest.raises(_lib.TsxError) as e:
        block_geometry(99)
    assert e.value.rc == _lib.TSX_ERR_UNSUPPORTED


def small_model(alignment=None):
    f = GgufFile()
    f.kv("general.architecture", STRING, "qwen35moe")
    if alignment:
        f.kv("general.alignment", U32, alignment)
    f.kv("u8", U8, 200).kv("i8", I8, -5).kv("u16", U16, 60000).kv("i16", I16, -300).kv("i32", I32, -70000)
    f.kv("f32", F32, 1.5).kv("flag", BOOL, True).kv("u64", U64, 2**40 + 3).kv("i64", I64, -(2**40)).kv("f64", F64, 0.1)
    f.kv("ints", ARRAY, list(range(100)), I32).kv("names", ARRAY, ["a", "bc", ""], STRING)
    f.kv("nested", ARRAY, [(U8, [1, 2]), (U8, [3])], ARRAY)
    f.add("w.f32", F32_T, (7, 3), np.arange(21, dtype=np.float32))
    f.add("w.q8", Q8_0, (64, 2), rnd(4 * 34, 1))
    f.add("w.iq3", IQ3_XXS, (256, 3), rnd(3 * 98, 2))
    f.add("w.odd", 99, (5,), rnd(7, 3))  # a type of unknown geometry: listed, no payload
    return f


@pytest.mark.parametrize("alignment", [None, 64])
def test_directory_metadata_and_payloads(tmp_path, alignment):
    f = small_model(alignment)
    path = f.write(tmp_path / "m.gguf")
    with GgufModel(path) as g:
        info = g.shard_info()
        al = alignment or 32
        assert info["version"] == 3 and info["alignment"] == al and info["data_start"] % al == 0
        ts = g.tensors()
        assert [t.name for t in ts] == ["w.f32", "w.q8", "w.iq3", "w.odd"]
        assert [t.shape for t in ts] == [(7, 3), (64, 2), (256, 3), (5,)]
        assert [t.bytes for t in ts] == [84, 4 * 34, 3 * 98, 0]
        assert all(t.offset % al == 0 for t in ts)
        assert ts[3].data == 0
        for t in f.tensors[:3]:
            assert g.tensor_bytes(t.name).tobytes() == t.data
        assert g.find("nope") is None
        assert g.meta("general.architecture") == "qwen35moe"
        assert (g.meta("u8"), g.meta("i8"), g.meta("u16"), g.meta("i16"), g.meta("i32")) == (200, -5, 60000, -300, -70000)
        assert g.meta("f32") == 1.5 and g.meta("flag") is True and g.meta("u64") == 2**40 + 3
        assert g.meta("i64") == -(2**40) and g.meta("f64") == 0.1
        assert g.meta("ints") == list(range(64))  # the first 64 items are kept
        assert g.meta("names") == ["a", "bc", ""]
        assert g.meta("missing", "d") == "d"
        assert g.keys()[0] == "general.architecture" and "nested" in g.keys()


def faulty(kind):
    f = small_model()
    if kind == "magic":
        f.magic = b"GGUX"
    elif kind == "version":
        f.version = 2
    elif kind == "dup":
        f.add("w.q8", Q8_0, (32,), rnd(34, 4))
    elif kind == "ndims":
        f.add("w.5d", F32_T, (1, 1, 1, 1, 1), rnd(4, 5))
    elif kind == "metatype":
        f.kv("bad", 13, 0)
    elif kind == "deep":
        f.kv("deep", ARRAY, [(ARRAY, [(U8, [1])])], ARRAY)
    return f


@pytest.mark.parametrize("kind,text", [("magic", "bad magic"), ("version", "v2"), ("dup", "duplicate tensor"),
                                       ("ndims", "n_dims"), ("metatype", "metadata value type"),
                                       ("deep", "nested too deep")])
def test_refusals(tmp_path, kind, text):
    f = faulty(kind)
    if kind == "metatype":
        # the writer cannot encode an unknown type's value; write the type id with no value after it
        f.meta[-1] = ("bad", U8, 0, None)
        raw = bytearray(f.to_bytes())
        key = b"\x03\x00\x00\x00\x00\x00\x00\x00bad"
        at = raw.index(key) + len(key)
        raw[at: at + 4] = (13).to_bytes(4, "little")
        path = tmp_path / "m.gguf"
        path.write_bytes(bytes(raw))
    else:
        path = f.write(tmp_path / "m.gguf")
    with pytest.raises(_lib.TsxError) as e:
        GgufModel(str(path))
    assert e.value.rc == _lib.TSX_ERR_FORMAT and text in str(e.value)


def test_truncated_header_and_payload_past_the_end(tmp_path):
    raw = small_model().to_bytes()
    hdr_end = raw.index(b"w.odd") + 5 + 4 + 8 + 4 + 8
    for cut in (3, 20, 60, hdr_end - 1):
        p = tmp_path / f"t{cut}.gguf"
        p.write_bytes(raw[:cut])
        with pytest.raises(_lib.TsxError) as e:
            GgufModel(str(p))
        assert e.value.rc == _lib.TSX_ERR_FORMAT, cut
    # the payloads cut off: the directory opens, the cut tensors have no data
    p = tmp_path / "short.gguf"
    p.write_bytes(raw[: len(raw) - 50])
    with GgufModel(str(p)) as g:
        t = {x.name: x for x in g.tensors()}
        assert t["w.f32"].data != 0 and t["w.iq3"].data == 0


def test_split_models(tmp_path):
    parts = []
    for i in range(3):
        f = GgufFile()
        if i == 0:
            f.kv("general.architecture", STRING, "qwen35moe")
        f.kv("split.count", U16, 3).kv("split.no", U16, i).kv("split.tensors.count", I32, 3)
        if i > 0:
            f.add(f"t{i}", Q8_0, (32, i), rnd(34 * i, 10 + i))
        if i == 2:
            f.add("t3", F32_T, (2,), np.ones(2, np.float32))
        parts.append(f)
    names = [str(tmp_path / f"model-{i + 1:05d}-of-00003.gguf") for i in range(3)]
    for f, n in zip(parts, names):
        f.write(n)
    assert split_paths(names[1]) == names
    assert split_paths(str(tmp_path / "plain.gguf")) == [str(tmp_path / "plain.gguf")]
    with GgufModel(names[2]) as g:
        assert g.shard_count == 3
        assert [t.name for t in g.tensors()] == ["t1", "t2", "t3"]
        assert g.find("t1").shard == 1 and g.find("t2").shard == 2 and g.find("t3").shard == 2
        assert g.tensor_bytes("t2").tobytes() == parts[2].tensors[0].data
        assert g.meta("general.architecture") == "qwen35moe"
    # a shard that does not declare itself, a count that does not add up, a missing shard, a lone shard 1
    bad = GgufFile().kv("split.count", U16, 3).kv("split.no", U16, 0).kv("split.tensors.count", I32, 3)
    bad.write(names[1])
    with pytest.raises(_lib.TsxError) as e:
        GgufModel(names[0])
    assert "shard 2 of 3" in str(e.value) and "does not match the set: split.no" in str(e.value)
    parts[1].write(names[1])
    parts[2].tensors.pop()
    parts[2].write(names[2])
    with pytest.raises(_lib.TsxError) as e:
        GgufModel(names[0])
    assert "split.tensors.count" in str(e.value)
    (tmp_path / "model-00003-of-00003.gguf").unlink()
    with pytest.raises(_lib.TsxError) as e:
        GgufModel(names[0])
    assert e.value.rc == _lib.TSX_ERR_NOT_FOUND and "1 of its 3 shard files not found" in str(e.value)
    with pytest.raises(_lib.TsxError) as e:
        GgufModel([names[0]])
    assert "is not a whole model" in str(e.value)


def test_split_names(tmp_path):
    # only "<stem>-NNNNN-of-MMMMM.gguf" with 1 <= NNNNN <= MMMMM names a split model; the stem may hold hyphens and
    # digits of its own, and only the shard number changes between the shards' names
    d = tmp_path / "snap-1-of-2"
    d.mkdir()
    names = [str(d / f"m-7-of-9-{i:05d}-of-00002.gguf") for i in (1, 2)]
    for n in names:
        GgufFile().kv("general.architecture", STRING, "x").write(n)
    assert split_paths(names[1]) == names
    for odd in ("m-0001-of-00002.gguf", "m-00003-of-00002.gguf", "m-00000-of-00002.gguf", "m-00001-of-00002.GGUF",
                "m-00001-of-00002.gguf.part", "-00001-of-00002.gguf"):
        assert split_paths(str(d / odd)) == [str(d / odd)]


def expert_file(gu, dn, n_embd, n_ff, n_exp, seed, shared=True, layer=3):
    gu_row, d_row = ops.iq_row_bytes(gu, n_embd), ops.iq_row_bytes(dn, n_ff)
    gate, up = rnd(n_exp * n_ff * gu_row, seed), rnd(n_exp * n_ff * gu_row, seed + 1)
    down = rnd(n_exp * n_embd * d_row, seed + 2)
    f = GgufFile().kv("general.architecture", STRING, "qwen35moe")
    f.add(f"blk.{layer}.ffn_gate_exps.weight", gu, (n_embd, n_ff, n_exp), gate)
    f.add(f"blk.{layer}.ffn_up_exps.weight", gu, (n_embd, n_ff, n_exp), up)
    f.add(f"blk.{layer}.ffn_down_exps.weight", dn, (n_ff, n_embd, n_exp), down)
    sh = None
    if shared:
        sh = (rnd(n_ff * gu_row, seed + 3), rnd(n_ff * gu_row, seed + 4), rnd(n_embd * d_row, seed + 5))
        f.add(f"blk.{layer}.ffn_gate_shexp.weight", gu, (n_embd, n_ff), sh[0])
        f.add(f"blk.{layer}.ffn_up_shexp.weight", gu, (n_embd, n_ff), sh[1])
        f.add(f"blk.{layer}.ffn_down_shexp.weight", dn, (n_ff, n_embd), sh[2])
    return f, (gate, up, down), sh


@pytest.mark.parametrize("gu,dn,n_embd,n_ff", [(IQ3_XXS, IQ3_S, 512, 256), (Q4_K, Q4_K, 256, 256),
                                               (Q8_0, Q8_0, 256, 64)])
def test_expert_repack(tmp_path, gu, dn, n_embd, n_ff):
    n_exp = 5
    f, (gate, up, down), sh = expert_file(gu, dn, n_embd, n_ff, n_exp, seed=7)
    path = f.write(tmp_path / "e.gguf")
    L = ops.native_expert_layout(gu, dn, n_embd, n_ff)
    gsz, dsz = n_ff * L.gu_row, n_embd * L.d_row
    with GgufModel(path) as g:
        src = g.layer_experts(3)
        assert src.n_expert == n_exp
        assert (src.L.gu_type, src.L.d_type, src.L.n_embd, src.L.n_ff, src.L.bytes) == (gu, dn, n_embd, n_ff, L.bytes)
        al = math.lcm(math.lcm(block_geometry(gu)[1], block_geometry(dn)[1]), 16)
        assert src.stride % al == 0 and src.stride - al < L.bytes <= src.stride
        for e in range(n_exp):
            want = np.concatenate([gate[e * gsz:(e + 1) * gsz], up[e * gsz:(e + 1) * gsz], down[e * dsz:(e + 1) * dsz]])
            assert np.array_equal(g.expert_blob(src, e), want), e
        s = g.layer_experts(3, shared=True)
        assert s.n_expert == 1 and s.L.bytes == L.bytes
        assert np.array_equal(g.expert_blob(s, 0), np.concatenate(sh))
        with pytest.raises(_lib.TsxError) as e:
            g.layer_experts(4)
        assert e.value.rc == _lib.TSX_ERR_NOT_FOUND and "blk.4.ffn_gate_exps.weight" in str(e.value)


def test_expert_repack_refusals(tmp_path):
    # a type pair the kernels do not take, gate/up shapes that differ, a down of the wrong shape
    f, _, _ = expert_file(IQ3_XXS, IQ3_S, 512, 256, 2, seed=1, shared=False)
    f.tensors[1].type = Q4_K
    f.tensors[1].data = rnd(2 * 256 * 2 * 144, 9).tobytes()
    with GgufModel(f.write(tmp_path / "a.gguf")) as g:
        with pytest.raises(_lib.TsxError) as e:
            g.layer_experts(3)
        assert e.value.rc == _lib.TSX_ERR_FORMAT and "gate and up differ" in str(e.value)
    f, _, _ = expert_file(IQ3_XXS, IQ3_S, 512, 256, 2, seed=1, shared=False)
    f.tensors[2].shape = (256, 256, 2)
    f.tensors[2].data = rnd(2 * 256 * 110, 9).tobytes()
    with GgufModel(f.write(tmp_path / "b.gguf")) as g:
        with pytest.raises(_lib.TsxError) as e:
            g.layer_experts(3)
        assert "down is not [n_ff, n_embd" in str(e.value)
    f = GgufFile()
    for p in ("gate", "up"):
        f.add(f"blk.0.ffn_{p}_exps.weight", 16, (256, 32, 2), rnd(2 * 32 * 66, 2))  # IQ2_XXS
    f.add("blk.0.ffn_down_exps.weight", 16, (32, 256, 2), rnd(64, 3))
    with GgufModel(f.write(tmp_path / "c.gguf")) as g:
        with pytest.raises(_lib.TsxError) as e:
            g.layer_experts(0)
        assert e.value.rc == _lib.TSX_ERR_UNSUPPORTED


def test_upload_argument_checks(tmp_path):
    f, _, _ = expert_file(IQ3_XXS, IQ3_S, 512, 256, 3, seed=2, shared=False)
    with GgufModel(f.write(tmp_path / "u.gguf")) as g:
        src = g.layer_experts(3)
        lib = _lib.lib()
        import ctypes as C
        assert lib.tsx_gguf_upload_experts(C.byref(src.raw), 0, 4, 16, src.stride, None) == _lib.TSX_ERR_ARG
        assert lib.tsx_gguf_upload_experts(C.byref(src.raw), 0, 1, 16, src.L.bytes - 16, None) == _lib.TSX_ERR_ARG
        assert lib.tsx_gguf_upload_experts(C.byref(src.raw), 0, 1, 8, src.stride, None) == _lib.TSX_ERR_ARG
        assert lib.tsx_gguf_upload_experts(C.byref(src.raw), 0, 0, 16, src.stride, None) == _lib.TSX_OK
