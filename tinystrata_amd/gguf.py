"""GGUF models through libtsx_moe's reader (include/tsx_gguf.h): the tensor directory and metadata of a (split)
GGUF v3 model, and a layer's routed and shared experts uploaded as the [gate | up | down] blobs the expert kernels
read.

Mirrors the reference's strata::GgufModel / GgufFile (include/strata/artifact/gguf_reader.hpp:233-666) and its
loader's expert repack (src/qwen35/q36_engine.cu:1144-1168, expert_blob :1196-1201).  The parsing is the library's
(C++, mmap); this module only holds the handle and converts values.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np
import torch

from . import _lib
from ._lib import ExpertLayout, GgufExperts, GgufTensor, check, lib
from .moe import MoEWeights

META_TYPES = ("U8", "I8", "U16", "I16", "U32", "I32", "F32", "BOOL", "STRING", "ARRAY", "U64", "I64", "F64")
_SIGNED = {1, 3, 5, 11}
_FLOAT = {6, 12}


def block_geometry(ggml_type: int) -> tuple[int, int]:
    """(values, bytes) per block of a ggml type id (reference block_geometry); raises for an unknown id."""
    e, b = C.c_int(), C.c_int()
    check(lib().tsx_gguf_block_geometry(ggml_type, C.byref(e), C.byref(b)), "gguf block_geometry")
    return e.value, b.value


def split_paths(any_shard: str) -> list[str]:
    """The shards of the model `any_shard` belongs to, in split order (reference gguf_split_paths)."""
    n, need = C.c_int(), C.c_size_t()
    rc = lib().tsx_gguf_split_paths(any_shard.encode(), None, 0, C.byref(n), C.byref(need))
    if rc not in (_lib.TSX_OK, _lib.TSX_ERR_ARG):
        check(rc, "gguf split_paths")
    buf = C.create_string_buffer(need.value)
    check(lib().tsx_gguf_split_paths(any_shard.encode(), buf, need.value, C.byref(n), C.byref(need)),
          "gguf split_paths")
    return [p.decode() for p in buf.raw[: need.value].split(b"\0")[: n.value]]


@dataclass(frozen=True)
class TensorInfo:
    """One directory entry (reference TensorInfo): shape in GGUF order, dim 0 fastest."""

    name: str
    type: int
    shape: tuple[int, ...]
    offset: int
    bytes: int
    shard: int
    data: int  # address of the payload in the mapping, 0 when it is unknown or outside the file


@dataclass(frozen=True)
class ExpertSource:
    """A layer's routed (or shared) experts inside the mapped model."""

    L: ExpertLayout
    stride: int
    n_expert: int
    raw: GgufExperts


class GgufModel:
    """An open GGUF v3 model: every shard mapped read-only until close()."""

    def __init__(self, path: str | list[str]):
        h = C.c_void_p()
        if isinstance(path, str):
            rc = lib().tsx_gguf_open_model(path.encode(), C.byref(h))
        else:
            arr = (C.c_char_p * len(path))(*[p.encode() for p in path])
            rc = lib().tsx_gguf_open(arr, len(path), C.byref(h))
        check(rc, f"gguf open {path}")
        self._h = h

    def close(self) -> None:
        if self._h:
            lib().tsx_gguf_close(self._h)
            self._h = C.c_void_p()

    def __enter__(self) -> "GgufModel":
        return self

    def __exit__(self, *exc) -> None:
        self.close()

    def __del__(self) -> None:
        try:
            self.close()
        except Exception:
            pass

    # ---- the directory
    @property
    def shard_count(self) -> int:
        return lib().tsx_gguf_shard_count(self._h)

    def shard_info(self, shard: int = 0) -> dict:
        v, a, d, s = C.c_uint32(), C.c_uint64(), C.c_uint64(), C.c_uint64()
        check(lib().tsx_gguf_shard_info(self._h, shard, C.byref(v), C.byref(a), C.byref(d), C.byref(s)),
              "gguf shard_info")
        return {"version": v.value, "alignment": a.value, "data_start": d.value, "file_size": s.value}

    @staticmethod
    def _info(t: GgufTensor) -> TensorInfo:
        return TensorInfo(name=t.name.decode(), type=t.type, shape=tuple(t.ne[: t.n_dims]), offset=t.offset,
                          bytes=t.bytes, shard=t.shard, data=t.data or 0)

    def tensors(self) -> list[TensorInfo]:
        out = []
        for i in range(lib().tsx_gguf_tensor_count(self._h)):
            t = GgufTensor()
            check(lib().tsx_gguf_tensor_at(self._h, i, C.byref(t)), "gguf tensor_at")
            out.append(self._info(t))
        return out

    def find(self, name: str) -> TensorInfo | None:
        t = GgufTensor()
        rc = lib().tsx_gguf_find(self._h, name.encode(), C.byref(t))
        if rc == _lib.TSX_ERR_NOT_FOUND:
            return None
        check(rc, f"gguf find {name}")
        return self._info(t)

    def tensor_bytes(self, name: str) -> np.ndarray:
        """A tensor's payload as a read-only uint8 view of the mapping (valid while the model is open)."""
        t = self.find(name)
        if t is None or not t.data:
            raise KeyError(f"{name}: no tensor, or its payload is not inside the file")
        buf = (C.c_uint8 * t.bytes).from_address(t.data)
        a = np.frombuffer(buf, dtype=np.uint8)
        a.flags.writeable = False
        return a

    # ---- metadata
    def keys(self) -> list[str]:
        return [lib().tsx_gguf_meta_key(self._h, i).decode() for i in range(lib().tsx_gguf_meta_count(self._h))]

    def meta(self, key: str, default=None):
        """The value of a metadata key: int, float, bool, str, or a list of the (first 64) array items."""
        ty, u, i, f, s, et, n = C.c_int(), C.c_uint64(), C.c_int64(), C.c_double(), C.c_char_p(), C.c_int(), C.c_uint64()
        rc = lib().tsx_gguf_meta(self._h, key.encode(), C.byref(ty), C.byref(u), C.byref(i), C.byref(f), C.byref(s),
                                 C.byref(et), C.byref(n))
        if rc == _lib.TSX_ERR_NOT_FOUND:
            return default
        check(rc, f"gguf meta {key}")
        return self._value(ty.value, u.value, i.value, f.value, s.value, key, et.value, n.value)

    def _value(self, ty, u, i, f, s, key, et, n):
        if ty == 9 and et < 0:
            return None  # an array inside an array: only the top level's items are readable
        if ty == 9:
            items = []
            for k in range(min(n, 64)):
                iu, fi, si = C.c_uint64(), C.c_double(), C.c_char_p()
                check(lib().tsx_gguf_meta_item(self._h, key.encode(), k, C.byref(iu), C.byref(fi), C.byref(si)),
                      "gguf meta_item")
                items.append(self._value(et, iu.value, C.c_int64(iu.value).value, fi.value, si.value, key, -1, 1))
            return items
        if ty == 8:
            return s.decode(errors="replace") if s is not None else ""
        if ty == 7:
            return bool(u)
        if ty in _FLOAT:
            return f
        return i if ty in _SIGNED else u

    # ---- experts
    def layer_experts(self, layer: int, shared: bool = False) -> ExpertSource:
        X = GgufExperts()
        check(lib().tsx_gguf_layer_experts(self._h, layer, int(shared), C.byref(X)),
              f"gguf layer {layer} {'shared expert' if shared else 'experts'}")
        return ExpertSource(L=X.L, stride=X.stride, n_expert=X.n_expert, raw=X)

    def expert_blob(self, src: ExpertSource, e: int) -> np.ndarray:
        """Expert e's [gate | up | down] blob (host bytes, reference expert_blob)."""
        out = np.zeros(src.L.bytes, np.uint8)
        check(lib().tsx_gguf_expert_blob(C.byref(src.raw), e, out.ctypes.data), "gguf expert_blob")
        return out

    def upload_experts(self, src: ExpertSource, dst: torch.Tensor, stride: int | None = None, e0: int = 0,
                       n: int | None = None, stream=None) -> None:
        """Experts e0 .. e0 + n - 1 into the device buffer dst (uint8), blob j at dst + j * stride; enqueued on the
        stream (the caller synchronizes before closing the model)."""
        stride = src.stride if stride is None else stride
        n = src.n_expert - e0 if n is None else n
        assert dst.dtype == torch.uint8 and dst.is_cuda and dst.numel() >= n * stride
        s = stream if stream is not None else torch.cuda.current_stream(dst.device).cuda_stream
        check(lib().tsx_gguf_upload_experts(C.byref(src.raw), e0, n, dst.data_ptr(), stride, s), "gguf upload")

    def load_layer(self, layer: int, device: torch.device | str = "cuda", with_shared: bool = True) -> MoEWeights:
        """A layer's experts (and shared expert, when the model has one) on the device as MoEWeights, at the
        reference's blob stride."""
        src = self.layer_experts(layer)
        blobs = torch.empty(src.n_expert * src.stride, dtype=torch.uint8, device=device)
        self.upload_experts(src, blobs)
        shared = None
        if with_shared and self.find(f"blk.{layer}.ffn_gate_shexp.weight") is not None:
            sh = self.layer_experts(layer, shared=True)
            if (sh.L.gu_type, sh.L.d_type, sh.L.n_embd, sh.L.n_ff) != (src.L.gu_type, src.L.d_type, src.L.n_embd,
                                                                      src.L.n_ff):
                raise ValueError(f"layer {layer}: the shared expert's layout differs from the routed experts'")
            shared = torch.empty(src.stride, dtype=torch.uint8, device=device)
            self.upload_experts(sh, shared, stride=src.stride)
        torch.cuda.current_stream(blobs.device).synchronize()
        return MoEWeights(L=src.L, n_expert=src.n_expert, stride=src.stride, blobs=blobs, shared=shared)
