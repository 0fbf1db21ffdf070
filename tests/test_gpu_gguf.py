"""A layer's experts loaded from a GGUF model file onto the GPU (tinystrata_amd.gguf.GgufModel.load_layer): the device
blobs equal the reference repack (expert_blob, src/qwen35/q36_engine.cu:1196-1201) byte for byte, and the decode
layer on them gives the same outputs, bit for bit, as on the same experts placed by the test pool."""
import numpy as np
import pytest
import torch

from tinystrata_amd import moe, ops
from tinystrata_amd._lib import IQ3_S, IQ3_XXS
from tinystrata_amd.gguf import GgufModel

from gguf_writer import STRING, U32, GgufFile
from gpu_util import dev, host, pool

pytestmark = pytest.mark.gpu


def gguf_from_blobs(path, L, blobs, shared_blob, layer):
    """A one-layer model whose ffn_*_exps hold the given blobs' parts (and the shared expert's, when given)."""
    N, FF = L.n_embd, L.n_ff
    gsz, dsz = L.up_off, L.bytes - L.down_off
    f = GgufFile().kv("general.architecture", STRING, "qwen35moe").kv("qwen35moe.expert_count", U32, len(blobs))
    E = len(blobs)
    f.add(f"blk.{layer}.ffn_gate_exps.weight", L.gu_type, (N, FF, E), np.concatenate([b[:gsz] for b in blobs]))
    f.add(f"blk.{layer}.ffn_up_exps.weight", L.gu_type, (N, FF, E),
          np.concatenate([b[L.up_off:L.up_off + gsz] for b in blobs]))
    f.add(f"blk.{layer}.ffn_down_exps.weight", L.d_type, (FF, N, E),
          np.concatenate([b[L.down_off:L.down_off + dsz] for b in blobs]))
    if shared_blob is not None:
        f.add(f"blk.{layer}.ffn_gate_shexp.weight", L.gu_type, (N, FF), shared_blob[:gsz])
        f.add(f"blk.{layer}.ffn_up_shexp.weight", L.gu_type, (N, FF), shared_blob[L.up_off:L.up_off + gsz])
        f.add(f"blk.{layer}.ffn_down_shexp.weight", L.d_type, (FF, N), shared_blob[L.down_off:L.down_off + dsz])
    return f.write(path)


@pytest.mark.parametrize("T", [1, 4])
def test_gguf_layer_on_the_gpu(tmp_path, T):
    N, FF, E, k, distinct = 2048, 512, 64, 8, 6
    L = ops.native_expert_layout(IQ3_XXS, IQ3_S, N, FF)
    p = pool(IQ3_XXS, IQ3_S, N, FF, distinct, 0)
    order = (np.arange(E) * 5 + 3) % (distinct - 1)
    blobs = [p[o][: L.bytes] for o in order]
    path = gguf_from_blobs(tmp_path / "layer.gguf", L, blobs, p[distinct - 1][: L.bytes], layer=2)
    print(f"GGUF layer T={T}: {E} IQ3_XXS/IQ3_S experts of {L.bytes} bytes", flush=True)
    with GgufModel(str(path)) as g:
        Wg = g.load_layer(2, "cuda")
        assert Wg.n_expert == E and Wg.stride % 16 == 0 and Wg.shared is not None
        got = host(Wg.blobs).reshape(E, Wg.stride)
        for e in range(E):
            assert np.array_equal(got[e, : L.bytes], g.expert_blob(g.layer_experts(2), e)), e
            assert np.array_equal(got[e, : L.bytes], blobs[e]), e
        assert np.array_equal(host(Wg.shared)[: L.bytes], p[distinct - 1][: L.bytes])
    Wp = moe.weights_from_pool(L, dev(p), E, order, distinct - 1)
    rng = np.random.default_rng(T)
    x = rng.normal(0, 1, (T, N)).astype(np.float32)
    logits = rng.normal(0, 1, (T, E)).astype(np.float32)
    sgate = rng.normal(0, 1, T).astype(np.float32)
    outs = []
    for W in (Wg, Wp):
        layer = moe.MoELayer(W, k, T, torch.device("cuda"))
        y = torch.zeros((T, N), device="cuda")
        layer(dev(x), dev(logits), dev(sgate), y)
        outs.append((host(y), host(layer.ids)))
    assert np.array_equal(outs[0][1], outs[1][1])
    assert np.array_equal(outs[0][0], outs[1][0])
