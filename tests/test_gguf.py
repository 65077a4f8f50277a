"""GGUF files: the reader (``gguf_model.GGUFFile``: metadata, tensor infos, raw tensors at the aligned offsets) on
a file written here, and ``MoELayer.from_gguf`` building a block's layer from one (the reference's loader path,
``src/artlite/gguf_model.py:396-525`` and ``model_config.py:735-766``)."""

import numpy as np
import pytest

from artlite_amd.gguf_model import TYPE_ID, GGUFFile
from oracle import layers

from .gguf_write import write_gguf
from .helpers import gpu_input, gpu_layer, layer_args


def block_file(path, spec: layers.Spec, layer: layers.Layer, block: int = 3, gating: int = 1) -> None:
    H, E, F = spec.H, spec.E, spec.F
    b = f"blk.{block}."
    t = [(b + "ffn_gate_inp.weight", (H, E), 0, layer.router),
         (b + "ffn_gate_exps.weight", (H, F, E), TYPE_ID[spec.gate_type], layer.gate),
         (b + "ffn_up_exps.weight", (H, F, E), TYPE_ID[spec.gate_type], layer.up),
         (b + "ffn_down_exps.weight", (F, H, E), TYPE_ID[spec.down_type], layer.down)]
    if layer.shared is not None:
        g, u, d = layer.shared
        st, sdt = TYPE_ID[spec.shared_type], TYPE_ID[spec.sdown_type]
        t += [(b + "ffn_gate_shexp.weight", (H, spec.shared_F), st, g), (b + "ffn_up_shexp.weight", (H, spec.shared_F), st, u),
              (b + "ffn_down_shexp.weight", (spec.shared_F, H), sdt, d)]
    if layer.shared_inp is not None:
        t.append((b + "ffn_gate_inp_shexp.weight", (H,), 0, layer.shared_inp))
    meta = {"general.architecture": "qwen3moe", "general.alignment": 64, "qwen3moe.block_count": block + 1,
            "qwen3moe.embedding_length": H, "qwen3moe.expert_count": E, "qwen3moe.expert_used_count": spec.k,
            "qwen3moe.expert_feed_forward_length": F, "qwen3moe.expert_gating_func": gating,
            "general.name": "synthetic", "qwen3moe.rope_pattern": [1, 0, 1]}
    if layer.shared is not None:
        meta["qwen3moe.expert_shared_feed_forward_length"] = spec.shared_F
    write_gguf(str(path), meta, t, alignment=64)


def test_gguf_reader(tmp_path) -> None:
    spec = layers.CONFIGS["mix_k8"]
    layer = layers.make_layer(spec, 2)
    block_file(tmp_path / "m.gguf", spec, layer)
    g = GGUFFile(str(tmp_path / "m.gguf"))
    assert g.arch == "qwen3moe" and g.arch_meta("expert_count") == spec.E and g.meta["general.name"] == "synthetic"
    assert list(g.arch_meta("rope_pattern")) == [1, 0, 1]
    dims, qtype, off, nbytes = g.tensor_info["blk.3.ffn_gate_exps.weight"]
    assert dims == (spec.H, spec.F, spec.E) and qtype == spec.gate_type and off % 64 == 0
    assert nbytes == layer.gate.nbytes
    for name, want in (("ffn_gate_exps", layer.gate), ("ffn_down_exps", layer.down), ("ffn_gate_shexp", layer.shared[0])):
        t = g.tensor(f"blk.3.{name}.weight")
        assert np.array_equal(np.asarray(t.raw).reshape(-1), want.reshape(-1).view(np.uint8)), name
    r = g.tensor("blk.3.ffn_gate_inp.weight")
    assert r.qtype == "F32" and np.array_equal(np.asarray(r.raw), layer.router)
    with pytest.raises(ValueError):
        (tmp_path / "bad.gguf").write_bytes(b"GGUX" + bytes(32))
        GGUFFile(str(tmp_path / "bad.gguf"))


@pytest.mark.gpu
@pytest.mark.parametrize(("name", "T", "gating"), [("decode", 16, 1), ("mix_q8k", 16, 2), ("prefill", 256, 1),
                                                ("kquants", 32, 1)])
def test_layer_from_gguf(tmp_path, name: str, T: int, gating: int) -> None:
    from artlite_amd.moe.layer import MoELayer

    spec = layers.CONFIGS[name]
    layer = layers.make_layer(spec, 4)
    block_file(tmp_path / "m.gguf", spec, layer, gating=gating)
    x = gpu_input(spec, layers.make_x(spec, T, 4))
    with MoELayer.from_gguf(GGUFFile(str(tmp_path / "m.gguf")), 3, max_tokens=T) as a:
        got = a(x)
    g = gpu_layer(layer, max_tokens=T) if gating == 1 else None
    if g is None:
        from artlite_amd.moe.layer import MoELayer as L

        g = L(**layer_args(layer.spec, T), gating="sigmoid")
        for n, t in (("ffn_gate_inp", layer.router), ("ffn_gate_exps", layer.gate), ("ffn_up_exps", layer.up),
                     ("ffn_down_exps", layer.down), ("ffn_gate_shexp", layer.shared[0]),
                     ("ffn_up_shexp", layer.shared[1]), ("ffn_down_shexp", layer.shared[2]),
                     ("ffn_gate_inp_shexp", layer.shared_inp)):
            g.upload(n, t)
    with g:
        want = g(x)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_from_gguf_errors(tmp_path) -> None:
    spec = layers.CONFIGS["cpu"]
    layer = layers.make_layer(spec, 0)
    write_gguf(str(tmp_path / "n.gguf"), {"general.architecture": "qwen3moe", "qwen3moe.embedding_length": spec.H},
               [("blk.0.ffn_gate_inp.weight", (spec.H, spec.E), 0, layer.router)])
    from artlite_amd.moe.layer import MoELayer

    with pytest.raises(ValueError, match="no MoE FFN"):
        MoELayer.from_gguf(GGUFFile(str(tmp_path / "n.gguf")), 0, max_tokens=4)
