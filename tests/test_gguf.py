"""GGUF files written here, read back: the reader's header parsing (``gguf_model.GGUFFile``), ``GGUFFile.rows`` against
the oracle's dequantization bit for bit, and ``MoELayer.from_gguf`` against the layer oracle (the reference's loader
path: ``src/artlite/gguf_model.py:494-525``, ``tests/moe/ref.py:27-40``, ``model_config.py:735-766``)."""

import struct

import numpy as np
import pytest

from artlite_amd.gguf_model import TYPE_ID, GGUFFile
from oracle import gguf_ref, layers, tensors

from .gguf_write import write_gguf
from .helpers import check_against_oracle, gpu_input


def block_file(path, spec: layers.Spec, layer: layers.Layer, block: int = 3, gating: int = 1,
               extra: dict | None = None) -> None:
    """A qwen3moe-style file holding one MoE block ``block`` of the layer (3-D expert tensors, dims H, F, E)."""
    H, E, F = spec.H, spec.E, spec.F
    b = f"blk.{block}."
    t = [(b + "ffn_gate_inp.weight", (H, E), 0, layer.router),
         (b + "ffn_gate_exps.weight", (H, F, E), TYPE_ID[spec.gate_type], layer.gate),
         (b + "ffn_up_exps.weight", (H, F, E), TYPE_ID[spec.gate_type], layer.up),
         (b + "ffn_down_exps.weight", (F, H, E), TYPE_ID[spec.down_type], layer.down)]
    if layer.shared is not None:
        g, u, d = layer.shared
        st, sdt = TYPE_ID[spec.shared_type], TYPE_ID[spec.sdown_type]
        Fs = spec.shared_F
        t += [(b + "ffn_gate_shexp.weight", (H, Fs), st, g), (b + "ffn_up_shexp.weight", (H, Fs), st, u),
              (b + "ffn_down_shexp.weight", (Fs, H), sdt, d)]
    if layer.shared_inp is not None:
        t.append((b + "ffn_gate_inp_shexp.weight", (H,), 0, layer.shared_inp))
    meta = {"general.architecture": "qwen3moe", "general.alignment": 64, "qwen3moe.block_count": block + 1,
            "qwen3moe.embedding_length": H, "qwen3moe.expert_count": E, "qwen3moe.expert_used_count": spec.k,
            "qwen3moe.expert_feed_forward_length": F, "qwen3moe.expert_gating_func": gating,
            "general.name": "synthetic", "qwen3moe.rope_pattern": [1, 0, 1]}
    if layer.shared is not None:
        meta["qwen3moe.expert_shared_feed_forward_length"] = spec.shared_F
    meta.update(extra or {})
    write_gguf(str(path), meta, t, alignment=64)


def test_gguf_header(tmp_path) -> None:
    """Metadata of every value type, string arrays left in the file until read, tensor infos at the aligned data
    start, tensor views of the mapped bytes."""
    spec = layers.CONFIGS["mix_k8"]
    layer = layers.make_layer(spec, 2)
    extra = {"tokenizer.ggml.tokens": ["<s>", "héllo", "", "wörld"], "t.u8": (0, 200), "t.i16": (3, -7),
             "t.u64": (10, 2 ** 40 + 3), "t.f64": (12, 0.1), "t.flag": True, "t.big": -2 ** 40, "t.f32": 0.5,
             "t.floats": [0.25, -1.5]}
    block_file(tmp_path / "m.gguf", spec, layer, extra=extra)
    with GGUFFile(str(tmp_path / "m.gguf")) as g:
        assert g.arch == "qwen3moe" and g.arch_meta("expert_count") == spec.E and g.meta["general.name"] == "synthetic"
        assert list(g.arch_meta("rope_pattern")) == [1, 0, 1]
        assert list(g.meta["tokenizer.ggml.tokens"]) == ["<s>", "héllo", "", "wörld"]
        assert g.meta["tokenizer.ggml.tokens"][3] == "wörld" and len(g.meta["tokenizer.ggml.tokens"]) == 4
        assert g.meta["t.u8"] == 200 and g.meta["t.i16"] == -7 and g.meta["t.u64"] == 2 ** 40 + 3
        assert g.meta["t.f64"] == 0.1 and g.meta["t.flag"] is True and g.meta["t.big"] == -2 ** 40
        assert g.meta["t.f32"] == 0.5 and g.meta["t.floats"].tolist() == [0.25, -1.5]
        info = g.tensor_info["blk.3.ffn_gate_exps.weight"]
        assert info.dims == (spec.H, spec.F, spec.E) and info.qtype == spec.gate_type and info.offset % 64 == 0
        assert info.nbytes == layer.gate.nbytes
        for name, want in (("ffn_gate_exps", layer.gate), ("ffn_down_exps", layer.down),
                           ("ffn_gate_shexp", layer.shared[0])):
            t = g.tensor(f"blk.3.{name}.weight")
            assert np.array_equal(np.asarray(t.raw).reshape(-1), want.reshape(-1).view(np.uint8)), name
        r = g.tensor("blk.3.ffn_gate_inp.weight")
        assert r.qtype == "F32" and r.raw.shape == (spec.E, spec.H) and np.array_equal(r.raw, layer.router)
        del t, r


def test_gguf_header_errors(tmp_path) -> None:
    """Bad magic, an unread version, a file cut short in its header or in a tensor."""
    p = tmp_path / "bad.gguf"
    p.write_bytes(b"GGUX" + bytes(32))
    with pytest.raises(ValueError, match="not a GGUF file"):
        GGUFFile(str(p))
    p.write_bytes(b"GGUF" + struct.pack("<IQQ", 1, 0, 0))
    with pytest.raises(ValueError, match="version 1"):
        GGUFFile(str(p))
    p.write_bytes(b"GGUF" + struct.pack("<IQQ", 3, 0, 5) + bytes(8))
    with pytest.raises(ValueError, match="past the end"):
        GGUFFile(str(p))
    spec = layers.CONFIGS["cpu"]
    layer = layers.make_layer(spec, 0)
    block_file(tmp_path / "cut.gguf", spec, layer)
    data = (tmp_path / "cut.gguf").read_bytes()
    (tmp_path / "cut.gguf").write_bytes(data[:len(data) - 4096])
    with pytest.raises(ValueError, match="runs past the end of the file"):
        GGUFFile(str(tmp_path / "cut.gguf"))


@pytest.mark.gpu
@pytest.mark.parametrize("qtype", ["Q4_0", "Q8_0", "Q4_K", "Q6_K", "Q3_K", "IQ4_XS", "F16", "BF16", "F32"])
def test_gguf_rows(tmp_path, qtype: str) -> None:
    """``rows`` of a 3-D expert tensor (an expert's rows, as ``tests/moe/ref.py:27-40`` reads them; scattered rows;
    the leading columns; with and without the page prefetch) equal the oracle's dequantization bit for bit."""
    E, F, H = 5, 24, 512
    rng = np.random.default_rng(TYPE_ID[qtype])
    if qtype in ("F16", "BF16", "F32"):
        vals = rng.standard_normal((E * F, H)).astype(np.float32)
        raw = {"F16": vals.astype(np.float16).view(np.uint8), "F32": vals.view(np.uint8),
               "BF16": tensors.bf16_bits(vals).view(np.uint8)}[qtype].reshape(E * F, -1)
    else:
        raw = tensors.random_blocks(qtype, E * F, H, rng)
    write_gguf(str(tmp_path / "r.gguf"), {"general.architecture": "x"}, [("w", (H, F, E), TYPE_ID[qtype], raw)])
    want = gguf_ref.dequantize(qtype, raw, H)
    with GGUFFile(str(tmp_path / "r.gguf")) as g:
        for idx, prefetch in ((np.arange(2 * F, 3 * F), True), (np.array([7, 0, 119, 7, 64]), False),
                              (np.array([5]), True), (np.arange(E * F)[::-1], True)):
            got = g.rows("w", idx, prefetch=prefetch)
            assert got.view(np.uint32).tobytes() == want[idx].view(np.uint32).tobytes(), (qtype, idx[:3])
        per = gguf_ref.BLOCKS[qtype][0]
        c = 256 if per == 256 else 64
        got = g.rows("w", [3, 4], cols=c)
        assert got.view(np.uint32).tobytes() == want[[3, 4], :c].view(np.uint32).tobytes()
        with pytest.raises(IndexError):
            g.rows("w", [E * F])
        if per > 1:
            with pytest.raises(ValueError, match="in blocks of"):
                g.rows("w", [0], cols=per + 1 if per < H else 16)


@pytest.mark.gpu
@pytest.mark.parametrize(("name", "T", "gating"), [("decode", 16, 1), ("mix_q8k", 16, 2), ("prefill", 256, 1),
                                                ("kquants", 32, 1), ("iq4", 24, 2)])
def test_layer_from_gguf(tmp_path, name: str, T: int, gating: int) -> None:
    """A block loaded by ``from_gguf`` against the layer oracle (routing, dispatch and output; sigmoid gating from
    ``expert_gating_func`` 2)."""
    from artlite_amd.moe.layer import MoELayer

    spec = layers.CONFIGS[name]
    layer = layers.make_layer(spec, 4)
    block_file(tmp_path / "m.gguf", spec, layer, gating=gating)
    x = layers.make_x(spec, T, 4)
    with GGUFFile(str(tmp_path / "m.gguf")) as f, MoELayer.from_gguf(f, 3, max_tokens=T) as a:
        y = a(gpu_input(spec, x))
        check_against_oracle(a, layer, x, y, gating="sigmoid" if gating == 2 else "softmax")


def test_from_gguf_errors(tmp_path) -> None:
    """A block without an MoE FFN, and routing the layer does not compute, are refused with ValueError before any
    device work."""
    from artlite_amd.moe.layer import MoELayer

    spec = layers.CONFIGS["cpu"]
    layer = layers.make_layer(spec, 0)
    write_gguf(str(tmp_path / "n.gguf"), {"general.architecture": "qwen3moe", "qwen3moe.embedding_length": spec.H},
               [("blk.0.ffn_gate_inp.weight", (spec.H, spec.E), 0, layer.router)])
    with GGUFFile(str(tmp_path / "n.gguf")) as f, pytest.raises(ValueError, match="no MoE FFN"):
        MoELayer.from_gguf(f, 0, max_tokens=4)
    for extra, key in (({"qwen3moe.expert_weights_scale": 2.5}, "expert_weights_scale"),
                       ({"qwen3moe.expert_weights_norm": False}, "expert_weights_norm"),
                       ({"qwen3moe.expert_group_count": 8}, "expert_group_count"),
                       ({"qwen3moe.expert_gating_func": 3}, "expert_gating_func"),
                       ({"qwen3moe.expert_gating_func": 0}, "expert_gating_func")):
        block_file(tmp_path / "u.gguf", spec, layer, block=0, extra=extra)
        with GGUFFile(str(tmp_path / "u.gguf")) as f, pytest.raises(ValueError, match=f"not modelled.*{key}"):
            MoELayer.from_gguf(f, 0, max_tokens=4)
    # a selection bias tensor
    block_file(tmp_path / "b.gguf", spec, layer, block=0)
    from .gguf_write import write_gguf as w

    with GGUFFile(str(tmp_path / "b.gguf")) as f:
        tensors_ = [(n, i.dims, TYPE_ID[i.qtype], np.asarray(f.tensor(n).raw).copy()) for n, i in f.tensor_info.items()]
        meta = {k: v for k, v in f.meta.items() if k not in ("qwen3moe.rope_pattern",)}
    tensors_.append(("blk.0.exp_probs_b.bias", (spec.E,), 0, np.zeros(spec.E, np.float32)))
    w(str(tmp_path / "b2.gguf"), meta, tensors_, alignment=64)
    with GGUFFile(str(tmp_path / "b2.gguf")) as f, pytest.raises(ValueError, match="exp_probs_b"):
        MoELayer.from_gguf(f, 0, max_tokens=4)
