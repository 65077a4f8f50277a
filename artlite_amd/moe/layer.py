"""A device-resident MoE FFN layer (``artlite_moe_layer_*``): the reference's MoE block (``src/artlite/moe/prefill.py``,
its semantics ``tests/moe/ref.py:43-60``) on one GPU -- router logits, routing, stable dispatch, the experts' SwiGLU
over raw GGUF blocks, the weighted combine, an optional shared expert.

Tensors are uploaded in their GGUF form under their GGUF names (``ffn_gate_inp``, ``ffn_gate_exps``, ``ffn_up_exps``,
``ffn_down_exps``, ``ffn_gate_shexp``, ``ffn_up_shexp``, ``ffn_down_shexp``, ``ffn_gate_inp_shexp``): the 3-D expert
tensors as their raw block bytes, an expert's matrix contiguous."""

import ctypes

import numpy as np

from .. import _hip
from ..gguf_model import TYPE_ID, GGUFFile

TENSORS = {"ffn_gate_inp": 0, "ffn_gate_exps": 1, "ffn_up_exps": 2, "ffn_down_exps": 3, "ffn_gate_shexp": 4,
           "ffn_up_shexp": 5, "ffn_down_shexp": 6, "ffn_gate_inp_shexp": 7, "ffn_norm": 8}
TAPS = {"logits": 0, "ids": 1, "weights": 2, "counts": 3, "offsets": 4, "order": 5, "slot": 6, "h": 7, "y_pairs": 8,
        "x_norm": 9, "y_shared": 10}
X_F32, X_BF16 = 0, 1


class MoELayer:
    """One MoE layer's weights in HBM and its forward pass. ``x``: (T, H) float32, or uint16 bf16 bit patterns."""

    def __init__(self, *, hidden: int, n_experts: int, top_k: int, expert_ffn: int, gate_type: str, down_type: str,
                 max_tokens: int, shared_ffn: int = 0, shared_type: str = "", shared_gated: bool = False,
                 gating: str = "softmax", norm_eps: float = 0.0, residual: bool = False, shared_down_type: str = ""):
        """norm_eps > 0: x is first RMS-normalised by the uploaded ``ffn_norm`` (the steps before the block's router);
        residual: y += x (the block's residual add after the combine); shared_down_type: the format of
        ``ffn_down_shexp`` when it is not ``shared_type``'s."""
        assert gating in ("softmax", "sigmoid"), gating
        self.H, self.E, self.k, self.F = hidden, n_experts, top_k, expert_ffn
        self.max_tokens = max_tokens
        d = _hip.Desc(hidden=hidden, n_experts=n_experts, top_k=top_k, expert_ffn=expert_ffn,
                      gate_type=TYPE_ID[gate_type], down_type=TYPE_ID[down_type], shared_ffn=shared_ffn,
                      shared_type=TYPE_ID[shared_type] if shared_ffn else 0, shared_gated=int(shared_gated),
                      gating=int(gating == "sigmoid"), max_tokens=max_tokens, norm_eps=norm_eps,
                      residual=int(residual),
                      shared_down_type=TYPE_ID[shared_down_type] if shared_ffn and shared_down_type else 0)
        h = ctypes.c_void_p()
        _hip.check(_hip.lib().artlite_moe_layer_create(ctypes.byref(d), ctypes.byref(h)))
        self._h = h
        self.T = -1

    @property
    def handle(self) -> ctypes.c_void_p:
        if self._h is None:
            raise _hip.Error("MoELayer: closed")
        return self._h

    def close(self) -> None:
        if getattr(self, "_h", None) is not None:
            _hip.lib().artlite_moe_layer_destroy(self._h)
            self._h = None

    def __del__(self) -> None:
        self.close()

    def __enter__(self) -> "MoELayer":
        return self

    def __exit__(self, *exc: object) -> None:
        self.close()

    @classmethod
    def from_gguf(cls, gguf: "GGUFFile", block: int, *, max_tokens: int, norm: bool = False) -> "MoELayer":
        """Block ``block``'s MoE FFN of a GGUF file (``gguf_model.GGUFFile``): its shape from the architecture's
        metadata (``embedding_length``, ``expert_count``, ``expert_used_count``, ``expert_feed_forward_length``,
        ``expert_shared_feed_forward_length``, ``expert_gating_func``: 1 softmax, 2 sigmoid; the reference's
        ``model_config.py:735-766``), its tensors ``blk.{block}.ffn_*`` uploaded as the file holds them (the router
        and a shared gate converted to fp32 exactly when stored as F16 / BF16). norm: with the steps either side,
        the block's ``ffn_norm`` (RMS, eps ``attention.layer_norm_rms_epsilon``) before and the residual add after.
        Raises ValueError for routing the layer does not compute: a gating function other than 1 or 2, a weights
        scale other than 1, ``expert_weights_norm`` false, more than one expert group, an ``exp_probs_b`` bias."""
        b = f"blk.{block}."
        m = gguf.arch_meta
        need = [b + n + ".weight" for n in ("ffn_gate_inp", "ffn_gate_exps", "ffn_up_exps", "ffn_down_exps")]
        missing = [n for n in need if n not in gguf]
        if missing:
            raise ValueError(f"{gguf.path}: block {block} has no MoE FFN ({', '.join(missing)} missing)")
        H, E, k, F = (int(m(key)) for key in ("embedding_length", "expert_count", "expert_used_count",
                                              "expert_feed_forward_length"))
        dims, gtype, _, _ = gguf.tensor_info[b + "ffn_gate_exps.weight"]
        _, utype, _, _ = gguf.tensor_info[b + "ffn_up_exps.weight"]
        ddims, dtype, _, _ = gguf.tensor_info[b + "ffn_down_exps.weight"]
        if tuple(dims) != (H, F, E) or tuple(ddims) != (F, H, E) or utype != gtype:
            raise ValueError(f"{gguf.path}: block {block} expert tensors {dims} / {ddims} ({gtype}, {utype}), "
                             f"expected ({H}, {F}, {E}) / ({F}, {H}, {E})")
        shared = b + "ffn_gate_shexp.weight" in gguf
        sF, stype, sdtype = 0, "", ""
        if shared:
            sdims, stype, _, _ = gguf.tensor_info[b + "ffn_gate_shexp.weight"]
            _, sutype, _, _ = gguf.tensor_info[b + "ffn_up_shexp.weight"]
            _, sdtype, _, _ = gguf.tensor_info[b + "ffn_down_shexp.weight"]
            if sutype != stype:
                raise ValueError(f"{gguf.path}: block {block} shared gate / up types {stype} / {sutype} differ")
            sF = int(m("expert_shared_feed_forward_length", sdims[1]))
        gated = b + "ffn_gate_inp_shexp.weight" in gguf
        # routing the layer does not model is refused, not silently dropped: a weights scale, unnormalised weights,
        # expert groups, a selection bias, gating functions other than softmax (1) and sigmoid (2) (the oracle's
        # "no scale, no groups, no selection bias", tests/moe/ref.py:12-14; model_config.py:735-737)
        gfunc = int(m("expert_gating_func", 1))
        unmodelled = {"expert_gating_func": gfunc not in (1, 2),
                      "expert_weights_scale": float(m("expert_weights_scale", 1.0)) != 1.0,
                      "expert_weights_norm": not bool(m("expert_weights_norm", True)),
                      "expert_group_count": int(m("expert_group_count", 1)) > 1,
                      "exp_probs_b": b + "exp_probs_b.bias" in gguf or b + "exp_probs_b" in gguf}
        bad = [key for key, refused in unmodelled.items() if refused]
        if bad:
            raise ValueError(f"{gguf.path}: block {block} routing not modelled by this layer: {', '.join(bad)}")
        gating = "sigmoid" if gfunc == 2 else "softmax"
        eps = float(m("attention.layer_norm_rms_epsilon", 1e-6)) if norm else 0.0
        if norm and b + "ffn_norm.weight" not in gguf:
            raise ValueError(f"{gguf.path}: block {block} has no ffn_norm")
        layer = cls(hidden=H, n_experts=E, top_k=k, expert_ffn=F, gate_type=gtype, down_type=dtype,
                    max_tokens=max_tokens, shared_ffn=sF, shared_type=stype, shared_gated=gated, gating=gating,
                    norm_eps=eps, residual=norm, shared_down_type=sdtype if sdtype != stype else "")
        try:
            for name in ("ffn_gate_inp", "ffn_gate_inp_shexp") + (("ffn_norm",) if norm else ()):
                if b + name + ".weight" in gguf:
                    t = gguf.tensor(b + name + ".weight")
                    raw = t.raw if t.qtype != "BF16" else (t.raw.astype(np.uint32) << 16).view(np.float32)
                    layer.upload(name, np.ascontiguousarray(raw, np.float32))
            for name in ("ffn_gate_exps", "ffn_up_exps", "ffn_down_exps") + (
                    ("ffn_gate_shexp", "ffn_up_shexp", "ffn_down_shexp") if shared else ()):
                layer.upload(name, gguf.tensor(b + name + ".weight").raw)
        except BaseException:
            layer.close()
            raise
        return layer

    def upload(self, name: str, data: np.ndarray) -> None:
        """A tensor's bytes (its GGUF layout, exactly its size)."""
        a = np.ascontiguousarray(data)
        _hip.check(_hip.lib().artlite_moe_layer_upload(self.handle, TENSORS[name], a.ctypes.data, a.nbytes))

    @staticmethod
    def _x(x: np.ndarray) -> tuple[np.ndarray, int]:
        a = np.ascontiguousarray(x)
        if a.dtype == np.uint16:
            return a, X_BF16
        return np.ascontiguousarray(a, np.float32), X_F32

    def stage(self, x: np.ndarray) -> None:
        """Copy x into the layer's device input (the timed runs then start from HBM)."""
        a, dt = self._x(x)
        assert a.ndim == 2 and a.shape[1] == self.H, a.shape
        _hip.check(_hip.lib().artlite_moe_layer_stage(self.handle, a.ctypes.data, dt, a.shape[0]))
        self.T = a.shape[0]

    def run(self) -> None:
        """Enqueue the forward pass of the staged tokens on the layer's stream."""
        _hip.check(_hip.lib().artlite_moe_layer_run(self.handle, self.T))

    def sync(self) -> None:
        _hip.check(_hip.lib().artlite_moe_layer_sync(self.handle))

    def output(self) -> np.ndarray:
        y = np.empty((self.T, self.H), np.float32)
        _hip.check(_hip.lib().artlite_moe_layer_output(self.handle, _hip.ptr(y, ctypes.c_float), self.T))
        return y

    def __call__(self, x: np.ndarray) -> np.ndarray:
        """y (T, H) float32 of x (synchronous)."""
        a, dt = self._x(x)
        assert a.ndim == 2 and a.shape[1] == self.H, a.shape
        y = np.empty((a.shape[0], self.H), np.float32)
        _hip.check(_hip.lib().artlite_moe_layer_forward(self.handle, a.ctypes.data, dt, a.shape[0],
                                                        _hip.ptr(y, ctypes.c_float)))
        self.T = a.shape[0]
        return y

    def tap(self, name: str) -> np.ndarray:
        """An intermediate result of the last run: logits (T, E), ids / weights (T, k), counts (E,), offsets (E + 1,),
        order / slot (T k,), h (T k, F) (sorted pairs), y_pairs (T k, H) (sorted pairs), x_norm (T, H), y_shared (T, H)
        (the shared expert's output before its gate)."""
        T, k, E = self.T, self.k, self.E
        shape, dtype = {"logits": ((T, E), np.float32), "ids": ((T, k), np.int32), "weights": ((T, k), np.float32),
                        "counts": ((E,), np.int32), "offsets": ((E + 1,), np.int32), "order": ((T * k,), np.int32),
                        "slot": ((T * k,), np.int32), "h": ((T * k, self.F), np.float32),
                        "y_pairs": ((T * k, self.H), np.float32), "x_norm": ((T, self.H), np.float32),
                        "y_shared": ((T, self.H), np.float32)}[name]
        out = np.empty(shape, dtype)
        _hip.check(_hip.lib().artlite_moe_layer_tap(self.handle, TAPS[name], out.ctypes.data, out.nbytes))
        return out

    def kernel_names(self) -> list[str]:
        buf = ctypes.create_string_buffer(1024)
        _hip.check(_hip.lib().artlite_moe_kernel_names(self.handle, self.T, buf, len(buf)))
        return buf.value.decode().split(";")


def time_layers(layers: list[MoELayer], *, warmup: int, iters: int, per_kernel: bool = True
                ) -> tuple[float, list[float], dict[str, float]]:
    """(ms per run over ``iters`` back-to-back runs cycling through ``layers`` after ``warmup``; each run's ms, from
    an event before each run of a second region; per kernel average ms, from a third timed region with an event before
    each kernel) with HIP events on the layers' stream."""
    T = layers[0].T
    hs = (ctypes.c_void_p * len(layers))(*[ly.handle.value for ly in layers])
    ms = ctypes.c_double(0)
    runs = (ctypes.c_double * iters)()
    names = layers[0].kernel_names()
    kms = (ctypes.c_double * len(names))()
    nk = ctypes.c_int32(0)
    _hip.check(_hip.lib().artlite_moe_layer_time(hs, len(layers), T, warmup, iters, ctypes.byref(ms), runs,
                                                 kms if per_kernel else None, len(names), ctypes.byref(nk)))
    return ms.value, list(runs), ({n: kms[i] for i, n in enumerate(names)} if per_kernel else {})


def hbm_copy_ms(nbytes: int, iters: int = 20) -> float:
    """ms of one plain device copy of nbytes (the HBM calibration of profile counters)."""
    ms = ctypes.c_double(0)
    _hip.check(_hip.lib().artlite_hbm_copy(nbytes, iters, ctypes.byref(ms)))
    return ms.value
