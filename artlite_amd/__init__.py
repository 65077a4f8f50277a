"""artlite_amd: artlite's mixture-of-experts FFN layer over GGUF-quantized experts, native to MI355X (gfx950).

The Python API of the reference's MoE operator (``artlite.moe``: ``plan.route``, ``plan.Plan``, ``route.top_k`` /
``deal`` / ``route`` / ``item_weights``), its GGUF row dequantization (``gguf_model``) and a device-resident layer
(``moe.layer.MoELayer``), all backed by the HIP library ``libartlite_moe.so`` through ctypes. No torch.
"""

from ._hip import Error, device_count

__all__ = ["Error", "device_count"]
__version__ = "0.1.0"
