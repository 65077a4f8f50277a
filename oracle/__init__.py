"""CPU oracle of artlite's MoE FFN path: TEST INFRASTRUCTURE, never part of the product.

A restatement, in numpy (and, for the reference's own C++ dequantizer, a build of that source into ``oracle/_ref``),
of the reference's arithmetic for the mixture-of-experts layer:

- ``np_ops``     float32 ops of the CPU references (``tests/np_ops.py``)
- ``moe_ref``    the layer oracle: routing by probability, SwiGLU, routed sum, shared expert (``tests/moe/ref.py``)
- ``host_ref``   the host routing and chunk plan of the C++ host step (``csrc/artlite/moe_host.cpp``)
- ``gguf_ref``   GGUF block fields and fp32 dequantization of Q4_0 / Q8_0 / Q4_K (``src/artlite/gguf_model.py``)
- ``tensors``    seeded random GGUF blocks (``tests/tensors.py``)
- ``layers``     the synthetic layers of the benchmark configurations
- ``ref_lib``    ctypes access to ``oracle/_ref/libartlite_ref.so`` (the reference's dequant.cpp, compiled)

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg may import this package, and only
as the checker or the timed CPU baseline. The product (``artlite_amd``) never imports it.

Parity pins (each function is checked by tests/test_oracle.py against a fixture, a known answer of the reference's
tests, the reference's compiled code, or a mathematical property; none is "parity unpinned").
"""
