"""The MoE layer's operator API (the reference's ``artlite.moe``): host routing and chunk plan (``plan``), the decode
routing model (``route``), the device-resident layer (``layer``)."""

COLS = 8  # the columns a plan deals its chunks to (the reference's ``operators.design.COLS``, design.py:18)
CHUNK = 192  # pairs of one expert per chunk (the reference's ``moe.expert_gemm.CHUNK`` = 3 x 64, expert_gemm.py:74-75)
