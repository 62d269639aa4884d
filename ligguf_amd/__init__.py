"""ligguf_amd -- MI355X (gfx950) decode path of LiGGUF FAST.

The product is the C-ABI shared library ``libligguf_hip.so``
(include/ligguf_hip.h).  This package holds its sources (``csrc/``), the
in-tree build (``build.py``) and a thin host-side mirror for Python callers:

* ``lib``    -- ctypes binding of every C-ABI symbol;
* ``ops``    -- per-op calls on torch device tensors, named after the
               reference's math layer (fast/lil_math.h);
* ``model``  -- host model description (synthetic or GGUF) and ``Engine``;
* ``gguf``   -- GGUF v3 reader/writer;
* ``encode`` -- weight encoders (fp32 -> GGUF blocks).
"""
from .lib import (F16, F32, Q1_0, Q1_G, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, Q8_0, Q8_K, ARCH_LLAMA, ARCH_QWEN3,  # noqa
                  LgError, row_size)
