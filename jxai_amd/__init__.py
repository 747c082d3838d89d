"""jxai_amd -- MI355X-native MoE expert path (router, top-k, dispatch,
quantized gate/up/down with SwiGLU, combine) behind a C ABI (include/jxmoe.h).

The compute lives in libjxmoe.so (hand-written HIP for gfx950); this package
is the host-side mirror of the reference's interfaces plus the seeded
synthetic-input generator.
"""
from . import formats  # noqa: F401
