"""MI355X (gfx950) backend of the AEXRT W8A8 convolution path.

The hot path (amax, activation quantize, int8 implicit-GEMM conv with
dequant/bias/SiLU, and the fp16 Winograd / implicit-GEMM fallbacks) runs as
hand-written HIP kernels in libaexrt_hip.so behind a C ABI
(include/aexrt_hip.h); this package holds the reference's Python surface
around it (graph IR, engine compiler and ``.aexrt`` writer, session/backend,
ctypes runtime).
"""
__version__ = "0.1.0"
