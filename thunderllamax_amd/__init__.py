"""thunderllamax_amd -- MI355X (gfx950) quantized-weight matmul path.

Hand-written HIP kernels behind a C ABI (``libtlx_hip.so``, declared in ``include/tlx.h``),
called from Python through ctypes with PyTorch-ROCm used for device memory and streams.
"""
__version__ = "0.1.0"
