"""metalops_amd -- MI355X (gfx950) native GGML block_q4_0 INT4 matmul path.

Drop-in for metalcore's q4_0 API (reference ``metalcore/quantization.py:288-454``,
re-exported by ``metalcore/__init__.py:39,182-184``): the same function names,
argument order, tensor layout ``[K/32, N, 18]`` uint8 and error behaviour, backed
by hand-written HIP kernels through the C ABI in ``include/mcq4.h``.
"""
from .quantization import (
    BLOCK_Q4_0_SIZE,
    QK4_0,
    dequantize_ggml_q4_0,
    matmul_ggml_q4_0,
    quantize_ggml_q4_0,
    quantize_ggml_q4_0_llama,
)

__version__ = "1.0.0"

__all__ = [
    "QK4_0",
    "BLOCK_Q4_0_SIZE",
    "quantize_ggml_q4_0",
    "quantize_ggml_q4_0_llama",
    "dequantize_ggml_q4_0",
    "matmul_ggml_q4_0",
]
