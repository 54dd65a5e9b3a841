"""metalops_amd -- MI355X (gfx950) native INT4 matmul paths.

Drop-in for metalcore's quantized-matmul API (reference
``metalcore/quantization.py``, re-exported by ``metalcore/__init__.py:38-39``):
the GGML block_q4_0 path (``quantization.py:288-454``, tensor layout
``[K/32, N, 18]`` uint8) and the per-group INT4 path (``quantization.py:26-239``
and ``Int4Linear`` :457-613, layout ``[K/2, N]`` uint8 + scales/zeros), with the
same function names, argument order and error behaviour, backed by
hand-written HIP kernels through the C ABI in ``include/mcq4.h``.
"""
from .quantization import (
    BLOCK_Q4_0_SIZE,
    QK4_0,
    dequantize_ggml_q4_0,
    matmul_ggml_q4_0,
    matmul_ggml_q4_0_grouped,
    quantize_ggml_q4_0,
    quantize_ggml_q4_0_llama,
)
from .int4 import (
    Int4Linear,
    dequantize_int4,
    fused_rmsnorm_linear_int4,
    matmul_int4,
    matmul_int4_gelu,
    matmul_int4_silu,
    matmul_int8,
    quantize_int4,
    quantize_to_int4,
)

__version__ = "1.1.0"

__all__ = [
    "QK4_0",
    "BLOCK_Q4_0_SIZE",
    "quantize_ggml_q4_0",
    "quantize_ggml_q4_0_llama",
    "dequantize_ggml_q4_0",
    "matmul_ggml_q4_0",
    "matmul_ggml_q4_0_grouped",
    "quantize_int4",
    "dequantize_int4",
    "matmul_int4",
    "matmul_int4_silu",
    "matmul_int4_gelu",
    "fused_rmsnorm_linear_int4",
    "quantize_to_int4",
    "matmul_int8",
    "Int4Linear",
]
