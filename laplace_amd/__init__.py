"""laplace_amd - MI355X (gfx950) GGUF quantized-matmul back-end for Laplace.

The product is the C-ABI library ``liblaplace_hip.so`` (include/laplace_hip.h)
built from ``csrc/``; this package is its Python host mirror of the
reference's matmul front-end (src/matmul.h). Importing it does not touch the
GPU; the first call loads the library and fails loudly if it is not built.
"""
from .matmul import (GGMLType, Tensor, bytes_per_block, dequantize, elements_per_block, fused_moe_gemm_idx,
                     fused_moe_gemm_multi, matmul_gemm_batch, matmul_lm_head,
                     matmul_register_weights, matmul_row, matmul_rows, quantize_act, row_bytes)
from .moe import moe_ffn, moe_grouped, moe_workspace_bytes
from .gguf import GGUFFile, write_gguf

__all__ = ["GGMLType", "Tensor", "bytes_per_block", "dequantize", "elements_per_block", "fused_moe_gemm_idx",
           "fused_moe_gemm_multi", "matmul_gemm_batch", "matmul_lm_head",
           "matmul_register_weights", "matmul_row", "matmul_rows", "quantize_act", "row_bytes",
           "moe_ffn", "moe_grouped", "moe_workspace_bytes", "GGUFFile", "write_gguf"]
