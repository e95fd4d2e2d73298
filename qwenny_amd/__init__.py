"""qwenny_amd: MI355X (gfx950) quantized-weight matrix products for qwenny's Qwen3.5 stack.

W4A16 (group-128 int4, compressed-tensors pack-quantized, symmetric or with packed int4 zero points) and W8A16 (int8)
products, and the dense 16-bit products of the same call sites, in hand-written HIP behind a C ABI (include/qwenny_hip.h, libqwenny_hip.so); this package is the host-side
mirror of the reference's `Mat` / `Gemm` runtime and checkpoint formats.
"""

from .core import (SKINNY_MAX_M, Epi, Gemm, Graph, Mat, Quant, Wt, add_rmsnorm, dequant, lora_add, lora_silu, pack_dense_bf16,
                   pack_dense_int8, pack_quant, packed_sizes, row_order, sum_parts, unpack_rows, unpack_rows_bf16)

__all__ = ["SKINNY_MAX_M", "Epi", "Gemm", "Graph", "Mat", "Quant", "Wt", "add_rmsnorm", "dequant", "lora_add", "lora_silu",
           "pack_dense_bf16", "pack_dense_int8", "pack_quant", "packed_sizes", "row_order", "sum_parts", "unpack_rows",
           "unpack_rows_bf16"]
