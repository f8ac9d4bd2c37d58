"""fused_lut_gemv (vllm_lut/fused_kernel.py:13-46): LUT dequantisation and the
matrix-vector product in one gfx950 kernel.

The reference compiles codebook[indices] * absmax[block] (bf16 weights, block
index clamped to the last absmax entry) followed by ``weights @ input_vec``
with torch.compile; here one kernel looks each code up, forms the same bf16
weight bf16(cb * absmax) and accumulates x * w in fp32 (lutmoe_fused_lut_gemv).
It differs from lut_gemv only in that the weights are rounded to bf16 before
the products, as the reference's dequantise-then-matmul path rounds them."""
from __future__ import annotations

import torch

from . import ops


def fused_lut_gemv(input_vec: torch.Tensor, indices: torch.Tensor, codebook: torch.Tensor,
                   absmax: torch.Tensor, block_size: int = 128) -> torch.Tensor:
    """input_vec [K] (or [T, K]) bf16; indices [M, K] uint8; codebook [256] bf16; absmax
    [num_blocks] bf16 -> [M] (or [T, M]) bf16 = bf16(cb[indices] * absmax[block]) @ input."""
    return ops.ref_gemv(input_vec, indices, codebook, absmax, block_size=block_size,
                        out_dtype=torch.bfloat16, dequantised=True)
