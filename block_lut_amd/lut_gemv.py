"""lut_gemv (vllm_lut/cuda_lut_gemv.py:153-169): fused LUT-dequant + GEMV on
the reference's REF tensors, as a gfx950 kernel behind the C ABI.

Differences from the reference's launcher, by design: the bf16 codebook is
read directly (no fp32 copy allocated per call), the launch is asynchronous on
the current stream (no device synchronisation), and several input vectors
([T, K]) may be passed at once."""
from __future__ import annotations

import torch

from . import ops


def lut_gemv(input_vec: torch.Tensor, indices: torch.Tensor, codebook: torch.Tensor,
             absmax: torch.Tensor) -> torch.Tensor:
    """input_vec [K] (or [T, K]) bf16; indices [M, K] uint8; codebook [256] bf16;
    absmax [num_blocks] bf16 (128-element blocks).  Returns [M] (or [T, M]) bf16:
    y[r] = sum_c x[c] * cb[idx[r, c]] * absmax[(r*K + c) // 128]."""
    return ops.ref_gemv(input_vec, indices, codebook, absmax, block_size=128,
                        out_dtype=torch.bfloat16)
