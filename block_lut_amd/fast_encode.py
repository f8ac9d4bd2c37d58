"""GPU REF encoder behind the reference's fast_encode interface
(vllm_lut/fast_encode.py: `encode_lut(weight, codebook_f, block_size=128)`).

bf16 weights [N] and an fp32[256] codebook -> uint8 indices [N] (nearest codebook
entry of weight / block absmax, the first entry on equal distances) and bf16 absmax
[ceil(N / block_size)] (max |weight| of each block, at least 1e-10).  The kernel is
`lutmoe_ref_encode` (csrc/encode.hip); there is no CPU path.
"""
from __future__ import annotations

from typing import Tuple

import torch

from . import ops

__all__ = ["encode_lut"]


def encode_lut(weight: torch.Tensor, codebook_f: torch.Tensor, block_size: int = 128
               ) -> Tuple[torch.Tensor, torch.Tensor]:
    """Same arguments and results as the reference's encode_lut
    (vllm_lut/fast_encode.py:172-180): the results are returned on the host, as there.
    `ops.ref_encode` returns them on the device without the synchronisation."""
    codes, absmax = ops.ref_encode(weight.reshape(-1), codebook_f, block_size)
    return codes.cpu(), absmax.cpu()
