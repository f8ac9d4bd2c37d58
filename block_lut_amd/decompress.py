"""BlockLUT decompression entry points of the reference:
decompress_blocklut (vllm_lut/quantizer.py:449-477) and the ctypes
LutDecompressor (vllm_lut/cuda/build_lut_kernel.py:78-139), both on the
gfx950 dequant kernel.  Output is bit-identical to the reference rule
bf16(f32(cb[code]) * f32(absmax[i // block_size])) (block index clamped to the
last absmax entry, quantizer.py:473-474)."""
from __future__ import annotations

import torch

from . import _native as N
from . import ops


def decompress_blocklut(indices: torch.Tensor, absmax: torch.Tensor, codebook: torch.Tensor,
                        block_size: int = 128) -> torch.Tensor:
    """[N] uint8 indices, [num_blocks] bf16 absmax, [256] bf16 codebook -> [N] bf16
    (device tensors; there is no CPU path)."""
    if not indices.is_cuda:
        raise ValueError("decompress_blocklut runs on the GPU: pass device tensors")
    idx = indices.reshape(-1).contiguous()
    am = absmax.reshape(-1).to(idx.device).contiguous()
    cb = codebook.to(idx.device).contiguous()
    n = idx.numel()
    nb = am.numel()
    if nb * block_size >= n:
        return ops.blocklut_decompress(idx, am, cb, block_size)
    # fewer absmax entries than blocks: the reference clamps the block index
    from .formats import RefStack
    st = RefStack(idx.view(1, 1, n), am.view(1, nb), cb, block_size)
    return ops.dequant(st).reshape(n)


class LutDecompressor:
    """Python wrapper of the C-ABI decompression kernel (build_lut_kernel.py:78-139)."""

    def __init__(self):
        self.lib = N.lib()

    def decompress(self, indices: torch.Tensor, absmax: torch.Tensor, codebook: torch.Tensor,
                   block_size: int = 128) -> torch.Tensor:
        assert indices.is_cuda and indices.dtype == torch.uint8
        assert absmax.is_cuda and absmax.dtype == torch.bfloat16
        assert codebook.is_cuda and codebook.dtype == torch.bfloat16
        assert codebook.shape[0] == 256
        try:
            return ops.blocklut_decompress(indices.reshape(-1).contiguous(), absmax.contiguous(),
                                           codebook.contiguous(), block_size)
        except RuntimeError as e:
            raise RuntimeError(f"HIP kernel launch failed ({e})") from e
