"""fused_lut_moe (vllm_lut/fast_moe.py:30-80): the whole routed-expert MoE in
one call on the reference's REF tensors (uint8 codes, bf16 absmax, bf16[256]
codebook).  Decode (few tokens) runs the grouped LUT-GEMV kernels, prefill
the grouped MFMA LUT-GEMM; no per-expert host loop and no host sync."""
from __future__ import annotations

import torch

from .formats import MoEWeights, RefStack
from . import ops


def fused_lut_moe(x: torch.Tensor, topk_ids: torch.Tensor, topk_weights: torch.Tensor,
                  w13_weight: torch.Tensor, w13_absmax: torch.Tensor, w2_weight: torch.Tensor,
                  w2_absmax: torch.Tensor, codebook: torch.Tensor,
                  block_size: int = 128) -> torch.Tensor:
    """x [T, H] or [H]; topk_ids / topk_weights [T, k]; w13_weight u8 [E, 2I, H];
    w2_weight u8 [E, H, I]; absmax bf16 [E, nb]; codebook bf16 [256].
    Returns [T, H] in the dtype of x."""
    x2 = x.unsqueeze(0) if x.dim() == 1 else x
    E, two_i, H = w13_weight.shape
    cb = codebook.to(x2.device)
    moe = MoEWeights(RefStack(w13_weight, w13_absmax, cb, block_size),
                     RefStack(w2_weight, w2_absmax, cb, block_size), H, two_i // 2, E, 0)
    xb = x2 if x2.dtype == torch.bfloat16 else x2.to(torch.bfloat16)
    out = ops.moe_forward(moe, xb.contiguous(), topk_weights, topk_ids, out_dtype=torch.bfloat16)
    return out if x2.dtype == torch.bfloat16 else out.to(x2.dtype)


# torch.library op, so that torch.compile graphs can hold the fused layer (the
# fake kernel gives the output's shape and dtype without running anything)
ops._lib_def.define("fused_lut_moe(Tensor x, Tensor topk_ids, Tensor topk_weights, Tensor w13_weight, "
                    "Tensor w13_absmax, Tensor w2_weight, Tensor w2_absmax, Tensor codebook, "
                    "int block_size=128) -> Tensor")


@torch.library.impl(ops._lib_def, "fused_lut_moe", "CUDA")
def _fused_lut_moe_impl(x, topk_ids, topk_weights, w13_weight, w13_absmax, w2_weight, w2_absmax, codebook,
                        block_size=128):
    return fused_lut_moe(x, topk_ids, topk_weights, w13_weight, w13_absmax, w2_weight, w2_absmax, codebook,
                         block_size)


@torch.library.register_fake("lutmoe::fused_lut_moe")
def _fused_lut_moe_fake(x, topk_ids, topk_weights, w13_weight, w13_absmax, w2_weight, w2_absmax, codebook,
                        block_size=128):
    shape = (1, x.shape[0]) if x.dim() == 1 else tuple(x.shape)
    return x.new_empty(shape)
