"""CPU baseline (test/bench infrastructure, not product): the reference's CPU
dequant + matmul path restated with torch on the host.

Per routed expert: dequantise to bf16 with a gather through the codebook
(decompress_blocklut, vllm_lut/quantizer.py:449-477; for BL4 the gather is
per 64-weight block, for a NestedLUT tier per block into its 2^b-entry
table), then F.linear in bf16 over every token of the batch, as the
reference's multi-token branch does (vllm_lut/quant_method.py:261-277:
gate_up = F.linear(x, W13); act = silu(gate) * up; F.linear(act, W2);
out[m] += expert_out[m] * w for the tokens m routed to the expert).  A single
linear (switch-base-8 shape) is the dequantised weights, widened to fp32,
through F.linear with fp32 activations.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F


def bl4_dequant_torch(codes: torch.Tensor, tables_bf16: torch.Tensor) -> torch.Tensor:
    """codes uint8 [M, K/2], tables bf16 [M, K/64, 16] -> bf16 [M, K]."""
    M, Kh = codes.shape
    K = 2 * Kh
    lo = (codes & 0x0F).long()
    hi = (codes >> 4).long()
    idx = torch.stack([lo, hi], dim=-1).reshape(M, K // 64, 64)
    return torch.gather(tables_bf16, 2, idx).reshape(M, K)


def moe_layer_step(x: torch.Tensor, topk_ids: torch.Tensor, topk_w: torch.Tensor, experts13,
                   experts2) -> torch.Tensor:
    """One MoE layer on the CPU.  experts13/experts2: dict e -> (codes, tables_bf16)."""
    T, H = x.shape
    out = torch.zeros(T, H, dtype=x.dtype)
    for e in torch.unique(topk_ids).tolist():
        W13 = bl4_dequant_torch(*experts13[e])
        W2 = bl4_dequant_torch(*experts2[e])
        I = W13.shape[0] // 2
        gu = F.linear(x, W13)
        act = F.silu(gu[:, :I]) * gu[:, I:]
        y = F.linear(act, W2)
        for k in range(topk_ids.shape[1]):
            m = topk_ids[:, k] == e
            if m.any():
                out[m] += y[m] * topk_w[m, k].unsqueeze(-1).to(y.dtype)
    return out


def table_dequant_torch(codes: torch.Tensor, tables_bf16: torch.Tensor) -> torch.Tensor:
    """One code per weight, uint8 [M, K] (values < 2^b), tables bf16 [M, K/64, 2^b]
    (a NestedLUT tier-b expert with its codes unpacked) -> bf16 [M, K]."""
    M, K = codes.shape
    idx = codes.long().reshape(M, K // 64, 64)
    return torch.gather(tables_bf16, 2, idx).reshape(M, K)


def linear_fp32(x: torch.Tensor, codes: torch.Tensor, tables_bf16: torch.Tensor) -> torch.Tensor:
    """Single BL4 linear: dequantise, widen to fp32, F.linear with fp32 x [T, K]."""
    return F.linear(x, bl4_dequant_torch(codes, tables_bf16).float())


def expert_all_tokens(x: torch.Tensor, W13: torch.Tensor, W2: torch.Tensor) -> torch.Tensor:
    """The reference's multi-token expert step: both projections over all T tokens (its
    rows are selected afterwards), bf16."""
    I = W13.shape[0] // 2
    gu = F.linear(x, W13)
    return F.linear(F.silu(gu[:, :I]) * gu[:, I:], W2)
