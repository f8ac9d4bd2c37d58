"""MoE layer with LUT-quantised experts (the role of DeepseekV2MoE_LUT and
LUTMoEExpertWrapper in vllm_lut/moe_layer.py), on the gfx950 kernels.

_routing        softmax in fp32 -> top-k (moe_layer.py:358-376) on the GPU.
LUTMoEExpertWrapper  one expert's LUT weights; get_weight dequantises to bf16
                (moe_layer.py:105-125), forward = F.linear (:127-139).
LUTMoELayer     router (bf16 gate linear, fp32 logits) -> fused LUT MoE with
                routing inside the layer kernels -> + always-on shared experts
                (customized/deepseek.py:111-115; optional sigmoid shared-expert
                gate as customized/qwen.py:99-100 is applied by the caller).
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch
import torch.nn as nn
import torch.nn.functional as F

from .formats import MoEWeights, WeightStack
from . import ops


def _routing(router_logits: torch.Tensor, top_k: int,
             renormalize: bool = False) -> Tuple[torch.Tensor, torch.Tensor]:
    """Standard softmax top-k routing: (topk_weights in the logits dtype,
    topk_indices int64), sorted descending, ties to the lower expert id."""
    w, ids = ops.route_topk(router_logits, top_k, renormalize=renormalize)
    return w.to(router_logits.dtype), ids.long()


class LUTMoEExpertWrapper(nn.Module):
    """One expert (index ``expert``) of LUT weight stacks w13 [2I, H] / w2 [H, I]."""

    def __init__(self, w13: WeightStack, w2: WeightStack, expert: int):
        super().__init__()
        self.w13, self.w2, self.expert = w13, w2, expert
        self.hidden_size = w13.cols
        self.intermediate_size = w13.rows // 2

    def get_weight(self, name: str) -> torch.Tensor:
        if name == "w13":
            return ops.dequant(self.w13, self.expert, 1)[0]
        if name == "w2":
            return ops.dequant(self.w2, self.expert, 1)[0]
        raise ValueError(f"Unknown weight name: {name}")

    def forward(self, x: torch.Tensor, name: str) -> torch.Tensor:
        st = self.w13 if name == "w13" else self.w2
        if x.dim() == 2 and x.shape[0] <= 4 and x.dtype == torch.bfloat16:
            return ops.gemv(st, x.contiguous(), self.expert)        # decode: fused LUT-GEMV
        return F.linear(x, self.get_weight(name).to(x.dtype))


class LUTMoELayer(nn.Module):
    """Router + LUT-quantised routed experts (+ shared experts as extra
    always-on slots of the same stacks)."""

    def __init__(self, moe: MoEWeights, gate_weight: torch.Tensor, top_k: int,
                 renormalize: bool = False, routed_scaling_factor: float = 1.0):
        super().__init__()
        self.moe = moe
        self.top_k = top_k
        self.renormalize = renormalize
        self.routed_scaling_factor = routed_scaling_factor
        self.gate = nn.Parameter(gate_weight, requires_grad=False)   # [E, H]
        self._gate_f32: Optional[torch.Tensor] = None                  # fp32 copy, made once
        self._ws: Optional[torch.Tensor] = None

    def forward(self, hidden_states: torch.Tensor) -> torch.Tensor:
        shape = hidden_states.shape
        x = hidden_states.reshape(-1, shape[-1])
        xb = x if x.dtype == torch.bfloat16 else x.to(torch.bfloat16)
        # fp32 router logits (MoEGate.forward, modeling_deepseek.py:423-470)
        if self._gate_f32 is None or self._gate_f32.device != self.gate.device:
            self._gate_f32 = self.gate.detach().float()
        logits = F.linear(xb.float(), self._gate_f32)
        need = ops.moe_workspace_bytes(self.moe, xb.shape[0], self.top_k)
        if self._ws is None or self._ws.numel() < need or self._ws.device != xb.device:
            self._ws = ops.new_workspace(self.moe, xb.shape[0], self.top_k, xb.device)
        out = ops.moe_forward_logits(self.moe, xb.contiguous(), logits, self.top_k,
                                     renormalize=self.renormalize,
                                     scaling=self.routed_scaling_factor, workspace=self._ws)
        return out.to(hidden_states.dtype).reshape(shape)
