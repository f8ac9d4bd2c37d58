"""MoE layer with LUT-quantised experts (the role of DeepseekV2MoE_LUT and
LUTMoEExpertWrapper in vllm_lut/moe_layer.py), on the gfx950 kernels.

_routing        softmax in fp32 -> top-k (moe_layer.py:358-376) on the GPU.
LUTMoEExpertWrapper  one expert's LUT weights; get_weight dequantises to bf16
                (moe_layer.py:105-125), forward = F.linear (:127-139).
LUTMoELayer     router -> fused LUT MoE -> + always-on shared experts
                (customized/deepseek.py:111-115), or Qwen's shared expert with
                its sigmoid gate (customized/qwen.py:99-100) through
                MoEWeights.shared_gate; shared experts LUT-quantised as extra
                slots of the stacks, or kept in dense bf16 as the reference
                keeps them (vllm_lut/moe_layer.py:186-200, 348-353) through
                MoEWeights.dense_shared, summed in the same layer call.  Router: the hand-written gate kernel
                (lutmoe_router_logits) for decode batches, torch's GEMM above.
                router_dtype=bfloat16 (default) is the reference's vLLM layer
                (vllm_lut/moe_layer.py:301-304, 358-376): bf16 gate logits, top-k
                weights cast to bf16; router_dtype=float32 is DeepSeek's MoEGate
                (modeling_deepseek.py:423-470): fp32 logits and weights, top-k
                inside the layer kernels.
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
    """Router + LUT-quantised routed experts (+ shared experts: extra always-on
    slots of the same stacks, and/or MoEWeights.dense_shared in bf16)."""

    ROUTER_KERNEL_MAX_T = 64   # decode batches: the gate kernel; larger: torch's GEMM

    def __init__(self, moe: MoEWeights, gate_weight: torch.Tensor, top_k: int,
                 renormalize: bool = False, routed_scaling_factor: float = 1.0,
                 router_dtype: torch.dtype = torch.bfloat16):
        super().__init__()
        if router_dtype not in (torch.bfloat16, torch.float32):
            raise ValueError("router_dtype must be torch.bfloat16 or torch.float32")
        self.moe = moe
        self.top_k = top_k
        self.renormalize = renormalize
        self.routed_scaling_factor = routed_scaling_factor
        self.router_dtype = router_dtype
        self.gate = nn.Parameter(gate_weight.to(torch.bfloat16).contiguous(), requires_grad=False)  # [E, H]
        self._gate_f32: Optional[torch.Tensor] = None                  # fp32 copy for large T
        self._ws: Optional[torch.Tensor] = None

    def router_logits(self, xb: torch.Tensor) -> torch.Tensor:
        """fp32 [T, E] logits of the gate; bf16-rounded values in bf16 router mode."""
        bf16 = self.router_dtype == torch.bfloat16
        if xb.shape[0] <= self.ROUTER_KERNEL_MAX_T:
            return ops.router_logits(xb, self.gate, round_bf16=bf16)
        if bf16:
            return F.linear(xb, self.gate).float()
        if self._gate_f32 is None or self._gate_f32.device != self.gate.device:
            self._gate_f32 = self.gate.detach().float()
        return F.linear(xb.float(), self._gate_f32)

    def forward(self, hidden_states: torch.Tensor) -> torch.Tensor:
        shape = hidden_states.shape
        x = hidden_states.reshape(-1, shape[-1])
        xb = (x if x.dtype == torch.bfloat16 else x.to(torch.bfloat16)).contiguous()
        logits = self.router_logits(xb)
        need = ops.moe_workspace_bytes(self.moe, xb.shape[0], self.top_k)
        if self._ws is None or self._ws.numel() < need or self._ws.device != xb.device:
            self._ws = ops.new_workspace(self.moe, xb.shape[0], self.top_k, xb.device)
        if self.router_dtype == torch.float32:
            # top-k from the logits inside the layer kernels
            out = ops.moe_forward_logits(self.moe, xb, logits, self.top_k,
                                         renormalize=self.renormalize,
                                         scaling=self.routed_scaling_factor, workspace=self._ws)
        else:
            # the reference's _routing: softmax top-k, weights cast to the logits dtype
            w, ids = ops.route_topk(logits, self.top_k, renormalize=self.renormalize,
                                    scaling=self.routed_scaling_factor)
            out = ops.moe_forward(self.moe, xb, w.to(torch.bfloat16).float(), ids, workspace=self._ws)
        return out.to(hidden_states.dtype).reshape(shape)
