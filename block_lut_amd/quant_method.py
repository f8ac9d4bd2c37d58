"""LUT quantization method: the drop-in for the reference's vLLM plugin
(vllm_lut/quant_method.py).

``LUTConfig`` / ``LUTFusedMoEMethod`` keep the reference's names, methods and
argument meaning (create_weights / process_weights_after_loading / apply) and
run the layer through liblutmoe.so.  vLLM is optional: when it is importable
the config registers itself as quantization method "lut" the way the
reference does (quant_method.py:322-331); without it the classes work on any
``torch.nn.Module`` that plays the routed-experts role.

Two weight formats:
  code_bits=8, codebook_scope="global"  REF, bit-compatible with the reference
      (uint8 codes, bf16 absmax per block_size elements, bf16[256] codebook);
  code_bits=4, codebook_scope="block"   BL4 (4-bit codes two per byte, one
      fp16[16] codebook per 64 weights along K).
"""
from __future__ import annotations

import math
import os
from typing import Any, Dict, Optional

import numpy as np
import torch

from .formats import BL4Stack, MoEWeights, RefStack
from . import ops

_CODE_TYPES = ("LUT", "BLOCKLUT", "NESTEDLUT")


class LUTConfig:
    """LUT quantization config (vllm_lut/quant_method.py:35-80)."""

    def __init__(self, code_type: str = "BLOCKLUT", lut_path: str = "", block_size: int = 128,
                 code_bits: int = 8, codebook_scope: str = "global",
                 codebook_dtype: str = "bfloat16", **kwargs):
        if code_type not in _CODE_TYPES:
            raise ValueError(f"Unsupported code_type: {code_type}. Must be one of {_CODE_TYPES}")
        if (code_bits, codebook_scope) not in ((8, "global"), (4, "block")):
            raise ValueError("supported formats: code_bits=8 with codebook_scope='global' (REF) "
                             "or code_bits=4 with codebook_scope='block' (BL4)")
        if block_size <= 0:
            raise ValueError("block_size must be positive")
        self.code_type = code_type
        self.lut_path = lut_path or kwargs.get("lut_path", "")
        self.block_size = int(block_size)
        self.code_bits = int(code_bits)
        self.codebook_scope = codebook_scope
        self.codebook_dtype = codebook_dtype

    @property
    def format(self) -> str:
        return "ref" if self.code_bits == 8 else "bl4"

    @classmethod
    def get_name(cls) -> str:
        return "lut"

    @classmethod
    def get_supported_act_dtypes(cls) -> list:
        return [torch.bfloat16, torch.float16]

    @classmethod
    def get_min_capability(cls) -> int:
        return 80

    @classmethod
    def get_config_filenames(cls) -> list:
        return []

    @classmethod
    def from_config(cls, config: Dict[str, Any]) -> "LUTConfig":
        cfg = dict(config)
        cfg.pop("quant_method", None)
        return cls(**cfg)

    def get_quant_method(self, layer, prefix: str = ""):
        if _is_routed_experts(layer):
            return LUTFusedMoEMethod(self)
        return None


def _is_routed_experts(layer) -> bool:
    try:  # vLLM present: the reference's isinstance check (quant_method.py:72-77)
        from vllm.model_executor.layers.fused_moe.routed_experts import RoutedExperts
        if isinstance(layer, RoutedExperts):
            return True
    except Exception:
        pass
    return bool(getattr(layer, "is_routed_experts", False)) or \
        type(layer).__name__ in ("RoutedExperts", "FusedMoE")


def _set_weight_attrs(param: torch.Tensor, extra: Dict[str, Any]) -> None:
    try:
        from vllm.model_executor.utils import set_weight_attrs
        set_weight_attrs(param, extra)
    except Exception:
        for k, v in (extra or {}).items():
            setattr(param, k, v)


class LUTFusedMoEMethod:
    """uint8 LUT codes + codebooks instead of bf16 expert weights
    (vllm_lut/quant_method.py:83-319)."""

    def __init__(self, quant_config: LUTConfig):
        self.quant_config = quant_config
        self._pw_moe_idx = 0

    # -------------------------------------------------------------- weights
    def create_weights(self, layer, num_experts: int, hidden_size: int,
                       intermediate_size_per_partition: int, params_dtype=None, **extra) -> None:
        """Registers the code / scale / codebook parameters on ``layer``
        (quant_method.py:117-163 for REF; the BL4 variant stores 4-bit codes
        and per-64-block fp16 codebooks)."""
        E, H, I = num_experts, hidden_size, intermediate_size_per_partition
        dev = extra.pop("device", "cuda")
        qc = self.quant_config

        def reg(name, t):
            p = torch.nn.Parameter(t, requires_grad=False)
            layer.register_parameter(name, p)
            _set_weight_attrs(p, extra)

        if qc.format == "ref":
            bs = qc.block_size
            reg("w13_weight", torch.empty(E, 2 * I, H, dtype=torch.uint8, device=dev))
            reg("w2_weight", torch.empty(E, H, I, dtype=torch.uint8, device=dev))
            reg("w13_absmax", torch.empty(E, math.ceil(2 * I * H / bs), dtype=torch.bfloat16, device=dev))
            reg("w2_absmax", torch.empty(E, math.ceil(H * I / bs), dtype=torch.bfloat16, device=dev))
            reg("_codebook", torch.zeros(256, dtype=torch.bfloat16, device=dev))
        else:
            if H % 64 or I % 64:
                raise ValueError("BL4 needs hidden and intermediate sizes divisible by 64")
            reg("w13_weight", torch.empty(E, 2 * I, H // 2, dtype=torch.uint8, device=dev))
            reg("w2_weight", torch.empty(E, H, I // 2, dtype=torch.uint8, device=dev))
            reg("w13_codebooks", torch.empty(E, 2 * I, H // 64, 16, dtype=torch.float16, device=dev))
            reg("w2_codebooks", torch.empty(E, H, I // 64, 16, dtype=torch.float16, device=dev))
        layer._lut_shape = (E, H, I)

    def process_weights_after_loading(self, layer) -> None:
        """Loads the codebook and absmax files (REF, quant_method.py:169-224) or
        converts the fp16 codebooks to the device bf16 tables (BL4), then builds
        the layer descriptor used by ``apply``."""
        if not hasattr(layer, "w13_weight"):
            return
        if getattr(layer, "_lut_moe", None) is not None:
            return
        E, H, I = layer._lut_shape
        qc = self.quant_config
        if qc.format == "ref":
            self._load_ref_files(layer)
            w13 = RefStack(layer.w13_weight.data, layer.w13_absmax.data, layer._codebook.data,
                           qc.block_size)
            w2 = RefStack(layer.w2_weight.data, layer.w2_absmax.data, layer._codebook.data,
                          qc.block_size)
        else:
            w13 = BL4Stack.from_fp16(layer.w13_weight.data, layer.w13_codebooks.data)
            w2 = BL4Stack.from_fp16(layer.w2_weight.data, layer.w2_codebooks.data)
        layer._lut_moe = MoEWeights(w13, w2, H, I, E, 0)
        layer._lut_codebook_loaded = True

    def _load_ref_files(self, layer) -> None:
        path = self.quant_config.lut_path or ""
        if path and os.path.isdir(path):
            for fname in ("blocklut_256.npy", "full256.npy"):
                f = os.path.join(path, fname)
                if os.path.exists(f):
                    cb = torch.from_numpy(np.load(f, allow_pickle=False).astype(np.float32))
                    layer._codebook.data.copy_(cb.to(torch.bfloat16))
                    break
        npz = os.path.join(path, "lut_absmax.npz") if path else ""
        if not (npz and os.path.exists(npz)):
            return
        data = np.load(npz, allow_pickle=False)
        keys = [k for k in data.files if "experts." in k and "shared_expert" not in k
                and k.endswith(".weight")]
        layer_ids = sorted({parts[i + 1] for k in keys for parts in [k.split(".")]
                            for i, p in enumerate(parts) if p == "layers"}, key=int)
        if not layer_ids:
            return
        lid = layer_ids[self._pw_moe_idx % len(layer_ids)]
        self._pw_moe_idx += 1
        for e in range(layer.w13_weight.shape[0]):
            gk = f"model.layers.{lid}.mlp.experts.{e}.gate_proj.weight"
            uk = f"model.layers.{lid}.mlp.experts.{e}.up_proj.weight"
            dk = f"model.layers.{lid}.mlp.experts.{e}.down_proj.weight"
            if gk in data.files and uk in data.files:
                a = torch.cat([torch.from_numpy(data[gk]), torch.from_numpy(data[uk])])
                layer.w13_absmax.data[e] = a.to(torch.bfloat16).to(layer.w13_absmax.device)
            if dk in data.files:
                layer.w2_absmax.data[e] = torch.from_numpy(data[dk]).to(torch.bfloat16).to(
                    layer.w2_absmax.device)

    # ---------------------------------------------------------------- forward
    def apply(self, layer, x: torch.Tensor, topk_weights: torch.Tensor, topk_ids: torch.Tensor,
              **kwargs) -> torch.Tensor:
        """out[T, H] (dtype of x) = sum_k topk_weights * FFN_{topk_ids}(x)
        (quant_method.py:230-279), fp32 accumulation on the GPU."""
        if getattr(layer, "_lut_moe", None) is None:
            self.process_weights_after_loading(layer)
        x2 = x if x.dtype == torch.bfloat16 else x.to(torch.bfloat16)
        T, k = x2.shape[0], topk_ids.shape[1]
        ws = getattr(layer, "_lut_ws", None)
        if ws is None or ws.device != x2.device or ws.numel() < ops.moe_workspace_bytes(layer._lut_moe, T, k):
            ws = layer._lut_ws = ops.new_workspace(layer._lut_moe, T, k, x2.device)
        out = ops.moe_forward(layer._lut_moe, x2.contiguous(), topk_weights, topk_ids,
                              out_dtype=torch.bfloat16, workspace=ws)
        return out if x.dtype == torch.bfloat16 else out.to(x.dtype)

    def __repr__(self) -> str:
        return f"LUTFusedMoEMethod({self.quant_config.code_type}, {self.quant_config.format})"


# Registration with vLLM when it is importable (quant_method.py:322-331).
try:  # pragma: no cover - vLLM is not part of this environment
    from vllm.model_executor.layers.quantization import (QUANTIZATION_METHODS,
                                                         _CUSTOMIZED_METHOD_TO_QUANT_CONFIG)
    if "lut" not in QUANTIZATION_METHODS:
        QUANTIZATION_METHODS.append("lut")
        _CUSTOMIZED_METHOD_TO_QUANT_CONFIG["lut"] = LUTConfig
except Exception:
    pass
