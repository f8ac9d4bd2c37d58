"""Torch-facing operators over the C ABI (and their torch.library registrations).

Every function takes device tensors, launches on
``torch.cuda.current_stream()`` and returns without synchronising.  There is
no CPU or PyTorch fallback: a missing library raises ``LutMoeNotBuilt``.
"""
from __future__ import annotations

import ctypes
from typing import Optional, Tuple

import torch

from . import _native as N
from .formats import MoEWeights, WeightStack, _dev, _stream

_DT = {torch.bfloat16: N.DTYPE_BF16, torch.float32: N.DTYPE_F32}


def _out_code(dtype: torch.dtype) -> int:
    if dtype not in _DT:
        raise TypeError(f"output dtype must be bfloat16 or float32, got {dtype}")
    return _DT[dtype]


# ------------------------------------------------------------------ dequant

def dequant(w: WeightStack, e0: int = 0, ne: Optional[int] = None) -> torch.Tensor:
    """bf16 [ne, M, K] dequantised weights of experts e0 .. e0+ne-1."""
    ne = w.num_experts - e0 if ne is None else ne
    dev = _any_tensor(w).device
    out = torch.empty((ne, w.rows, w.cols), dtype=torch.bfloat16, device=dev)
    d = w.desc()
    N.check("lutmoe_dequant", N.lib().lutmoe_dequant(ctypes.byref(d), e0, ne, out.data_ptr(),
                                                     _stream()))
    return out


def blocklut_decompress(indices: torch.Tensor, absmax: torch.Tensor, codebook: torch.Tensor,
                        block_size: int = 128) -> torch.Tensor:
    """launch_blocklut_decompress (lut_decompress_kernel.cu:125-154): bf16 [N]."""
    _dev(indices, torch.uint8, "indices")
    _dev(absmax, torch.bfloat16, "absmax")
    _dev(codebook, torch.bfloat16, "codebook")
    if codebook.numel() != 256:
        raise ValueError("codebook must have 256 entries")
    n = indices.numel()
    if absmax.numel() < (n + block_size - 1) // block_size:
        raise ValueError("absmax shorter than ceil(N / block_size)")
    out = torch.empty(n, dtype=torch.bfloat16, device=indices.device)
    rc = N.lib().launch_blocklut_decompress(out.data_ptr(), indices.data_ptr(), absmax.data_ptr(),
                                            codebook.data_ptr(), n, block_size, _stream())
    if rc != 0:
        raise RuntimeError(f"launch_blocklut_decompress failed (code={rc})")
    return out


def unpack_4bit_(data: torch.Tensor, num_elements: int) -> torch.Tensor:
    """In place: the first num_elements/2 bytes (low-nibble section) become
    num_elements one-byte codes (lut_moe_launch_unpack_4bit)."""
    _dev(data, torch.uint8, "data")
    if data.numel() < num_elements:
        raise ValueError("buffer shorter than num_elements")
    N.lib().lut_moe_launch_unpack_4bit(data.data_ptr(), num_elements, _stream())
    N.check_last("lut_moe_launch_unpack_4bit")
    return data


def unpack_6bit(packed: torch.Tensor, num_elements: int) -> torch.Tensor:
    """6-bit tier codes (low nibble | mid 2 bits << 4) from [low | mid] sections."""
    _dev(packed, torch.uint8, "packed")
    if packed.numel() < num_elements // 2 + num_elements // 4:
        raise ValueError("packed buffer shorter than the low+mid sections")
    out = torch.empty(num_elements, dtype=torch.uint8, device=packed.device)
    N.check("lutmoe_unpack_6bit", N.lib().lutmoe_unpack_6bit(packed.data_ptr(), out.data_ptr(),
                                                             num_elements, _stream()))
    return out


def pack_bitplanes(codes: torch.Tensor) -> torch.Tensor:
    """One-byte codes -> the BLOCKLUT8 bit-plane sections [low n/2 | mid n/4 | high n/4]
    (convert_lut.py:95-110), on the device."""
    _dev(codes, torch.uint8, "codes")
    n = codes.numel()
    if n % 4:
        raise ValueError("bit-plane packing needs a multiple of 4 codes")
    out = torch.empty(n, dtype=torch.uint8, device=codes.device)
    N.check("lutmoe_pack_bitplanes", N.lib().lutmoe_pack_bitplanes(codes.data_ptr(), n, out.data_ptr(), _stream()))
    return out


def merge_bitplane_(codes: torch.Tensor, plane: torch.Tensor, shift: int) -> torch.Tensor:
    """In place: code i of ``codes`` takes the 2-bit field
    ``(plane[i // 4] >> 2 * (i % 4)) & 3`` at bits [shift, shift + 2) -- one
    BLOCKLUT8 mid (shift 4) or high (shift 6) section merged into resident
    codes, a tier upgrade that reads only the new section
    (csrc/tensor_engine/tensor_engine.cpp:504-510 read sizes)."""
    _dev(codes, torch.uint8, "codes")
    _dev(plane, torch.uint8, "plane")
    n = codes.numel()
    if n % 4 or plane.numel() < n // 4:
        raise ValueError("codes must be a multiple of 4 and the plane hold codes/4 bytes")
    if plane.device != codes.device:
        raise ValueError("codes and plane must be on the same device")
    N.check("lutmoe_merge_bitplane", N.lib().lutmoe_merge_bitplane(codes.data_ptr(), plane.data_ptr(), n,
                                                                   int(shift), _stream()))
    return codes


def blocklut_recover(indices: torch.Tensor, absmax: torch.Tensor, lut: torch.Tensor) -> torch.Tensor:
    """lut_moe_launch_blocklut_recover (tensor_recover.cu:144-159), 128-element blocks."""
    _dev(indices, torch.uint8, "indices")
    _dev(absmax, torch.bfloat16, "absmax")
    _dev(lut, torch.bfloat16, "lut")
    n = indices.numel()
    out = torch.empty(n, dtype=torch.bfloat16, device=indices.device)
    N.lib().lut_moe_launch_blocklut_recover(out.data_ptr(), indices.data_ptr(), absmax.data_ptr(),
                                            lut.data_ptr(), n, _stream())
    N.check_last("lut_moe_launch_blocklut_recover")
    return out


# --------------------------------------------------------------------- GEMV

def gemv(w: WeightStack, x: torch.Tensor, expert: int = 0,
         out_dtype: torch.dtype = torch.bfloat16, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """y [T, M] = x [T, K] . W[expert]^T (fp32 accumulation); x bf16, or fp32 (BL4 and REF
    weights); ``out`` (contiguous [T, M], its dtype bf16 or fp32) receives the result
    without an allocation."""
    squeeze = x.dim() == 1
    x2 = x.unsqueeze(0) if squeeze else x
    if x2.dtype not in (torch.bfloat16, torch.float32):
        raise TypeError(f"x must be bf16 or fp32, got {x2.dtype}")
    _dev(x2, x2.dtype, "x")
    if x2.shape[1] != w.cols:
        raise ValueError(f"x has {x2.shape[1]} features, weights expect {w.cols}")
    if out is None:
        y = torch.empty((x2.shape[0], w.rows), dtype=out_dtype, device=x2.device)
    else:
        y = _dev(out, out.dtype, "out").view(x2.shape[0], w.rows)
        out_dtype = out.dtype
    d = w.desc()
    N.check("lutmoe_gemv", N.lib().lutmoe_gemv_ex(ctypes.byref(d), expert, x2.data_ptr(), _out_code(x2.dtype),
                                                  x2.shape[0], y.data_ptr(), _out_code(out_dtype), _stream()))
    return y[0] if squeeze else y


def ref_gemv(x: torch.Tensor, indices: torch.Tensor, codebook: torch.Tensor, absmax: torch.Tensor,
             block_size: int = 128, out_dtype: torch.dtype = torch.bfloat16,
             dequantised: bool = False) -> torch.Tensor:
    """REF LUT-GEMV on the reference's raw tensors: lut_gemv's (x * cb) * absmax products
    (cuda_lut_gemv.py:153-169), or with ``dequantised`` the bf16(cb * absmax) weights of
    fused_lut_gemv (fused_kernel.py:13-46)."""
    squeeze = x.dim() == 1
    x2 = x.unsqueeze(0) if squeeze else x
    _dev(x2, torch.bfloat16, "input")
    _dev(indices, torch.uint8, "indices")
    _dev(codebook, torch.bfloat16, "codebook")
    _dev(absmax, torch.bfloat16, "absmax")
    if indices.dim() != 2 or indices.shape[1] != x2.shape[1]:
        raise ValueError("indices must be [M, K] with K = input features")
    if codebook.numel() != 256:
        raise ValueError("codebook must have 256 entries")
    M, K = indices.shape
    y = torch.empty((x2.shape[0], M), dtype=out_dtype, device=x2.device)
    fn = "lutmoe_fused_lut_gemv" if dequantised else "lutmoe_ref_gemv"
    N.check(fn, getattr(N.lib(), fn)(x2.data_ptr(), indices.data_ptr(), codebook.data_ptr(),
                                     absmax.data_ptr(), y.data_ptr(), M, K, x2.shape[0],
                                     absmax.numel(), block_size, _out_code(out_dtype), _stream()))
    return y[0] if squeeze else y


def router_logits(x: torch.Tensor, gate: torch.Tensor, round_bf16: bool = False,
                  out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Router gate logits [T, E] fp32 = x [T, H] . gate [E, H]^T (bf16 inputs, fp32
    accumulation; ``round_bf16`` rounds each logit to bf16 as a bf16 gate linear does)."""
    _dev(x, torch.bfloat16, "x")
    _dev(gate, torch.bfloat16, "gate")
    T, H = x.shape
    E = gate.shape[0]
    if gate.shape[1] != H:
        raise ValueError("gate must be [E, H]")
    lg = torch.empty((T, E), dtype=torch.float32, device=x.device) if out is None else \
        _dev(out, torch.float32, "out")
    N.check("lutmoe_router_logits",
            N.lib().lutmoe_router_logits(x.data_ptr(), gate.data_ptr(), T, H, E, lg.data_ptr(),
                                         int(bool(round_bf16)), _stream()))
    return lg


# ---------------------------------------------------------------- routing

def route_topk(logits: torch.Tensor, top_k: int, renormalize: bool = False,
               scaling: float = 1.0, out_w: Optional[torch.Tensor] = None,
               out_ids: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """softmax(fp32) -> top-k (sorted, ties to the lower id); weights fp32 [T,k], ids int32."""
    lg = logits if logits.dtype == torch.float32 else logits.float()
    lg = _dev(lg.contiguous(), torch.float32, "logits")
    T, E = lg.shape
    w = torch.empty((T, top_k), dtype=torch.float32, device=lg.device) if out_w is None else \
        _dev(out_w, torch.float32, "out_w")
    ids = torch.empty((T, top_k), dtype=torch.int32, device=lg.device) if out_ids is None else \
        _dev(out_ids, torch.int32, "out_ids")
    if tuple(w.shape) != (T, top_k) or tuple(ids.shape) != (T, top_k):
        raise ValueError("route_topk outputs must be [T, top_k]")
    N.check("lutmoe_route_topk",
            N.lib().lutmoe_route_topk(lg.data_ptr(), T, E, top_k, int(bool(renormalize)),
                                      float(scaling), w.data_ptr(), ids.data_ptr(), _stream()))
    return w, ids


def permute(topk_ids: torch.Tensor, num_experts: int):
    """Expert-major pair permutation: (offsets [E+1], perm [T*k], inv [T*k], active [E+1])."""
    ids = _dev(topk_ids.to(torch.int32).contiguous(), torch.int32, "topk_ids")
    T, k = ids.shape
    dev = ids.device
    offsets = torch.empty(num_experts + 1, dtype=torch.int32, device=dev)
    perm = torch.empty(T * k, dtype=torch.int32, device=dev)
    inv = torch.empty(T * k, dtype=torch.int32, device=dev)
    active = torch.empty(num_experts + 1, dtype=torch.int32, device=dev)
    N.check("lutmoe_permute",
            N.lib().lutmoe_permute(ids.data_ptr(), T, k, num_experts, offsets.data_ptr(),
                                   perm.data_ptr(), inv.data_ptr(), active.data_ptr(), _stream()))
    return offsets, perm, inv, active


# --------------------------------------------------------------- MoE layer

PATH_AUTO, PATH_GEMV, PATH_MFMA = 0, 1, 2


def moe_workspace_bytes(moe: MoEWeights, T: int, k: int) -> int:
    d = moe.desc()
    return int(N.lib().lutmoe_moe_workspace_size(ctypes.byref(d), T, k))


def new_workspace(moe: MoEWeights, T: int, k: int, device) -> torch.Tensor:
    """A workspace for the MoE layer at up to T tokens (zero-filled for
    determinism; no kernel needs it zeroed).  Reuse it across calls; do not
    share it between calls that overlap in time."""
    return torch.zeros(max(moe_workspace_bytes(moe, T, k), 256), dtype=torch.uint8, device=device)


def moe_forward(moe: MoEWeights, x: torch.Tensor, topk_weights: torch.Tensor,
                topk_ids: torch.Tensor, out: Optional[torch.Tensor] = None,
                out_dtype: torch.dtype = torch.bfloat16, path: int = PATH_AUTO,
                workspace: Optional[torch.Tensor] = None, stages: int = N.STAGE_ALL) -> torch.Tensor:
    """Fused LUT MoE layer: out[T, H] = sum_k w * FFN_{ids}(x) + shared experts."""
    _dev(x, torch.bfloat16, "x")
    T, H = x.shape
    if H != moe.hidden:
        raise ValueError(f"x has {H} features, layer expects {moe.hidden}")
    w = topk_weights if topk_weights.dtype == torch.float32 else topk_weights.float()
    w = _dev(w.contiguous(), torch.float32, "topk_weights")
    ids = topk_ids if topk_ids.dtype == torch.int32 else topk_ids.to(torch.int32)
    ids = _dev(ids.contiguous(), torch.int32, "topk_ids")
    k = ids.shape[1]
    if out is None:
        out = torch.empty((T, H), dtype=out_dtype, device=x.device)
    else:
        _dev(out, out.dtype, "out")
        out_dtype = out.dtype
    need = moe_workspace_bytes(moe, T, k)
    if workspace is None or workspace.numel() < need:
        workspace = new_workspace(moe, T, k, x.device)
    d = moe.desc()
    N.check("lutmoe_moe_forward",
            N.lib().lutmoe_moe_forward_stages(ctypes.byref(d), x.data_ptr(), w.data_ptr(),
                                              ids.data_ptr(), T, k, out.data_ptr(),
                                              _out_code(out_dtype), workspace.data_ptr(),
                                              workspace.numel(), path, stages, _stream()))
    return out


def moe_forward_logits(moe: MoEWeights, x: torch.Tensor, logits: torch.Tensor, top_k: int,
                       renormalize: bool = False, scaling: float = 1.0,
                       out: Optional[torch.Tensor] = None, out_dtype: torch.dtype = torch.bfloat16,
                       path: int = PATH_AUTO, workspace: Optional[torch.Tensor] = None,
                       stages: int = N.STAGE_ALL) -> torch.Tensor:
    """MoE block forward from router logits: softmax(fp32) -> top-k -> layer."""
    _dev(x, torch.bfloat16, "x")
    T, H = x.shape
    if H != moe.hidden:
        raise ValueError(f"x has {H} features, layer expects {moe.hidden}")
    lg = logits if logits.dtype == torch.float32 else logits.float()
    lg = _dev(lg.contiguous(), torch.float32, "logits")
    if tuple(lg.shape) != (T, moe.num_routed):
        raise ValueError(f"logits must be [T, {moe.num_routed}]")
    if out is None:
        out = torch.empty((T, H), dtype=out_dtype, device=x.device)
    else:
        _dev(out, out.dtype, "out")
        out_dtype = out.dtype
    need = moe_workspace_bytes(moe, T, top_k)
    if workspace is None or workspace.numel() < need:
        workspace = new_workspace(moe, T, top_k, x.device)
    d = moe.desc()
    N.check("lutmoe_moe_forward_logits",
            N.lib().lutmoe_moe_forward_logits(ctypes.byref(d), x.data_ptr(), lg.data_ptr(), T, top_k,
                                              int(bool(renormalize)), float(scaling), out.data_ptr(),
                                              _out_code(out_dtype), workspace.data_ptr(),
                                              workspace.numel(), path, stages, _stream()))
    return out


# ----------------------------------------------------------------- encoders

def bl4_encode(weight: torch.Tensor, n_iter: int = 50) -> Tuple[torch.Tensor, torch.Tensor]:
    """Per-64-block k-means BL4 encoder on the GPU.  weight fp32 [..., K], K % 64 == 0.
    Returns (codes uint8 [..., K/2], fp16 tables [..., K/64, 16])."""
    _dev(weight, torch.float32, "weight")
    K = weight.shape[-1]
    if K % 64:
        raise ValueError("K must be a multiple of 64")
    lead = tuple(weight.shape[:-1])
    nb = weight.numel() // 64
    codes = torch.empty(lead + (K // 2,), dtype=torch.uint8, device=weight.device)
    tables = torch.empty(lead + (K // 64, 16), dtype=torch.float16, device=weight.device)
    N.check("lutmoe_bl4_encode", N.lib().lutmoe_bl4_encode(weight.data_ptr(), nb, n_iter,
                                                           codes.data_ptr(), tables.data_ptr(),
                                                           _stream()))
    return codes, tables


def ref_encode(weight: torch.Tensor, codebook: torch.Tensor, block_size: int = 128
               ) -> Tuple[torch.Tensor, torch.Tensor]:
    """REF encoder on the GPU (the reference's encode_lut, vllm_lut/fast_encode.py:22-72):
    bf16 weights (any shape, flattened) and an fp32[256] codebook -> (uint8 codes [N],
    bf16 absmax [ceil(N / block_size)])."""
    _dev(weight, torch.bfloat16, "weight")
    _dev(codebook, torch.float32, "codebook")
    if codebook.numel() != 256:
        raise ValueError("codebook must hold 256 entries")
    if block_size <= 0:
        raise ValueError("block_size must be positive")
    w = weight.contiguous().reshape(-1)
    cb = codebook.contiguous()
    n = w.numel()
    codes = torch.empty(n, dtype=torch.uint8, device=w.device)
    absmax = torch.empty(-(-n // block_size), dtype=torch.bfloat16, device=w.device)
    N.check("lutmoe_ref_encode", N.lib().lutmoe_ref_encode(w.data_ptr(), cb.data_ptr(), n, block_size,
                                                           codes.data_ptr(), absmax.data_ptr(), _stream()))
    return codes, absmax


def _any_tensor(w: WeightStack) -> torch.Tensor:
    for name in ("codes", "tables", "absmax"):
        t = getattr(w, name, None)
        if isinstance(t, torch.Tensor):
            return t
    return w.codes[0]  # NestedStack


# ------------------------------------------------------- torch.library ops

_lib_def = torch.library.Library("lutmoe", "DEF")
_lib_def.define("lut_gemv(Tensor input, Tensor indices, Tensor codebook, Tensor absmax) -> Tensor")
_lib_def.define("blocklut_decompress(Tensor indices, Tensor absmax, Tensor codebook, "
                "int block_size=128) -> Tensor")


@torch.library.impl(_lib_def, "lut_gemv", "CUDA")
def _lut_gemv_impl(input, indices, codebook, absmax):
    return ref_gemv(input, indices, codebook, absmax)


@torch.library.register_fake("lutmoe::lut_gemv")
def _lut_gemv_fake(input, indices, codebook, absmax):
    shape = (indices.shape[0],) if input.dim() == 1 else (input.shape[0], indices.shape[0])
    return input.new_empty(shape, dtype=torch.bfloat16)


@torch.library.impl(_lib_def, "blocklut_decompress", "CUDA")
def _decompress_impl(indices, absmax, codebook, block_size=128):
    return blocklut_decompress(indices, absmax, codebook, block_size)


@torch.library.register_fake("lutmoe::blocklut_decompress")
def _decompress_fake(indices, absmax, codebook, block_size=128):
    return indices.new_empty((indices.numel(),), dtype=torch.bfloat16)
