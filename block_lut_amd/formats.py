"""Device-resident LUT weight stacks and their C-ABI descriptors.

REF  (the reference's format, vllm_lut/quant_method.py:117-163):
     codes uint8 [E, M, K], absmax bf16 [E, nb] (nb = ceil(M*K/block_size)),
     codebook bf16 [256], or [E, 256] when experts sit at different tiers
     (each row the table of its expert's tier).
BL4  (4-bit, per-64-block codebooks): codes uint8 [E, M, K/2] (even element in
     the low nibble), tables bf16 [E, M, K/64, 16] holding the dequantised
     entries bf16(fp16 codebook) -- the fp16 codebooks are the wire format,
     converted once by ``BL4Stack.from_fp16``.
NL   (NestedLUT 2/3/4-bit tiers): per expert, bit-plane sections
     [p01 | p2 | p3] (a tier-b expert keeps the first 2, 3 or all of them) and
     a bf16 table [M, K/64, 2^b].
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import List, Optional

import torch

from . import _native as N


def _dev(t: torch.Tensor, dtype: torch.dtype, name: str) -> torch.Tensor:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if not t.is_cuda:
        raise ValueError(f"{name} must be a device (cuda/HIP) tensor")
    if t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    return t


class WeightStack:
    format: int
    num_experts: int
    rows: int
    cols: int

    def desc(self) -> N.lutmoe_weights:
        raise NotImplementedError

    def hbm_bytes_per_expert(self) -> int:
        raise NotImplementedError


class RefStack(WeightStack):
    """The reference's uint8 + bf16 absmax + bf16[256] codebook stack.  ``codebook`` is
    one bf16[256] table for all experts, or [E, 256]: one per expert (tiered experts,
    csrc/tensor_engine/tensor_engine.hpp:287-291)."""

    format = N.FMT_REF

    def __init__(self, codes: torch.Tensor, absmax: torch.Tensor, codebook: torch.Tensor,
                 block_size: int = 128):
        if codes.dim() == 2:
            codes = codes.unsqueeze(0)
        if absmax.dim() == 1:
            absmax = absmax.unsqueeze(0)
        self.codes = _dev(codes, torch.uint8, "codes")
        self.absmax = _dev(absmax, torch.bfloat16, "absmax")
        self.codebook = _dev(codebook, torch.bfloat16, "codebook")
        self.num_experts, self.rows, self.cols = self.codes.shape
        if self.codebook.dim() == 2 and tuple(self.codebook.shape) == (self.num_experts, 256):
            self.codebook_stride = 256
        elif self.codebook.numel() == 256:
            self.codebook_stride = 0
        else:
            raise ValueError("REF codebook must be [256] or [num_experts, 256]")
        self.block_size = int(block_size)
        if self.absmax.shape[0] != self.num_experts:
            raise ValueError("absmax must have one row per expert")
        if self.absmax.shape[1] < 1:
            raise ValueError("absmax needs at least one block per expert")
        # fewer entries than ceil(M*K/block_size) is legal: block indices are
        # clamped to the last entry, as decompress_blocklut does
        # (vllm_lut/quantizer.py:473-474)
        self.full_absmax = self.absmax.shape[1] >= math.ceil(self.rows * self.cols / self.block_size)

    def desc(self) -> N.lutmoe_weights:
        d = N.lutmoe_weights()
        d.format = N.FMT_REF
        d.num_experts, d.rows, d.cols = self.num_experts, self.rows, self.cols
        d.codes = self.codes.data_ptr()
        d.tables = self.absmax.data_ptr()
        d.codebook = self.codebook.data_ptr()
        d.tier_bits = None
        d.absmax_per_expert = self.absmax.shape[1]
        d.block_size = self.block_size
        d.codebook_stride = self.codebook_stride
        return d

    def hbm_bytes_per_expert(self) -> int:
        return self.rows * self.cols + 2 * self.absmax.shape[1]


class BL4Stack(WeightStack):
    """4-bit codes + per-64-block bf16 tables."""

    format = N.FMT_BL4

    def __init__(self, codes: torch.Tensor, tables_bf16: torch.Tensor):
        if codes.dim() == 2:
            codes = codes.unsqueeze(0)
        if tables_bf16.dim() == 3:
            tables_bf16 = tables_bf16.unsqueeze(0)
        self.codes = _dev(codes, torch.uint8, "codes")
        self.tables = _dev(tables_bf16, torch.bfloat16, "tables")
        E, M, Kh = self.codes.shape
        K = 2 * Kh
        if K % 64:
            raise ValueError("BL4 needs K % 64 == 0")
        if tuple(self.tables.shape) != (E, M, K // 64, 16):
            raise ValueError(f"tables shape {tuple(self.tables.shape)} != {(E, M, K // 64, 16)}")
        self.num_experts, self.rows, self.cols = E, M, K

    @classmethod
    def from_fp16(cls, codes: torch.Tensor, tables_f16: torch.Tensor) -> "BL4Stack":
        """Wire format (fp16 codebooks) -> device format (bf16 dequantised entries)."""
        t = _dev(tables_f16, torch.float16, "tables_f16")
        out = torch.empty(t.shape, dtype=torch.bfloat16, device=t.device)
        N.check("lutmoe_bl4_tables_from_f16",
                N.lib().lutmoe_bl4_tables_from_f16(t.data_ptr(), out.data_ptr(), t.numel(),
                                                   _stream()))
        return cls(codes, out)

    def desc(self) -> N.lutmoe_weights:
        d = N.lutmoe_weights()
        d.format = N.FMT_BL4
        d.num_experts, d.rows, d.cols = self.num_experts, self.rows, self.cols
        d.codes = self.codes.data_ptr()
        d.tables = self.tables.data_ptr()
        d.codebook = None
        d.tier_bits = None
        d.absmax_per_expert = 0
        d.block_size = 64
        return d

    def hbm_bytes_per_expert(self) -> int:
        return self.rows * self.cols // 2 + self.rows * (self.cols // 64) * 32


@dataclass
class NestedExpert:
    bits: int
    planes: torch.Tensor     # uint8 [M*K/4 + (bits>=3)*M*K/8 + (bits>=4)*M*K/8]
    table: torch.Tensor      # bf16 [M, K/64, 2^bits]


class NestedStack(WeightStack):
    """Per-expert NestedLUT tiers (2/3/4 bits).

    The experts arrive as stored: bit-plane sections, a tier's prefix of
    [p01 | p2 | p3].  On construction each expert's planes are regrouped on
    the device (lutmoe_nested_group_planes: the planes of every 32 weights
    together, M*K*b/8 bytes), the layout every kernel reads.  keep_planes=False
    drops the stack's references to the plane tensors afterwards."""

    format = N.FMT_NESTED

    def __init__(self, experts: List[NestedExpert], rows: int, cols: int, keep_planes: bool = True):
        if cols % 64:
            raise ValueError("NestedLUT needs K % 64 == 0")
        self.experts = experts
        self.num_experts, self.rows, self.cols = len(experts), rows, cols
        n = rows * cols
        for i, e in enumerate(experts):
            if e.bits not in (2, 3, 4):
                raise ValueError(f"expert {i}: tier bits must be 2, 3 or 4")
            need = n // 4 + (n // 8 if e.bits >= 3 else 0) + (n // 8 if e.bits >= 4 else 0)
            _dev(e.planes, torch.uint8, "planes")
            _dev(e.table, torch.bfloat16, "table")
            if e.planes.numel() != need:
                raise ValueError(f"expert {i}: planes hold {e.planes.numel()} bytes, need {need}")
            if tuple(e.table.shape) != (rows, cols // 64, 1 << e.bits):
                raise ValueError(f"expert {i}: table shape {tuple(e.table.shape)}")
        dev = experts[0].planes.device
        stream = torch.cuda.current_stream(dev).cuda_stream
        self.codes = []
        for e in experts:
            g = torch.empty(n * e.bits // 8, dtype=torch.uint8, device=dev)
            N.check("lutmoe_nested_group_planes",
                    N.lib().lutmoe_nested_group_planes(e.planes.data_ptr(), e.bits, n, g.data_ptr(), stream))
            self.codes.append(g)
        if not keep_planes:
            self.experts = [NestedExpert(e.bits, None, e.table) for e in experts]
        self._code_ptrs = torch.tensor([g.data_ptr() for g in self.codes], dtype=torch.int64,
                                       device=dev)
        self._table_ptrs = torch.tensor([e.table.data_ptr() for e in experts], dtype=torch.int64,
                                        device=dev)
        self._bits = torch.tensor([e.bits for e in experts], dtype=torch.int8, device=dev)

    def desc(self) -> N.lutmoe_weights:
        d = N.lutmoe_weights()
        d.format = N.FMT_NESTED
        d.num_experts, d.rows, d.cols = self.num_experts, self.rows, self.cols
        d.codes = self._code_ptrs.data_ptr()
        d.tables = self._table_ptrs.data_ptr()
        d.codebook = None
        d.tier_bits = self._bits.data_ptr()
        d.absmax_per_expert = 0
        d.block_size = 64
        return d

    def hbm_bytes_expert(self, e: int) -> int:
        b = self.experts[e].bits
        n = self.rows * self.cols
        return n * b // 8 + (n // 64) * (1 << b) * 2


@dataclass
class MoEWeights:
    """Routed experts 0..E-1 followed by num_shared always-on expert slots.

    A shared expert with intermediate size m*I takes m slots (``split_shared_bl4`` /
    ``split_shared_ref`` cut its matrices).  Shared slots weigh 1 (DeepSeek's shared
    experts, customized/deepseek.py:111-115) or, with ``shared_gate`` (bf16 [H], the
    weight of Qwen's shared_expert_gate Linear(H, 1)), sigmoid(x . shared_gate) per token
    (customized/qwen.py:42-43, 99-100).

    ``dense_shared`` = (w13 bf16 [2*Is, H], w2 bf16 [H, Is]): a shared expert kept in dense
    bf16, as the reference keeps a model's shared experts (bf16 linears beside the LUT
    experts, vllm_lut/moe_layer.py:186-200, 348-353; customized/qwen.py:40-43, 96-100):
    every token adds its MLP output, weighted by 1 or by ``shared_gate``'s sigmoid."""

    w13: WeightStack
    w2: WeightStack
    hidden: int
    inter: int
    num_routed: int
    num_shared: int = 0
    shared_gate: Optional[torch.Tensor] = None
    dense_shared: Optional[tuple] = None
    _desc: Optional[N.lutmoe_moe_desc] = field(default=None, repr=False)

    def __post_init__(self):
        if self.w13.rows != 2 * self.inter or self.w13.cols != self.hidden:
            raise ValueError("w13 must be [E, 2I, H]")
        if self.w2.rows != self.hidden or self.w2.cols != self.inter:
            raise ValueError("w2 must be [E, H, I]")
        tot = self.num_routed + self.num_shared
        if self.w13.num_experts < tot or self.w2.num_experts < tot:
            raise ValueError("weight stacks hold fewer experts than routed + shared")
        if self.shared_gate is not None:
            g = _dev(self.shared_gate, torch.bfloat16, "shared_gate")
            if g.numel() != self.hidden:
                raise ValueError(f"shared_gate must hold {self.hidden} values (hidden size)")
            if self.num_shared == 0 and self.dense_shared is None:
                raise ValueError("shared_gate given but the layer has no shared expert")
            self.shared_gate = g.reshape(-1)
        if self.dense_shared is not None:
            w13s, w2s = self.dense_shared
            _dev(w13s, torch.bfloat16, "dense_shared w13")
            _dev(w2s, torch.bfloat16, "dense_shared w2")
            if w13s.dim() != 2 or w13s.shape[1] != self.hidden or w13s.shape[0] % 2:
                raise ValueError("dense_shared w13 must be [2*Is, H]")
            Is = w13s.shape[0] // 2
            if Is % 64:
                raise ValueError("the dense shared expert's intermediate size must be a multiple of 64")
            if tuple(w2s.shape) != (self.hidden, Is):
                raise ValueError(f"dense_shared w2 must be [{self.hidden}, {Is}]")

    def desc(self) -> N.lutmoe_moe_desc:
        if self._desc is None:
            d = N.lutmoe_moe_desc()
            d.w13 = self.w13.desc()
            d.w2 = self.w2.desc()
            d.hidden, d.inter = self.hidden, self.inter
            d.num_routed, d.num_shared = self.num_routed, self.num_shared
            d.shared_gate = None if self.shared_gate is None else self.shared_gate.data_ptr()
            if self.dense_shared is not None:
                d.dense_inter = self.dense_shared[0].shape[0] // 2
                d.dense_w13 = self.dense_shared[0].data_ptr()
                d.dense_w2 = self.dense_shared[1].data_ptr()
            self._desc = d
        return self._desc


def _slot_count(shared_inter: int, inter: int) -> int:
    if shared_inter % inter:
        raise ValueError(f"shared intermediate size {shared_inter} is not a multiple of {inter}")
    return shared_inter // inter


def split_shared_bl4(codes13: torch.Tensor, tables13: torch.Tensor, codes2: torch.Tensor,
                     tables2: torch.Tensor, inter: int):
    """One BL4 shared expert with intermediate size m*I -> m slots of intermediate size I.

    codes13 [2*m*I, H/2] and tables13 [2*m*I, H/64, 16] hold gate rows [0, m*I) and up
    rows [m*I, 2*m*I); codes2 [H, m*I/2], tables2 [H, m*I/64, 16].  Slot j takes gate and
    up rows [j*I, (j+1)*I) and down columns [j*I, (j+1)*I) (whole 64-weight blocks, so
    I % 64 == 0).  SwiGLU acts per intermediate index, so the slots' outputs sum to the
    expert's.  Returns (codes13 [m, 2I, H/2], tables13 [m, 2I, H/64, 16],
    codes2 [m, H, I/2], tables2 [m, H, I/64, 16]); tables keep their dtype."""
    if inter % 64:
        raise ValueError("splitting a BL4 shared expert needs I % 64 == 0")
    m = _slot_count(codes13.shape[0] // 2, inter)
    Is = m * inter
    c13, t13, c2, t2 = [], [], [], []
    for j in range(m):
        g, u = slice(j * inter, (j + 1) * inter), slice(Is + j * inter, Is + (j + 1) * inter)
        c13.append(torch.cat([codes13[g], codes13[u]]))
        t13.append(torch.cat([tables13[g], tables13[u]]))
        c2.append(codes2[:, j * inter // 2:(j + 1) * inter // 2])
        t2.append(tables2[:, j * inter // 64:(j + 1) * inter // 64])
    return (torch.stack(c13).contiguous(), torch.stack(t13).contiguous(), torch.stack(c2).contiguous(),
            torch.stack(t2).contiguous())


def split_shared_ref(codes13: torch.Tensor, absmax13: torch.Tensor, codes2: torch.Tensor,
                     absmax2: torch.Tensor, inter: int, block_size: int = 128):
    """One REF shared expert with intermediate size m*I -> m slots of intermediate size I.

    codes13 [2*m*I, H], absmax13 [2*m*I*H / block_size]; codes2 [H, m*I], absmax2
    [H*m*I / block_size] (absmax blocks of the row-major flattened matrices).  Each slot
    gets the absmax entries of its own elements, so every absmax block must lie inside
    one slot row: H, I and m*I multiples of block_size.  Returns (codes13 [m, 2I, H],
    absmax13 [m, 2I*H/bs], codes2 [m, H, I], absmax2 [m, H*I/bs])."""
    H = codes13.shape[1]
    m = _slot_count(codes13.shape[0] // 2, inter)
    Is = m * inter
    if H % block_size or inter % block_size:
        raise ValueError("splitting a REF shared expert needs H and I multiples of block_size")
    a13 = absmax13.reshape(2 * Is, H // block_size)
    a2 = absmax2.reshape(H, Is // block_size)
    nb = inter // block_size
    c13, b13, c2, b2 = [], [], [], []
    for j in range(m):
        g, u = slice(j * inter, (j + 1) * inter), slice(Is + j * inter, Is + (j + 1) * inter)
        c13.append(torch.cat([codes13[g], codes13[u]]))
        b13.append(torch.cat([a13[g], a13[u]]).reshape(-1))
        c2.append(codes2[:, j * inter:(j + 1) * inter])
        b2.append(a2[:, j * nb:(j + 1) * nb].reshape(-1))
    return (torch.stack(c13).contiguous(), torch.stack(b13).contiguous(), torch.stack(c2).contiguous(),
            torch.stack(b2).contiguous())


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream
