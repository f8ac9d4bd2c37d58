"""Loading the reference's on-disk LUT checkpoints into device weight stacks.

Two layouts the reference writes for MoE expert weights (REF format: one uint8 code
per weight into a bf16[256] codebook, one bf16 absmax per 128 consecutive weights):

* convert_checkpoint.py (`vllm_lut/convert_checkpoint.py:150-176`): per expert weight
  tensor `...experts.{e}.{gate,up,down}_proj.weight` the flattened uint8 codes, beside it
  `<name>.absmax` (bf16, one per 128 weights), and the codebook as
  `model._lut_codebook`.  `load_converted_layer` builds a layer from such a mapping (a
  safetensors file opened with `safetensors.torch.load_file`, or any dict of tensors).
* GGUF (`llama-cpp-port/scripts/convert_lut.py:236-405`): expert tensors of type
  BLOCKLUT8, each one blob `[codes | absmax]` - the codes either one byte per weight or,
  with `lut-moe.nested_lut`, the bit-plane sections `[low 4 bits | bits 4-5 | bits 6-7]`
  (`:95-110`) - and the metadata `lut-moe.block_size`, `lut-moe.lut_table` (bf16 bits of
  the 256-entry codebook) and, for nested files, `lut-moe.lut_mapped64` /
  `lut-moe.lut_mapped16` (the tier tables, `:113-140`).  `read_gguf` parses the file
  (memory-mapped, nothing executed), `load_gguf_layer` builds a layer at a tier: 8-bit
  codes with the full table, or the low 6 / 4 bits (unpacked on the GPU by
  `lutmoe_unpack_6bit` / `lut_moe_launch_unpack_4bit`) with the mapped table, as the
  reference's tier reader (`csrc/tensor_engine/tensor_engine.cpp:504-548`); the tier may
  differ per expert (the reference keeps one per expert node).  `upgrade_gguf_experts`
  promotes resident experts to a higher-precision tier by reading only the sections they
  lack and merging them into the device codes (`lutmoe_merge_bitplane`), where the
  reference reloads the whole expert (`csrc/topology/model_topology.cpp:74-80`).

The BLOCKLUT8 type id lives in the reference's patched gguf-py, which is not part of it;
tensors are therefore recognised by name (`is_expert_tensor`, `convert_lut.py:143-176`)
and sized by the offset of the next tensor, whatever their type id.
"""
from __future__ import annotations

import struct
from typing import Dict, Iterable, Mapping, Optional, Sequence, Tuple, Union

import numpy as np
import torch

from . import ops
from .formats import MoEWeights, RefStack

__all__ = ["read_gguf", "GGUFFile", "is_expert_tensor", "expert_key", "load_converted_layer",
           "load_gguf_layer", "upgrade_gguf_experts"]

# tier -> metadata key of its table (convert_lut.py:113-140; tensor_engine.hpp:287-291)
_TIER_TABLE = {0: "lut-moe.lut_table", 1: "lut-moe.lut_mapped64", 2: "lut-moe.lut_mapped16"}

GGUF_MAGIC = 0x46554747
_SCALARS = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<?", 10: "<Q",
            11: "<q", 12: "<d"}
_T_STRING, _T_ARRAY = 8, 9


def is_expert_tensor(name: str) -> bool:
    """Routed-expert weight names, as convert_lut.py:143-176 decides them (shared experts
    and routers excluded)."""
    n = name.lower()
    pats = ("experts.", "mlp.experts", ".experts.", "ffn_gate_exps", "ffn_up_exps",
            "ffn_down_exps", "gate_exps", "down_exps", "up_exps")
    excl = ("shared_expert", "shexp", "gate_inp", "gate.weight", "router")
    return any(p in n for p in pats) and not any(x in n for x in excl)


def expert_key(layer: int, e: int, proj: str) -> str:
    """HF name of an expert projection (the keys quant_method.py:190-222 reads)."""
    return f"model.layers.{layer}.mlp.experts.{e}.{proj}_proj.weight"


class GGUFFile:
    """A parsed GGUF file: `kv` (metadata) and `tensors` (name -> (dims, type id, raw
    bytes as a read-only uint8 memmap))."""

    def __init__(self, kv: Dict[str, object], tensors: Dict[str, Tuple[tuple, int, np.ndarray]]):
        self.kv = kv
        self.tensors = tensors


class _Reader:
    def __init__(self, buf: memoryview):
        self.buf, self.pos = buf, 0

    def take(self, fmt: str):
        v = struct.unpack_from(fmt, self.buf, self.pos)[0]
        self.pos += struct.calcsize(fmt)
        return v

    def string(self) -> str:
        n = self.take("<Q")
        s = bytes(self.buf[self.pos:self.pos + n]).decode("utf-8")
        self.pos += n
        return s

    def value(self, t: int):
        if t in _SCALARS:
            return self.take(_SCALARS[t])
        if t == _T_STRING:
            return self.string()
        if t == _T_ARRAY:
            et, n = self.take("<I"), self.take("<Q")
            if et in _SCALARS and et != 7:
                fmt = _SCALARS[et]
                a = np.frombuffer(self.buf, dtype=np.dtype(fmt), count=n, offset=self.pos).copy()
                self.pos += n * a.itemsize
                return a
            return [self.value(et) for _ in range(n)]
        raise ValueError(f"unknown GGUF value type {t}")


def read_gguf(path: str) -> GGUFFile:
    """Parse a GGUF (v2/v3) file: header, metadata, tensor infos; tensor data stays in a
    read-only memory map."""
    mm = np.memmap(path, dtype=np.uint8, mode="r")
    r = _Reader(memoryview(mm))
    if r.take("<I") != GGUF_MAGIC:
        raise ValueError(f"{path}: not a GGUF file")
    version = r.take("<I")
    if version not in (2, 3):
        raise ValueError(f"{path}: GGUF version {version} not supported")
    n_tensors, n_kv = r.take("<Q"), r.take("<Q")
    kv: Dict[str, object] = {}
    for _ in range(n_kv):
        key = r.string()
        kv[key] = r.value(r.take("<I"))
    infos = []
    for _ in range(n_tensors):
        name = r.string()
        nd = r.take("<I")
        dims = tuple(r.take("<Q") for _ in range(nd))
        ttype = r.take("<I")
        off = r.take("<Q")
        infos.append((name, dims, ttype, off))
    align = int(kv.get("general.alignment", 32))
    data0 = (r.pos + align - 1) // align * align
    ends = sorted(off for _, _, _, off in infos) + [mm.size - data0]
    tensors = {}
    for name, dims, ttype, off in infos:
        nxt = min(e for e in ends if e > off) if any(e > off for e in ends) else mm.size - data0
        tensors[name] = (dims, ttype, mm[data0 + off:data0 + nxt])
    return GGUFFile(kv, tensors)


def _split_blocklut(raw: np.ndarray, n: int, block_size: int) -> Tuple[np.ndarray, np.ndarray]:
    """One BLOCKLUT8 blob -> (codes or bit-plane bytes [n], absmax bf16 bits [nb])."""
    nb = -(-n // block_size)
    if raw.size < n + 2 * nb:
        raise ValueError(f"BLOCKLUT8 tensor of {raw.size} bytes is shorter than {n} + {2 * nb}")
    return np.asarray(raw[:n]), np.asarray(raw[n:n + 2 * nb]).view(np.uint16)


def _table256(vals: np.ndarray) -> torch.Tensor:
    """bf16 bits of a (possibly shorter) table, padded to 256 entries with its last one
    (convert_lut.py:124-128)."""
    v = np.asarray(vals, dtype=np.uint16).reshape(-1)
    out = np.full(256, v[-1], dtype=np.uint16)
    out[:min(256, v.size)] = v[:256]
    return torch.from_numpy(out.view(np.int16)).view(torch.bfloat16)


def _stack(codes_list, absmax_list, codebook_bf16, block_size, rows, cols, device) -> RefStack:
    codes = torch.stack([torch.as_tensor(c).reshape(rows, cols) for c in codes_list]).to(device)
    am = torch.stack([torch.as_tensor(a).reshape(-1) for a in absmax_list]).to(device)
    return RefStack(codes.contiguous(), am.contiguous(), codebook_bf16.to(device), block_size)


def load_converted_layer(tensors: Mapping[str, torch.Tensor], layer: int, num_experts: int,
                         hidden: int, inter: int, device="cuda",
                         codebook_key: str = "model._lut_codebook",
                         num_shared: int = 0) -> MoEWeights:
    """One MoE layer from convert_checkpoint.py's tensors: per routed expert e the flattened
    uint8 codes of gate/up/down (`expert_key`) and `<key>.absmax` (bf16, 128 weights per
    entry), and the bf16[256] codebook.  W13 = gate rows then up rows (quant_method.py:254),
    its absmax the gate blocks then the up blocks (I*H is a multiple of 128, so no block
    straddles the two)."""
    cb = tensors[codebook_key].to(torch.bfloat16).reshape(-1)
    if cb.numel() != 256:
        raise ValueError("the codebook must hold 256 entries")
    c13, a13, c2, a2 = [], [], [], []
    for e in range(num_experts):
        g, u, d = (expert_key(layer, e, p) for p in ("gate", "up", "down"))
        c13.append(torch.cat([tensors[g].reshape(-1), tensors[u].reshape(-1)]).to(torch.uint8))
        a13.append(torch.cat([tensors[g + ".absmax"].reshape(-1), tensors[u + ".absmax"].reshape(-1)]))
        c2.append(tensors[d].reshape(-1).to(torch.uint8))
        a2.append(tensors[d + ".absmax"].reshape(-1))
    a13 = [a.to(torch.bfloat16) for a in a13]
    a2 = [a.to(torch.bfloat16) for a in a2]
    w13 = _stack(c13, a13, cb, 128, 2 * inter, hidden, device)
    w2 = _stack(c2, a2, cb, 128, hidden, inter, device)
    return MoEWeights(w13, w2, hidden, inter, num_experts - num_shared, num_shared)


def _tier_codes(raw_codes: np.ndarray, n: int, nested: bool, tier: int, device) -> torch.Tensor:
    """Device uint8 codes [n] at a tier from a BLOCKLUT8 code section: the bytes
    themselves (plain files), or the bit-plane sections unpacked on the GPU: tier 0 = all
    eight bits, tier 1 = the low six (low 4 | bits 4-5), tier 2 = the low four."""
    if not nested:
        if tier != 0:
            raise ValueError("a plain (non-nested) BLOCKLUT file has only tier 0")
        return torch.from_numpy(np.array(raw_codes)).to(device)
    if n % 4:
        raise ValueError("bit-plane sections need a multiple of 4 weights")
    low = torch.from_numpy(np.array(raw_codes[:n // 2])).to(device)
    if tier == 2:
        buf = torch.empty(n, dtype=torch.uint8, device=device)
        buf[:n // 2] = low
        ops.unpack_4bit_(buf, n)
        return buf
    mid = torch.from_numpy(np.array(raw_codes[n // 2:n // 2 + n // 4])).to(device)
    c6 = ops.unpack_6bit(torch.cat([low, mid]), n)
    if tier == 1:
        return c6
    high = torch.from_numpy(np.array(raw_codes[n // 2 + n // 4:n])).to(device)
    return ops.merge_bitplane_(c6, high, 6)


def _tier_table(g: "GGUFFile", tier: int) -> torch.Tensor:
    key = _TIER_TABLE[tier]
    if key not in g.kv:
        raise ValueError(f"{key} missing from the GGUF metadata")
    return _table256(np.asarray(g.kv[key]))


def load_gguf_layer(g: GGUFFile, layer: int, num_experts: int, hidden: int, inter: int,
                    tier: Union[int, Sequence[int]] = 0, device="cuda",
                    num_shared: int = 0) -> MoEWeights:
    """One MoE layer from a convert_lut.py GGUF file (expert tensors named as
    `expert_key`).  tier 0: 8-bit codes with `lut-moe.lut_table`; tiers 1 / 2 (nested
    files only): the low 6 / 4 bits with `lut-moe.lut_mapped64` / `lut-moe.lut_mapped16`
    padded to 256 entries.  ``tier`` is one tier for every expert or one per expert
    (num_experts entries); mixed tiers give the stacks one codebook row per expert.
    The stacks record the tiers in ``.tiers`` (read by `upgrade_gguf_experts`)."""
    bs = int(g.kv.get("lut-moe.block_size", 128))
    nested = bool(g.kv.get("lut-moe.nested_lut", False))
    tiers = [int(tier)] * num_experts if isinstance(tier, (int, np.integer)) else [int(t) for t in tier]
    if len(tiers) != num_experts or any(t not in _TIER_TABLE for t in tiers):
        raise ValueError("tier must be 0, 1 or 2, or a list of those with one entry per expert")
    tables = {t: _tier_table(g, t) for t in sorted(set(tiers))}
    cb = tables[tiers[0]] if len(tables) == 1 else torch.stack([tables[t] for t in tiers])

    def proj(name, n, t):
        dims, _, raw = g.tensors[name]
        codes, am = _split_blocklut(raw, n, bs)
        return (_tier_codes(codes, n, nested, t, device),
                torch.from_numpy(np.array(am).view(np.int16)).view(torch.bfloat16))

    n13, n2 = inter * hidden, hidden * inter
    c13, a13, c2, a2 = [], [], [], []
    for e in range(num_experts):
        cg, ag = proj(expert_key(layer, e, "gate"), n13, tiers[e])
        cu, au = proj(expert_key(layer, e, "up"), n13, tiers[e])
        cd, ad = proj(expert_key(layer, e, "down"), n2, tiers[e])
        c13.append(torch.cat([cg, cu]))
        a13.append(torch.cat([ag, au]))
        c2.append(cd)
        a2.append(ad)
    w13 = _stack(c13, a13, cb, bs, 2 * inter, hidden, device)
    w2 = _stack(c2, a2, cb, bs, hidden, inter, device)
    w13.tiers = w2.tiers = tiers
    return MoEWeights(w13, w2, hidden, inter, num_experts - num_shared, num_shared)


def upgrade_gguf_experts(moe: MoEWeights, g: GGUFFile, layer: int, experts: Iterable[int],
                         tier: int) -> MoEWeights:
    """Promote resident experts of a layer built by `load_gguf_layer` from a nested
    GGUF file to ``tier`` (0 or 1; a lower tier number has more bits) in place.

    Only the sections the resident codes lack are read from the file: bits 4-5 (the mid
    section, n/4 bytes) for tier 2 -> 1, bits 6-7 (the high section) for 1 -> 0, both
    for 2 -> 0 -- the deltas between the reference's per-tier read sizes
    (`csrc/tensor_engine/tensor_engine.cpp:504-510`) -- and merged into the device codes
    by `lutmoe_merge_bitplane`; the experts then use the new tier's table.  The
    result equals `load_gguf_layer` at the new tiers.  Experts already at ``tier`` or
    above are left alone; the call is stream-ordered with the layer's other work.

    Codes and codebook rows change in place, so graphs captured earlier stay valid,
    except on the first mixed-tier promotion of a layer loaded at one tier: its shared
    codebook then becomes one row per expert (a new tensor; capture again)."""
    w13, w2 = moe.w13, moe.w2
    tiers = getattr(w13, "tiers", None)
    if tiers is None or not isinstance(w13, RefStack) or not isinstance(w2, RefStack):
        raise ValueError("the layer must come from load_gguf_layer")
    if not g.kv.get("lut-moe.nested_lut", False):
        raise ValueError("tier upgrades need a nested (bit-plane) GGUF file")
    if tier not in (0, 1):
        raise ValueError("the target tier must be 0 or 1")
    inter, hidden = moe.inter, moe.hidden
    n13, n2 = inter * hidden, hidden * inter
    dev = w13.codes.device
    up = [int(e) for e in experts if tiers[int(e)] > tier]
    if not up:
        return moe
    for e in up:
        secs = ([("mid", 4)] if tiers[e] == 2 else []) + ([("high", 6)] if tier == 0 else [])
        for stack, name, n, row0 in ((w13, "gate", n13, 0), (w13, "up", n13, inter),
                                     (w2, "down", n2, 0)):
            raw = g.tensors[expert_key(layer, e, name)][2]
            codes = stack.codes[e, row0:row0 + n // stack.cols].view(-1)   # a view: merged in place
            for sec, shift in secs:
                a = n // 2 if sec == "mid" else n // 2 + n // 4
                plane = torch.from_numpy(np.array(raw[a:a + n // 4])).to(dev)
                ops.merge_bitplane_(codes, plane, shift)
        tiers[e] = tier
    table = _tier_table(g, tier).to(dev)
    for stack in (w13, w2):
        if stack.codebook_stride == 0 and all(t == tier for t in tiers):
            stack.codebook.copy_(table.reshape(stack.codebook.shape))
        else:
            if stack.codebook_stride == 0:
                stack.codebook = stack.codebook.reshape(1, 256).repeat(stack.num_experts, 1)
                stack.codebook_stride = 256
            stack.codebook[up] = table
    moe._desc = None
    return moe
