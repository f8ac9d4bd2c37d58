"""Shared helpers for the parity tests: seeded inputs, host<->device bf16 moves,
and the oracle-side builders of the same weights the GPU sees."""
from __future__ import annotations

import os

import numpy as np

import oracle as O

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def to_dev_bf16(bits: np.ndarray, device):
    import torch
    return torch.from_numpy(np.ascontiguousarray(bits, np.uint16).view(np.int16)).view(
        torch.bfloat16).to(device)


def to_dev_f16(bits: np.ndarray, device):
    import torch
    return torch.from_numpy(np.ascontiguousarray(bits, np.uint16).view(np.float16)).to(device)


def bf16_bits(t) -> np.ndarray:
    import torch
    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def rel_maxabs(got, ref) -> float:
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    den = np.abs(ref).max()
    return float(np.abs(got - ref).max() / (den if den > 0 else 1.0))


def rel_excess_bf16(got, ref) -> float:
    """For a bf16 result: max over elements of (|got - bf16(ref)| minus one bf16 ulp of
    bf16(ref), at least 0) / max|ref|.  The result may sit one rounding step from the oracle
    rounded to bf16 (its fp32 sum and the oracle's float64 sum can round to neighbouring
    bf16 values); everything beyond that step is held to the same relative bar as an fp32
    result."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    refb = O.bf16_to_f32(O.f32_to_bf16(ref.astype(np.float32))).astype(np.float64)
    ulp = np.spacing(np.abs(refb).astype(np.float32)).astype(np.float64) * 65536.0
    excess = np.maximum(np.abs(got - refb) - ulp, 0.0)
    den = np.abs(ref).max()
    return float(excess.max() / (den if den > 0 else 1.0))


def golden_codebook() -> np.ndarray:
    """bf16 bits of the reference's shipped Qwen blocklut_256 codebook (derived fixture)."""
    return np.load(os.path.join(GOLDEN, "codebooks.npz"))["qwen_blocklut_256_bf16"]


class BL4Expertset:
    """E BL4-encoded matrices [M, K] built by the CPU oracle from seeded N(0, std) weights."""

    def __init__(self, E, M, K, seed, std=0.02, n_iter=20):
        rng = np.random.default_rng(seed)
        self.E, self.M, self.K = E, M, K
        self.codes = np.empty((E, M, K // 2), np.uint8)
        self.tables = np.empty((E, M, K // 64, 16), np.uint16)
        for e in range(E):
            w = (rng.standard_normal((M, K)) * std).astype(np.float32)
            self.codes[e], self.tables[e] = O.bl4_encode(w, n_iter=n_iter)

    def deq_f32(self, e) -> np.ndarray:
        return O.bf16_to_f32(O.bl4_dequant(self.codes[e], self.tables[e]))

    def stack(self, device):
        import torch
        from block_lut_amd.formats import BL4Stack
        return BL4Stack.from_fp16(torch.from_numpy(self.codes).to(device),
                                  to_dev_f16(self.tables, device))


TIER_MASK = {0: 0xFF, 1: 0x3F, 2: 0x0F}


def tier_tables(cb_bits):
    """Tier 0 / 1 / 2 tables of a sorted 256-entry codebook: itself and its first 64 /
    16 entries padded with their last (convert_lut.py:113-140 prefix-pad rule)."""
    cb_bits = np.asarray(cb_bits, np.uint16)

    def pad(k):
        t = np.full(256, cb_bits[k - 1], np.uint16)
        t[:k] = cb_bits[:k]
        return t
    return {0: cb_bits.copy(), 1: pad(64), 2: pad(16)}


class RefExpertset:
    """E REF matrices quantized by the oracle's restatement of LUTQuantizer.quantize.
    With ``tiers`` (one of 0/1/2 per expert) expert e keeps the low 8/6/4 code bits and
    its tier's table: the stack then carries one codebook per expert."""

    def __init__(self, E, M, K, seed, std=0.02, block_size=128, tiers=None):
        rng = np.random.default_rng(seed)
        self.E, self.M, self.K, self.bs = E, M, K, block_size
        self.cb = golden_codebook()
        self.tiers = list(tiers) if tiers is not None else None
        tabs = tier_tables(self.cb)
        self.cbs = [tabs[t] for t in self.tiers] if self.tiers else [self.cb] * E
        nb = -(-M * K // block_size)
        self.codes = np.empty((E, M, K), np.uint8)
        self.absmax = np.empty((E, nb), np.uint16)
        for e in range(E):
            w = (rng.standard_normal((M, K)) * std).astype(np.float32)
            idx, am = O.ref_quantize(w, self.cb, block_size)
            if self.tiers:
                idx = idx & TIER_MASK[self.tiers[e]]
            self.codes[e] = idx.reshape(M, K)
            self.absmax[e] = am

    def deq_f32(self, e) -> np.ndarray:
        return O.bf16_to_f32(O.ref_dequant(self.codes[e], self.absmax[e], self.cbs[e], self.bs)).reshape(
            self.M, self.K)

    def gemv_f32(self, e) -> np.ndarray:
        """Weights as the reference's decode GEMV sees them: f32(cb[c]) * f32(absmax)
        without the bf16 rounding of the dequantised tensor (vllm_lut/cuda_lut_gemv.py:50-57)."""
        cb = O.bf16_to_f32(self.cbs[e])
        am = O.bf16_to_f32(self.absmax[e])
        blk = np.minimum(np.arange(self.M * self.K) // self.bs, am.size - 1)
        return (cb[self.codes[e].reshape(-1)] * am[blk]).astype(np.float32).reshape(self.M, self.K)

    def stack(self, device):
        import torch
        from block_lut_amd.formats import RefStack
        cb = np.stack(self.cbs) if self.tiers else self.cb
        return RefStack(torch.from_numpy(self.codes).to(device), to_dev_bf16(self.absmax, device),
                        to_dev_bf16(cb, device), self.bs)


class NestedExpertset:
    """E NestedLUT matrices [M, K] built by the CPU oracle's nested encoder from
    seeded N(0, std) weights; expert e is kept at tier bits[e] (2, 3 or 4):
    bit-plane sections [p01 | p2 | p3] of its low bits[e] code bits and the
    tier's bf16 tables [M, K/64, 2^b]."""

    def __init__(self, bits, M, K, seed, std=0.02, n_iter=20):
        rng = np.random.default_rng(seed)
        self.bits = list(bits)
        self.E, self.M, self.K = len(self.bits), M, K
        self.codes, self.tables = [], []
        for b in self.bits:
            w = (rng.standard_normal((M, K)) * std).astype(np.float32)
            codes, t2, t3, t4 = O.nested_encode(w, n_iter=n_iter)
            self.codes.append(codes & ((1 << b) - 1))
            self.tables.append({2: t2, 3: t3, 4: t4}[b])

    def planes(self, e) -> np.ndarray:
        pl = O.nested_pack_planes(self.codes[e])
        parts = [pl["p01"].reshape(-1)]
        if self.bits[e] >= 3:
            parts.append(pl["p2"].reshape(-1))
        if self.bits[e] >= 4:
            parts.append(pl["p3"].reshape(-1))
        return np.concatenate(parts)

    def table_bf16(self, e) -> np.ndarray:
        return O.f32_to_bf16(O.f16_to_f32(self.tables[e]))

    def deq_bits(self, e) -> np.ndarray:
        return O.nested_dequant(self.codes[e], self.tables[e], self.bits[e])

    def deq_f32(self, e) -> np.ndarray:
        return O.bf16_to_f32(self.deq_bits(e))

    def stack(self, device):
        import torch
        from block_lut_amd.formats import NestedExpert, NestedStack
        ex = [NestedExpert(b, torch.from_numpy(self.planes(e)).to(device),
                           to_dev_bf16(self.table_bf16(e), device))
              for e, b in enumerate(self.bits)]
        return NestedStack(ex, self.M, self.K)


# ------------------------------------------------------------------ GGUF files
# A minimal GGUF v3 writer for the loader tests: the layout of the GGUF
# specification (header, typed metadata, tensor infos, data aligned to 32
# bytes), as convert_lut.py's GGUFWriter produces it.  BLOCKLUT8's type id is
# defined in the reference's (absent) patched gguf-py; any id works for the
# loader, which sizes tensors by their offsets.
GGUF_BLOCKLUT8_TEST_ID = 1024


def write_gguf(path, kv, tensors, align=32):
    """kv: list of (key, value) with value bool / int (uint32) / float / str / list of
    uint16; tensors: list of (name, dims, type_id, raw bytes)."""
    import struct

    def s(x):
        b = x.encode()
        return struct.pack("<Q", len(b)) + b

    def val(v):
        if isinstance(v, bool):
            return struct.pack("<I", 7) + struct.pack("<?", v)
        if isinstance(v, int):
            return struct.pack("<I", 4) + struct.pack("<I", v)
        if isinstance(v, float):
            return struct.pack("<I", 6) + struct.pack("<f", v)
        if isinstance(v, str):
            return struct.pack("<I", 8) + s(v)
        a = np.asarray(v, dtype=np.uint16)
        return struct.pack("<I", 9) + struct.pack("<IQ", 2, a.size) + a.tobytes()

    head = struct.pack("<IIQQ", 0x46554747, 3, len(tensors), len(kv))
    head += b"".join(s(k) + val(v) for k, v in kv)
    off = 0
    infos, blobs = b"", []
    for name, dims, tid, raw in tensors:
        infos += s(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        infos += struct.pack("<IQ", tid, off)
        raw = bytes(raw)
        pad = (-len(raw)) % align
        blobs.append(raw + b"\0" * pad)
        off += len(raw) + pad
    body = head + infos
    body += b"\0" * ((-len(body)) % align)
    with open(path, "wb") as f:
        f.write(body + b"".join(blobs))
