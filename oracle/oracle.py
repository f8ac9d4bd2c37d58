"""numpy restatement of the reference's LUT-MoE arithmetic (test infrastructure).

Formats
-------
REF   the reference's on-device format: one uint8 code per weight, one bf16
      absmax per 128 consecutive elements of the row-major flattened [out, in]
      matrix, one global bf16[256] codebook
      (vllm_lut/quant_method.py:127-163, vllm_lut/quantizer.py:36-40).
BL4   4-bit codes packed two per byte (even element in the low nibble, as
      runtime/model_offload.py:752-755 packs its low section) and one sorted
      16-entry fp16 k-means codebook per 64 consecutive weights along K.
NL    NestedLUT tiers b in {2, 3, 4}: the tier-b code is the low b bits of the
      4-bit code; tables T2[4] / T3[8] / T4[16] per 64-weight block; codes
      stored as bit-plane sections [bits0-1 | bit2 | bit3] so a tier-b reader
      takes a prefix, the way the reference's tier reader takes a prefix of its
      [low4 | mid2 | high2] sections (csrc/tensor_engine/tensor_engine.cpp:504-510).

Dequantised weight (bit-exact rule, shared with the HIP kernels):
  REF : bf16_rne(f32(cb[c]) * f32(absmax[min(i // 128, nb-1)]))
        (csrc/kernels/tensor_recover.cu:120-127; quantizer.py:335-349)
  BL4 : bf16_rne(f32(fp16 table[c]))
  NL  : bf16_rne(f32(fp16 T_b[c & (2^b-1)]))
"""
from __future__ import annotations

import ctypes
import math
import os
import subprocess

import numpy as np

REF_BLOCK = 128
BL_BLOCK = 64

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None


# --------------------------------------------------------------------------
# C part (sequential float order that the HIP encoder reproduces)
# --------------------------------------------------------------------------

def build_c(force: bool = False) -> str:
    """Compile oracle/lutmoe_oracle.c into oracle/_build/liboracle.so."""
    out_dir = os.path.join(_HERE, "_build")
    out = os.path.join(out_dir, "liboracle.so")
    src = os.path.join(_HERE, "lutmoe_oracle.c")
    if not force and os.path.exists(out) and os.path.getmtime(out) >= os.path.getmtime(src):
        return out
    os.makedirs(out_dir, exist_ok=True)
    tmp = out + f".tmp{os.getpid()}"
    subprocess.check_call(["gcc", "-O2", "-ffp-contract=off", "-fno-fast-math", "-fPIC",
                           "-shared", "-o", tmp, src, "-lm"])
    os.replace(tmp, out)
    return out


def _lib():
    global _LIB
    if _LIB is None:
        path = build_c()
        lib = ctypes.CDLL(path)
        P = ctypes.c_void_p
        I64 = ctypes.c_int64
        lib.oracle_bl4_encode.argtypes = [P, I64, ctypes.c_int, P, P]
        lib.oracle_nested_encode.argtypes = [P, I64, ctypes.c_int, P, P, P, P]
        lib.oracle_ref_gemv.argtypes = [P, P, P, P, I64, I64, I64, P]
        lib.oracle_f32_to_bf16_array.argtypes = [P, P, I64]
        lib.oracle_f32_to_f16_array.argtypes = [P, P, I64]
        _LIB = lib
    return _LIB


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


# --------------------------------------------------------------------------
# 16-bit float helpers
# --------------------------------------------------------------------------

def f32_to_bf16(x) -> np.ndarray:
    """IEEE round-to-nearest-even float32 -> bf16 bits (torch's .to(bfloat16))."""
    a = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    u = a.view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(nan, np.uint16(0x7FC0), r).astype(np.uint16)


def bf16_to_f32(h) -> np.ndarray:
    h = np.asarray(h, dtype=np.uint16)
    return (h.astype(np.uint32) << 16).view(np.float32)


def f32_to_f16(x) -> np.ndarray:
    """float32 -> fp16 bits, round-to-nearest-even (numpy's cast)."""
    return np.asarray(x, dtype=np.float32).astype(np.float16).view(np.uint16)


def f16_to_f32(h) -> np.ndarray:
    return np.asarray(h, dtype=np.uint16).view(np.float16).astype(np.float32)


def c_f32_to_bf16(x) -> np.ndarray:
    a = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(a.shape, np.uint16)
    _lib().oracle_f32_to_bf16_array(_ptr(a), _ptr(out), a.size)
    return out


def c_f32_to_f16(x) -> np.ndarray:
    a = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(a.shape, np.uint16)
    _lib().oracle_f32_to_f16_array(_ptr(a), _ptr(out), a.size)
    return out


# --------------------------------------------------------------------------
# REF format (the reference's own)
# --------------------------------------------------------------------------

def ref_quantize(weight, codebook_bf16, block_size: int = REF_BLOCK, input_is_bf16: bool = False):
    """LUTQuantizer.quantize, BLOCKLUT branch (vllm_lut/quantizer.py:242-306).

    weight: float32 values (if input_is_bf16, they must be bf16-representable
    and the normalisation is done in bf16 as torch does for a bf16 tensor,
    quantizer.py:284).  Returns (indices uint8 [N], absmax bf16 bits [nb]).
    """
    flat = np.asarray(weight, dtype=np.float32).reshape(-1)
    n = flat.size
    nb = math.ceil(n / block_size)
    pad = nb * block_size - n
    if pad:                                                     # :274-279
        flat = np.concatenate([flat, np.zeros(pad, np.float32)])
    blocks = flat.reshape(nb, block_size)
    absmax = np.abs(blocks).max(axis=1, keepdims=True)          # :282
    if input_is_bf16:
        absmax = np.maximum(absmax, bf16_to_f32(f32_to_bf16(np.float32(1e-10))))  # :283
        normalized = bf16_to_f32(f32_to_bf16(blocks / absmax))                   # :284 bf16 div
    else:
        absmax = np.maximum(absmax, np.float32(1e-10))
        normalized = (blocks / absmax).astype(np.float32)
    cb = bf16_to_f32(codebook_bf16)
    norm = normalized.reshape(-1)
    idx = np.empty(norm.size, np.uint8)
    step = 1 << 16
    for s in range(0, norm.size, step):                         # :293-296
        d = np.abs(norm[s:s + step, None] - cb[None, :])
        idx[s:s + step] = d.argmin(axis=1)
    return idx[:n], f32_to_bf16(absmax.reshape(-1))             # :298-304


def ref_encode_fast(w_bf16_bits, codebook_f32, block_size: int = REF_BLOCK):
    """encode_blocklut_kernel (vllm_lut/fast_encode.py:22-72): bf16 weights, fp32[256]
    codebook.  Per block of block_size weights (the last one shorter, no padding):
    absmax = max |w| in fp32, at least 1e-10 (:43-47); v = w / absmax in fp32 (:51, IEEE
    here); index of the nearest codebook entry, the first one on equal distances (strict <
    in the scan, :54-62, which is numpy's argmin); absmax stored as bf16 (:68).
    Returns (indices uint8 [N], absmax bf16 bits [ceil(N / block_size)])."""
    w = bf16_to_f32(np.asarray(w_bf16_bits, np.uint16).reshape(-1))
    cb = np.asarray(codebook_f32, np.float32).reshape(-1)
    n = w.size
    nb = -(-n // block_size)
    idx = np.empty(n, np.uint8)
    am = np.empty(nb, np.float32)
    for b in range(nb):
        blk = w[b * block_size:(b + 1) * block_size]
        m = np.float32(max(np.float32(np.abs(blk).max()), np.float32(1e-10)))
        am[b] = m
        v = (blk / m).astype(np.float32)
        d = np.abs(v[:, None] - cb[None, :]).astype(np.float32)
        idx[b * block_size:b * block_size + blk.size] = d.argmin(axis=1)
    return idx, f32_to_bf16(am)


def ref_encode_midpoints(weight, sorted_codebook_f32, block_size: int = REF_BLOCK):
    """The offload runtime's encoder (runtime/model_offload.py:897-907): fp32 weights in
    blocks of block_size (the last one zero-padded, :899), absmax = max |w| at least
    fp32(1e-12) (:900-901), v = w / absmax in fp32 (:902), code = np.searchsorted over the
    fp32 midpoints (c_i + c_{i+1}) / 2 of the ascending codebook (:903-904).
    Returns (indices uint8 [N], absmax bf16 bits [nb])."""
    x = np.asarray(weight, np.float32).reshape(-1)
    n = x.size
    nb = -(-n // block_size)
    pad = nb * block_size - n
    if pad:
        x = np.pad(x, (0, pad))
    blocks = x.reshape(nb, block_size)
    am = np.maximum(np.max(np.abs(blocks), axis=1), np.float32(1e-12))
    v = (blocks / am[:, None]).astype(np.float32).reshape(-1)
    cb = np.asarray(sorted_codebook_f32, np.float32)
    mid = ((cb[:-1] + cb[1:]) / np.float32(2.0)).astype(np.float32)
    idx = np.searchsorted(mid, v).astype(np.uint8)
    return idx[:n], f32_to_bf16(am.astype(np.float32))


def ref_dequant(indices, absmax_bf16, codebook_bf16, block_size: int = REF_BLOCK) -> np.ndarray:
    """decompress_blocklut (quantizer.py:449-477) == cuda_blocklut_recover_to_bf16
    (csrc/kernels/tensor_recover.cu:101-142): bf16(f32(cb[c]) * f32(absmax[blk]))."""
    idx = np.asarray(indices, np.uint8).reshape(-1)
    am = bf16_to_f32(absmax_bf16).reshape(-1)
    cb = bf16_to_f32(codebook_bf16)
    blk = np.minimum(np.arange(idx.size) // block_size, am.size - 1)  # clamp :473-474
    return f32_to_bf16(cb[idx] * am[blk])


def ref_gemv(x_bf16, indices, codebook_bf16, absmax_bf16) -> np.ndarray:
    """lut_gemv_kernel arithmetic (vllm_lut/cuda_lut_gemv.py:23-80), float64 row sums
    of the fp32 products (x * cb) * absmax.  indices [M, K]."""
    idx = np.ascontiguousarray(indices, dtype=np.uint8)
    M, K = idx.shape
    x = np.ascontiguousarray(x_bf16, dtype=np.uint16)
    cb = np.ascontiguousarray(codebook_bf16, dtype=np.uint16)
    am = np.ascontiguousarray(absmax_bf16, dtype=np.uint16)
    y = np.empty(M, np.float64)
    _lib().oracle_ref_gemv(_ptr(x), _ptr(idx), _ptr(cb), _ptr(am), M, K, am.size, _ptr(y))
    return y


def bitplane_pack_ref(indices) -> np.ndarray:
    """3-section bit-plane packing (runtime/model_offload.py:747-758,
    llama-cpp-port/scripts/convert_lut.py:95-110): [low nibble 2/B | mid 2b 4/B | high 2b 4/B]."""
    c = np.asarray(indices, np.uint8).reshape(-1)
    assert c.size % 4 == 0
    low = c & 0x0F
    mid = (c >> 4) & 0x03
    high = (c >> 6) & 0x03
    pl = low[0::2] | (low[1::2] << 4)
    pm = mid[0::4] | (mid[1::4] << 2) | (mid[2::4] << 4) | (mid[3::4] << 6)
    ph = high[0::4] | (high[1::4] << 2) | (high[2::4] << 4) | (high[3::4] << 6)
    return np.concatenate([pl, pm, ph]).astype(np.uint8)


def unpack_4bit_ref(packed, n: int) -> np.ndarray:
    """unpack_4bit_stage1/2 (csrc/kernels/tensor_recover.cu:166-192): the first n/2 bytes
    (low section) become n codes out[2i] = p & 0xF, out[2i+1] = p >> 4."""
    p = np.asarray(packed, np.uint8).reshape(-1)[: n // 2]
    out = np.empty(n, np.uint8)
    out[0::2] = p & 0x0F
    out[1::2] = (p >> 4) & 0x0F
    return out


def unpack_6bit_ref(packed, n: int) -> np.ndarray:
    """CPU 6-bit tier unpack (csrc/tensor_engine/tensor_engine.cpp:535-548):
    code = low nibble | mid 2 bits << 4, reading the low and mid sections."""
    p = np.asarray(packed, np.uint8).reshape(-1)
    low = unpack_4bit_ref(p, n)
    mid_b = p[n // 2: n // 2 + n // 4]
    mid = np.empty(n, np.uint8)
    for j in range(4):
        mid[j::4] = (mid_b >> (2 * j)) & 0x03
    return (low | (mid << 4)).astype(np.uint8)


def merge_bitplane_ref(codes, plane, shift: int) -> np.ndarray:
    """Tier upgrade by one 2-bit section: code i takes (plane[i // 4] >> 2 * (i % 4)) & 3
    at bits [shift, shift + 2), replacing them.  The field rule is the reference's CPU
    6-bit unpack (csrc/tensor_engine/tensor_engine.cpp:535-548: mid bits << 4) and the
    section layout its packer's (llama-cpp-port/scripts/convert_lut.py:95-110); the
    high section (shift 6) follows the same layout."""
    c = np.asarray(codes, np.uint8).reshape(-1).copy()
    p = np.asarray(plane, np.uint8).reshape(-1)
    n = c.size
    assert n % 4 == 0 and p.size >= n // 4 and shift in (0, 2, 4, 6)
    f = np.empty(n, np.uint8)
    for j in range(4):
        f[j::4] = (p[: n // 4] >> (2 * j)) & 0x03
    keep = np.uint8(0xFF ^ (0x03 << shift))
    return ((c & keep) | (f << shift)).astype(np.uint8)


def nested_tables_prefix_pad(lut256_f32) -> tuple:
    """build_nested_luts (llama-cpp-port/scripts/convert_lut.py:113-140): the K-entry
    tier tables are the first K sorted centroids padded with the last one; all bf16 bits."""
    lut = np.asarray(lut256_f32, np.float32)

    def pad(part):
        t = np.full(256, part[-1], np.float32)
        t[: part.size] = part
        return f32_to_bf16(t)

    return pad(lut), pad(lut[:64]), pad(lut[:16])


def nested_tables_merge_map(nested_lut_f32, map_256_to_k) -> np.ndarray:
    """Merge-map tables (evaluation/generate_nested_lut.py:93-176,264-269):
    mappedK[i] = bf16(C_K[map256toK[i]])."""
    return f32_to_bf16(np.asarray(nested_lut_f32, np.float32)[np.asarray(map_256_to_k, np.int64)])


def ref_tier_dequant(packed_sections, absmax_bf16, tables_bf16, n: int, tier: int) -> np.ndarray:
    """Tier-t REF dequant: tier 2 reads the low section (unpack_4bit), tier 1 the low+mid
    sections (6-bit unpack), tier 0 the full code; the tier's 256-entry table is chosen by
    get_lut_device_for_tier (csrc/tensor_engine/tensor_engine.hpp:287-291) and applied by
    blocklut_recover (csrc/topology/model_topology.cpp:597-619)."""
    p = np.asarray(packed_sections, np.uint8).reshape(-1)
    if tier == 2:
        codes = unpack_4bit_ref(p, n)
    else:
        codes = unpack_6bit_ref(p, n)
        if tier == 0:
            hb = p[n // 2 + n // 4: n]
            high = np.empty(n, np.uint8)
            for j in range(4):
                high[j::4] = (hb >> (2 * j)) & 0x03
            codes = (codes | (high << 6)).astype(np.uint8)
    return ref_dequant(codes, absmax_bf16, tables_bf16)


# --- LUTQuantizer training (restated with torch CPU so the randperm stream matches) ---

def train_kmeans_ref(data, k: int, n_iter: int, seed: int, max_samples: int = 200000):
    """LUTQuantizer._train_kmeans (vllm_lut/quantizer.py:120-178) on CPU after
    torch.manual_seed(seed).  Returns bf16 bits of the sorted centroids."""
    import torch
    torch.manual_seed(seed)
    data = torch.as_tensor(np.asarray(data, np.float32)).float()
    n_total = data.shape[0]
    if n_total > max_samples:                                   # :142-147
        train = data[torch.randperm(n_total)[:max_samples]]
    else:
        train = data
    n_init = min(k, train.shape[0])
    cent = train[torch.randperm(train.shape[0])[:n_init]].clone()  # :150-152
    if train.shape[0] < k:
        cent = torch.cat([cent, torch.zeros(k - n_init)])
    for _ in range(n_iter):                                     # :158-173
        chunk = min(65536, train.shape[0])
        parts = []
        for s in range(0, train.shape[0], chunk):
            c = train[s:s + chunk]
            parts.append(torch.abs(c.unsqueeze(1) - cent.unsqueeze(0)).argmin(dim=1))
        a = torch.cat(parts)
        for i in range(k):
            m = a == i
            if m.any():
                cent[i] = train[m].mean()
    cent, _ = torch.sort(cent)                                  # :176
    return cent.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)  # :177


def greedy_merge_ref(centroids_f32, target_k: int) -> np.ndarray:
    """LUTQuantizer._greedy_merge (quantizer.py:202-221) in float32; returns float32."""
    import torch
    c = torch.as_tensor(np.asarray(centroids_f32, np.float32)).clone()
    while c.shape[0] > target_k:
        d = torch.abs(c.unsqueeze(0) - c.unsqueeze(1))
        d = d + torch.eye(c.shape[0]) * float("inf")
        i, j = divmod(d.argmin().item(), c.shape[0])
        c[i] = (c[i] + c[j]) / 2
        c = torch.cat([c[:j], c[j + 1:]])
    c, _ = torch.sort(c)
    return c.numpy()


def build_mapped_table_ref(centroids_f32, table_size: int = 256) -> np.ndarray:
    """LUTQuantizer._build_mapped_table (quantizer.py:223-236): repeat, then bf16 bits."""
    c = np.asarray(centroids_f32, np.float32)
    reps, rem = divmod(table_size, c.size)
    t = np.concatenate([np.tile(c, reps), c[:rem]])
    return f32_to_bf16(t)


# --------------------------------------------------------------------------
# BL4 (per-64-block fp16 16-entry codebooks)
# --------------------------------------------------------------------------

def bl4_pack(codes) -> np.ndarray:
    """[M, K] codes 0..15 -> [M, K/2] bytes, even element in the low nibble."""
    c = np.asarray(codes, np.uint8)
    return (c[..., 0::2] | (c[..., 1::2] << 4)).astype(np.uint8)


def bl4_unpack(packed) -> np.ndarray:
    p = np.asarray(packed, np.uint8)
    out = np.empty(p.shape[:-1] + (p.shape[-1] * 2,), np.uint8)
    out[..., 0::2] = p & 0x0F
    out[..., 1::2] = p >> 4
    return out


def bl4_encode(weight, n_iter: int = 50):
    """Per-64-block k-means (k=16) BL4 encoder.  weight [M, K] float32, K % 64 == 0.
    Returns (packed codes uint8 [M, K/2], tables fp16 bits [M, K/64, 16])."""
    w = np.ascontiguousarray(weight, dtype=np.float32)
    M, K = w.shape
    assert K % BL_BLOCK == 0
    nb = M * K // BL_BLOCK
    codes = np.empty(M * K, np.uint8)
    table = np.empty(nb * 16, np.uint16)
    _lib().oracle_bl4_encode(_ptr(w), nb, n_iter, _ptr(codes), _ptr(table))
    return bl4_pack(codes.reshape(M, K)), table.reshape(M, K // BL_BLOCK, 16)


def bl4_tables_bf16(tables_f16) -> np.ndarray:
    """fp16 codebook entries -> the bf16 dequantised values (bit-exact rule)."""
    return f32_to_bf16(f16_to_f32(tables_f16))


def bl4_dequant(packed, tables_f16) -> np.ndarray:
    """bf16 bits [M, K] of the dequantised BL4 matrix."""
    codes = bl4_unpack(packed).astype(np.int64)
    M, K = codes.shape
    tb = bl4_tables_bf16(tables_f16).reshape(M, K // BL_BLOCK, 16)
    blk = np.broadcast_to(np.arange(K) // BL_BLOCK, (M, K))
    return tb[np.arange(M)[:, None], blk, codes]


_F16_BF16_F32 = None


def bl4_dequant_f32(packed, tables_f16, row_chunk: int = 1024) -> np.ndarray:
    """float32 [M, K] values of the dequantised BL4 matrix (bl4_dequant's bf16
    values widened), gathered per 64-weight block with take_along_axis, a few
    rows at a time so that large matrices (Mixtral's 28672 x 4096) stay within
    a bounded amount of host memory."""
    global _F16_BF16_F32
    if _F16_BF16_F32 is None:   # every fp16 pattern -> its bf16 value (bl4_tables_bf16) as f32
        _F16_BF16_F32 = bf16_to_f32(bl4_tables_bf16(np.arange(65536, dtype=np.uint16)))
    p = np.asarray(packed, np.uint8)
    M, Kh = p.shape
    K = 2 * Kh
    nb = K // BL_BLOCK
    tb = np.asarray(tables_f16, np.uint16).reshape(M, nb, 16)
    out = np.empty((M, K), np.float32)
    for r0 in range(0, M, row_chunk):
        r1 = min(M, r0 + row_chunk)
        t = _F16_BF16_F32[tb[r0:r1]]                                       # [m, nb, 16]
        c = p[r0:r1].reshape(r1 - r0, nb, 32)
        o = out[r0:r1].reshape(r1 - r0, nb, 64)
        o[..., 0::2] = np.take_along_axis(t, (c & 0x0F).astype(np.intp), axis=2)
        o[..., 1::2] = np.take_along_axis(t, (c >> 4).astype(np.intp), axis=2)
    return out


# --------------------------------------------------------------------------
# NestedLUT 2/3/4-bit tiers
# --------------------------------------------------------------------------

def nested_encode(weight, n_iter: int = 50):
    """Tree-structured nested encoder (see lutmoe_oracle.c).  weight [M, K] f32.
    Returns (codes uint8 [M, K] 0..15, t2 [M,K/64,4], t3 [M,K/64,8], t4 [M,K/64,16])."""
    w = np.ascontiguousarray(weight, dtype=np.float32)
    M, K = w.shape
    assert K % BL_BLOCK == 0
    nb = M * K // BL_BLOCK
    codes = np.empty(M * K, np.uint8)
    t2 = np.empty(nb * 4, np.uint16)
    t3 = np.empty(nb * 8, np.uint16)
    t4 = np.empty(nb * 16, np.uint16)
    _lib().oracle_nested_encode(_ptr(w), nb, n_iter, _ptr(codes), _ptr(t2), _ptr(t3), _ptr(t4))
    kb = K // BL_BLOCK
    return (codes.reshape(M, K), t2.reshape(M, kb, 4), t3.reshape(M, kb, 8),
            t4.reshape(M, kb, 16))


def nested_pack_planes(codes) -> dict:
    """Bit-plane sections of the 4-bit nested codes, per row:
    p01 [M, K/4]: bits 0-1, element 4i in bits 0-1 of byte i (reference mid/high
    packing order, model_offload.py:756-757); p2 / p3 [M, K/8]: bit 2 / bit 3,
    element 8i in bit 0."""
    c = np.asarray(codes, np.uint8)
    f = c & 3
    p01 = f[..., 0::4] | (f[..., 1::4] << 2) | (f[..., 2::4] << 4) | (f[..., 3::4] << 6)
    planes = {"p01": p01.astype(np.uint8)}
    for name, bit in (("p2", 2), ("p3", 3)):
        b = (c >> bit) & 1
        v = np.zeros(b.shape[:-1] + (b.shape[-1] // 8,), np.uint8)
        for j in range(8):
            v |= (b[..., j::8] << j).astype(np.uint8)
        planes[name] = v
    return planes


def nested_unpack_planes(planes: dict, bits: int) -> np.ndarray:
    p01 = np.asarray(planes["p01"], np.uint8)
    K = p01.shape[-1] * 4
    c = np.empty(p01.shape[:-1] + (K,), np.uint8)
    for j in range(4):
        c[..., j::4] = (p01 >> (2 * j)) & 3
    for name, bit in (("p2", 2), ("p3", 3)):
        if bits > bit:
            p = np.asarray(planes[name], np.uint8)
            for j in range(8):
                c[..., j::8] |= ((p >> j) & 1) << bit
    return c


def nested_planes_split(buf, bits: int, M: int, K: int) -> dict:
    """One expert's device buffer of bit-plane sections [p01 M*K/4 | p2 M*K/8 |
    p3 M*K/8] (a tier-b expert holds the first 2, 3 or all of them) -> the
    section dict of nested_pack_planes (rows of the row-major matrix)."""
    b = np.asarray(buf, np.uint8).reshape(-1)
    n = M * K
    pl = {"p01": b[: n // 4].reshape(M, K // 4)}
    if bits >= 3:
        pl["p2"] = b[n // 4: n // 4 + n // 8].reshape(M, K // 8)
    if bits >= 4:
        pl["p3"] = b[n // 4 + n // 8: n // 2].reshape(M, K // 8)
    return pl


def nested_group_planes(buf, bits: int, M: int, K: int) -> np.ndarray:
    """The device order of one expert's codes (this library's own layout, no reference
    counterpart).  Each 32 consecutive weights of the flat row-major order (w_j = code of
    weight j of the group) become the first `bits` of four little-endian uint32 words:
      f0: nibble n = (w_n & 3) | (w_{n+8} & 3) << 2
      f1: nibble n = (w_{n+16} & 3) | (w_{n+24} & 3) << 2
      b2: nibble n bit q = bit 2 of w_{n+8q}   (bits >= 3)
      b3: nibble n bit q = bit 3 of w_{n+8q}   (bits == 4)."""
    codes = nested_unpack_planes(nested_planes_split(buf, bits, M, K), bits).reshape(-1, 32).astype(np.uint32)
    words = []
    f0 = np.zeros(codes.shape[0], np.uint32)
    f1 = np.zeros(codes.shape[0], np.uint32)
    for j in range(8):
        f0 |= ((codes[:, j] & 3) | ((codes[:, j + 8] & 3) << 2)) << np.uint32(4 * j)
        f1 |= ((codes[:, j + 16] & 3) | ((codes[:, j + 24] & 3) << 2)) << np.uint32(4 * j)
    words += [f0, f1]
    for bit in (2, 3):
        if bits > bit:
            w = np.zeros(codes.shape[0], np.uint32)
            for j in range(8):
                for q in range(4):
                    w |= ((codes[:, j + 8 * q] >> np.uint32(bit)) & 1) << np.uint32(4 * j + q)
            words.append(w)
    return np.ascontiguousarray(np.stack(words, axis=1).astype("<u4")).view(np.uint8).reshape(-1)


def nested_ungroup(grouped, bits: int, M: int, K: int) -> dict:
    """Inverse of nested_group_planes: the section dict of nested_pack_planes."""
    g = np.ascontiguousarray(np.asarray(grouped, np.uint8)).view("<u4").reshape(M * K // 32, bits)
    codes = np.zeros((g.shape[0], 32), np.uint8)
    for j in range(8):
        for q in range(4):
            f = g[:, q // 2]
            c = (f >> np.uint32(4 * j + 2 * (q & 1))) & 3
            for bit in (2, 3):
                if bits > bit:
                    c |= ((g[:, bit] >> np.uint32(4 * j + q)) & 1) << np.uint32(bit)
            codes[:, j + 8 * q] = c.astype(np.uint8)
    pl = nested_pack_planes(codes.reshape(M, K))
    return {name: pl[name] for name, bit in (("p01", 0), ("p2", 2), ("p3", 3)) if bits > bit}


def nested_dequant_f32(codes, tables_f16, bits: int, row_chunk: int = 1024) -> np.ndarray:
    """float32 [M, K] values of nested_dequant (its bf16 values widened), gathered per
    64-weight block with take_along_axis, a few rows at a time."""
    global _F16_BF16_F32
    if _F16_BF16_F32 is None:
        _F16_BF16_F32 = bf16_to_f32(bl4_tables_bf16(np.arange(65536, dtype=np.uint16)))
    c = np.asarray(codes, np.uint8)
    M, K = c.shape
    nb, ne = K // BL_BLOCK, 1 << bits
    tb = np.asarray(tables_f16, np.uint16).reshape(M, nb, ne)
    out = np.empty((M, K), np.float32)
    for r0 in range(0, M, row_chunk):
        r1 = min(M, r0 + row_chunk)
        idx = (c[r0:r1] & (ne - 1)).reshape(r1 - r0, nb, 64).astype(np.intp)
        out[r0:r1] = np.take_along_axis(_F16_BF16_F32[tb[r0:r1]], idx, axis=2).reshape(r1 - r0, K)
    return out


def nested_dequant(codes, tables_f16, bits: int) -> np.ndarray:
    """bf16 bits [M, K]: T_b[code & (2^b - 1)] with T_b the tier-b table [M, K/64, 2^b]."""
    c = np.asarray(codes, np.int64) & ((1 << bits) - 1)
    M, K = c.shape
    tb = f32_to_bf16(f16_to_f32(tables_f16)).reshape(M, K // BL_BLOCK, 1 << bits)
    blk = np.broadcast_to(np.arange(K) // BL_BLOCK, (M, K))
    return tb[np.arange(M)[:, None], blk, c]


# --------------------------------------------------------------------------
# Routing, permutation, MoE layer
# --------------------------------------------------------------------------

def route(logits, top_k: int, renormalize: bool = False, scaling: float = 1.0):
    """_routing (vllm_lut/moe_layer.py:358-376) / Qwen __prepare_expert_route
    (customized/qwen.py:44-54): softmax in fp32, top-k sorted descending (ties to the
    lower expert id), optional renormalisation, scaling (DeepSeek routed_scaling_factor).
    Ranking uses the logits (softmax is monotone), so ids do not depend on exp().
    Returns (weights float32 [T, k], ids int32 [T, k])."""
    lg = np.asarray(logits, np.float32)
    T, E = lg.shape
    order = np.lexsort((np.broadcast_to(np.arange(E), (T, E)), -lg), axis=-1)[:, :top_k]
    m = lg.max(axis=1, keepdims=True)
    e = np.exp((lg - m).astype(np.float64))
    p = (e / e.sum(axis=1, keepdims=True)).astype(np.float32)
    w = np.take_along_axis(p, order, axis=1)
    if renormalize:
        w = (w / w.sum(axis=1, keepdims=True)).astype(np.float32)
    w = (w * np.float32(scaling)).astype(np.float32)
    return w, order.astype(np.int32)


def permute(ids, num_experts: int):
    """Expert-major, pair-index-ascending order of the T*k (token, slot) pairs
    (llama-cpp-port/patches/0001:96-110: experts ascending, tokens ascending).
    Returns (offsets int32 [E+1], perm int32 [T*k] pair index, inv int32 [T*k] position)."""
    ids = np.asarray(ids, np.int64).reshape(-1)
    counts = np.bincount(ids, minlength=num_experts)
    offsets = np.zeros(num_experts + 1, np.int32)
    offsets[1:] = np.cumsum(counts)
    perm = np.argsort(ids, kind="stable").astype(np.int32)
    inv = np.empty_like(perm)
    inv[perm] = np.arange(perm.size, dtype=np.int32)
    return offsets, perm, inv


def silu_mul_f32(g, u) -> np.ndarray:
    g = np.asarray(g, np.float32)
    return (g / (np.float32(1) + np.exp(-g)) * np.asarray(u, np.float32)).astype(np.float32)


def moe_layer(x_bf16, ids, weights, w13_f32, w2_f32, shared=None, act_round_bf16: bool = True,
              shared_w=None, blas_dtype=np.float64):
    """fp32 restatement of the fused-MoE apply (vllm_lut/quant_method.py:230-279,
    vllm_lut/fast_moe.py:30-80) with float64 accumulation:
      gu = x @ W13[e]^T ; a = silu(gu[:, :I]) * gu[:, I:] (fp32) ; a -> bf16 (the input
      dtype of the down projection, as the reference's lut_gemv/F.linear take bf16);
      y = a @ W2[e]^T ; out[t] = sum_k w[t,k] * y_{e_k}[t]  (+ shared experts, weight 1).
    w13_f32 / w2_f32: callables e -> float32 dequantised matrices [2I, H] / [H, I].
    shared: list of matrix pairs (w13, w2) for always-on experts (customized/deepseek.py:111-115).
    shared_w: None (every shared expert with weight 1) or float [T] per-token weights of the
    shared experts (Qwen's sigmoid(x . g), customized/qwen.py:99-100).
    w2_f32 may return a subset of W2's rows (output columns): the result then has that
    many columns.
    blas_dtype: the dtype of the down projection's product (float64 by default; float32 for
    full-shape prefill checks: its sums of a few thousand products carry a relative error
    near 1e-6, far below the 1e-3 bar).  The gate/up product stays float64 whatever
    blas_dtype is: its result is rounded to bf16, and a float32 sum flips enough of those
    roundings to move the output by about 3e-4 of its range.  Results accumulate in float64.
    Returns float64 [T, H] (or [T, rows of the W2 given])."""
    x = bf16_to_f32(x_bf16).astype(np.float64)
    ids = np.asarray(ids, np.int64)
    wts = np.asarray(weights, np.float32)
    T = x.shape[0]
    out = None

    def expert(rows, W13, W2):
        gu = x[rows] @ W13.astype(np.float64).T
        I = W13.shape[0] // 2
        a = silu_mul_f32(gu[:, :I].astype(np.float32), gu[:, I:].astype(np.float32))
        if act_round_bf16:
            a = bf16_to_f32(f32_to_bf16(a))
        return (a.astype(blas_dtype) @ W2.astype(blas_dtype, copy=False).T).astype(np.float64)

    def acc(rows, y):
        # a token listing an expert twice adds both pairs, as the reference's loop
        # over the k slots does (vllm_lut/fast_moe.py:58-61)
        nonlocal out
        if out is None:
            out = np.zeros((T, y.shape[1]), np.float64)
        if np.unique(rows).size == rows.size:
            out[rows] += y
        else:
            np.add.at(out, rows, y)

    for e in np.unique(ids):
        tok, slot = np.nonzero(ids == e)
        y = expert(tok, w13_f32(int(e)), w2_f32(int(e)))
        acc(tok, wts[tok, slot][:, None].astype(np.float64) * y)
    sw = None if shared_w is None else np.asarray(shared_w, np.float64).reshape(T, 1)
    for (W13, W2) in (shared or []):
        y = expert(np.arange(T), W13, W2)
        acc(np.arange(T), y if sw is None else sw * y)
    if out is None:
        out = np.zeros((T, x.shape[1]), np.float64)
    return out
