"""Device-resident random LUT weight stacks for the full-shape GPU tests.

The stacks are generated on the GPU (seeded torch generators: fast at every
configured shape) in their wire formats: BL4 codes + fp16 codebooks, REF codes
+ bf16 absmax + bf16 codebook, NestedLUT bit-plane sections + fp16 tier
tables.  The oracle side copies those inputs back and dequantises them on the
host (oracle.bl4_dequant_f32 / ref_dequant / nested_dequant_f32), so no value
the oracle uses was computed by a kernel under test.  Dequantised experts are
cached per stack: the full-shape tests touch each expert's matrices once.
"""
from __future__ import annotations

import numpy as np

import oracle as O


class DevBL4:
    """E BL4 matrices [M, K]: random codes, sorted N(0, std) fp16 codebooks."""

    def __init__(self, E, M, K, gen, device, std=0.02):
        import torch
        from block_lut_amd.formats import BL4Stack
        self.E, self.M, self.K = E, M, K
        self.codes = torch.randint(0, 256, (E, M, K // 2), dtype=torch.uint8, generator=gen, device=device)
        t = torch.randn((E, M, K // 64, 16), generator=gen, device=device) * std
        self.tabs = torch.sort(t, dim=-1).values.to(torch.float16)
        del t
        self.stack = BL4Stack.from_fp16(self.codes, self.tabs)
        self._cache = {}

    def host(self, e, rows=None):
        """float32 [M, K] (or the given rows) of expert e, dequantised on the host."""
        key = (e, None if rows is None else tuple(np.asarray(rows).tolist()))
        if key not in self._cache:
            c = self.codes[e].cpu().numpy()
            t = self.tabs[e].cpu().numpy().view(np.uint16)
            if rows is not None:
                c, t = c[rows], t[rows]
            self._cache[key] = O.bl4_dequant_f32(c, t)
        return self._cache[key]


class DevRef:
    """E REF matrices [M, K]: random uint8 codes, bf16 absmax per 128 elements,
    one sorted bf16[256] codebook."""

    def __init__(self, E, M, K, gen, device, block_size=128):
        import torch
        from block_lut_amd.formats import RefStack
        self.E, self.M, self.K, self.bs = E, M, K, block_size
        self.codes = torch.randint(0, 256, (E, M, K), dtype=torch.uint8, generator=gen, device=device)
        nb = -(-M * K // block_size)
        self.absmax = (torch.rand((E, nb), generator=gen, device=device) * 0.05 + 0.01).to(torch.bfloat16)
        self.cb = torch.sort(torch.randn(256, generator=gen, device=device)).values.to(torch.bfloat16)
        self.stack = RefStack(self.codes, self.absmax, self.cb, block_size)
        self._cache = {}
        self._cb_host = None

    def _inputs(self, e):
        import torch
        if self._cb_host is None:
            self._cb_host = self.cb.view(torch.int16).cpu().numpy().view(np.uint16)
        return (self.codes[e].cpu().numpy().reshape(-1),
                self.absmax[e].view(torch.int16).cpu().numpy().view(np.uint16), self._cb_host)

    def host(self, e):
        """Dequantised bf16(cb * absmax) weights as float32 [M, K]."""
        if ("deq", e) not in self._cache:
            c, a, cb = self._inputs(e)
            self._cache[("deq", e)] = O.bf16_to_f32(O.ref_dequant(c, a, cb, self.bs)).reshape(self.M, self.K)
        return self._cache[("deq", e)]

    def host_gemv(self, e):
        """The reference decode GEMV's unrounded f32(cb) * f32(absmax) weights."""
        if ("gemv", e) not in self._cache:
            c, a, cb = self._inputs(e)
            blk = np.minimum(np.arange(c.size) // self.bs, a.size - 1)
            w = O.bf16_to_f32(cb)[c] * O.bf16_to_f32(a)[blk]
            self._cache[("gemv", e)] = w.astype(np.float32).reshape(self.M, self.K)
        return self._cache[("gemv", e)]


class DevNested:
    """NestedLUT experts [M, K] at tiers bits[e]: random bit-plane sections and
    sorted N(0, std) fp16 tier tables (the device keeps their bf16 values)."""

    def __init__(self, bits, M, K, gen, device, std=0.02):
        import torch
        from block_lut_amd import _native as N
        from block_lut_amd.formats import NestedExpert, NestedStack
        self.bits = [int(b) for b in bits]
        self.E, self.M, self.K = len(self.bits), M, K
        n = M * K
        self.planes, self.tabs, ex = [], [], []
        for b in self.bits:
            size = n // 4 + (n // 8 if b >= 3 else 0) + (n // 8 if b >= 4 else 0)
            pl = torch.randint(0, 256, (size,), dtype=torch.uint8, generator=gen, device=device)
            t = torch.sort(torch.randn((M, K // 64, 1 << b), generator=gen, device=device) * std,
                           dim=-1).values.to(torch.float16)
            tb = torch.empty(t.shape, dtype=torch.bfloat16, device=device)
            N.check("lutmoe_bl4_tables_from_f16",
                    N.lib().lutmoe_bl4_tables_from_f16(t.data_ptr(), tb.data_ptr(), t.numel(),
                                                       torch.cuda.current_stream().cuda_stream))
            self.planes.append(pl)
            self.tabs.append(t)
            ex.append(NestedExpert(b, pl, tb))
        self.stack = NestedStack(ex, M, K)
        self._cache = {}

    def host(self, e):
        if e not in self._cache:
            b = self.bits[e]
            buf = self.planes[e].cpu().numpy()
            codes = O.nested_unpack_planes(O.nested_planes_split(buf, b, self.M, self.K), b)
            t = self.tabs[e].cpu().numpy().view(np.uint16)
            self._cache[e] = O.nested_dequant_f32(codes, t, b)
        return self._cache[e]
