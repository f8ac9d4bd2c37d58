"""LUT-MoE configuration surface (vllm_lut/config.py:17-115): the code type
and tier fields with the reference's validation; the offload, cache and
prefetch fields of the reference belong to its SSD-offload runtime, which is
not part of this library."""
from __future__ import annotations

from dataclasses import dataclass


@dataclass
class LUT_MoE_vLLMConfig:
    code_type: str = "BLOCKLUT"     # 'BLOCKLUT' (8-bit), 'NESTEDLUT' (tiers), 'LUT'
    lut_path: str = ""
    lut_tier: int = 0               # 0 = full, 1 = mid, 2 = coarsest tier
    block_size: int = 128
    code_bits: int = 8              # 8: REF format, 4: BL4 format
    verbose: bool = False

    def __post_init__(self):
        if self.code_type not in ("LUT", "BLOCKLUT", "NESTEDLUT"):
            raise ValueError(f"Unsupported code_type: {self.code_type}. "
                             "Must be one of: LUT, BLOCKLUT, NESTEDLUT")
        if self.lut_tier not in (0, 1, 2):
            raise ValueError(f"lut_tier must be 0, 1, or 2, got {self.lut_tier}")
        if self.code_bits not in (4, 8):
            raise ValueError(f"code_bits must be 4 or 8, got {self.code_bits}")
