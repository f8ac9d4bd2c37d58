"""CPU oracle for the LUT-dequant MoE expert path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import this package, and only to check results against (or, for the
CPU baseline, as the timed CPU restatement).  The product package
``block_lut_amd`` never imports it and fails loudly when its HIP library is
missing.

Contents: a numpy (and, where bit-exact sequential float order matters, C)
restatement of the reference's LUT arithmetic.  Every function cites the
reference file:line it follows.

Pinning status (how each function is checked; see tests/test_oracle_*.py):
  * f32->bf16 / f32->f16 rounding ........ numpy/torch casts on every 16-bit pattern
  * ref_quantize / ref_dequant ............ golden vectors written from the reference's
                                           quantizer.py (tests/golden/make_golden.py)
  * train_kmeans_ref, greedy_merge_ref,
    build_mapped_table_ref ............... golden vectors from quantizer.py
  * bitplane_pack_ref / unpack_4bit /
    unpack_6bit .......................... closed form + brute force over all 256 codes
  * nested_tables_prefix_pad /
    nested_tables_merge_map .............. the reference's shipped models/*/nested_lut_mapped*.npy
  * ref_gemv .............................. closed form vs float64 matmul of ref_dequant
  * bl4_* (no reference exists) .......... invariants: argmin optimality of every code,
                                           sorted tables, Lloyd fixed point, brute force
                                           k-means on tiny blocks, numpy float16 cast
  * nested_* (no reference exists) ....... invariants: partition refinement across tiers,
                                           tier-t reconstruction uses only the low t bits
  * route / permute ....................... brute force (argsort) + bijection invariants
  * moe_layer ............................. float64 dense restatement vs per-expert loop
"""
from .oracle import *  # noqa: F401,F403
