"""block_lut_amd: MI355X (gfx950) LUT-dequant MoE expert compute.

Hand-written HIP kernels behind a C ABI (include/lutmoe.h, liblutmoe.so):
decode LUT-GEMV, prefill grouped LUT-GEMM on MFMA, token routing /
permutation / combine, dequantisation and the BL4 k-means encoder.  The
Python modules mirror the reference's LUT quant-method / fused-MoE interface
(LUTConfig, LUTFusedMoEMethod, fused_lut_moe, lut_gemv, decompress_blocklut,
LutDecompressor).
"""
__version__ = "0.1.0"
