"""The C ABI on the CPU: the library loads, exports every function declared in
include/lutmoe.h, and rejects invalid calls with its error codes before any
HIP call (no kernel is launched here)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "lutmoe.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?(?:int|void|size_t|char)\s*\**\s*(\w+)\s*\(",
                                 text, flags=re.M)))


@pytest.fixture(scope="module")
def lib():
    from block_lut_amd import _native as N
    return N.lib()


def test_header_declares_the_expected_surface():
    names = declared_functions()
    for must in ("launch_blocklut_decompress", "launch_batch_blocklut_decompress",
                 "lut_moe_launch_blocklut_recover", "lut_moe_launch_unpack_4bit",
                 "launch_lut_gemv_kernel", "lutmoe_ref_gemv", "lutmoe_dequant", "lutmoe_gemv",
                 "lutmoe_route_topk", "lutmoe_permute", "lutmoe_moe_forward",
                 "lutmoe_moe_forward_logits", "lutmoe_moe_workspace_size", "lutmoe_strerror",
                 "lutmoe_bl4_encode", "lutmoe_ref_encode", "lutmoe_merge_bitplane",
                 "lutmoe_nested_group_planes", "lutmoe_ref_quantize"):
        assert must in names


def test_every_declared_symbol_is_exported_and_bound(lib):
    from block_lut_amd import _native as N
    for name in declared_functions():
        assert hasattr(lib, name), f"{name} not exported by liblutmoe.so"
        assert name in N.PROTOTYPES, f"{name} has no ctypes prototype"


def test_strerror(lib):
    from block_lut_amd import _native as N
    assert lib.lutmoe_strerror(N.LUTMOE_OK) == b"ok"
    assert b"invalid" in lib.lutmoe_strerror(N.LUTMOE_EINVAL)
    assert b"workspace" in lib.lutmoe_strerror(N.LUTMOE_EWORKSPACE)
    assert lib.lutmoe_strerror(-99) == b"unknown error"


def _bl4_weights(N, E=2, M=128, K=256, codes=0x10000, tables=0x20000):
    w = N.lutmoe_weights()
    w.format, w.num_experts, w.rows, w.cols = N.FMT_BL4, E, M, K
    w.codes, w.tables = codes, tables
    w.block_size = 64
    return w


def _desc(N, H=256, I=128, E=4, S=0, fmt=None):
    d = N.lutmoe_moe_desc()
    d.w13 = _bl4_weights(N, E + S, 2 * I, H)
    d.w2 = _bl4_weights(N, E + S, H, I)
    if fmt is not None:
        d.w13.format = fmt
        d.w2.format = fmt
    d.hidden, d.inter, d.num_routed, d.num_shared = H, I, E, S
    return d


def test_validation_before_any_hip_call(lib):
    from block_lut_amd import _native as N
    P = ctypes.c_void_p
    # null descriptors / pointers
    assert lib.lutmoe_gemv(None, 0, P(0x100), 1, P(0x100), 0, None) == N.LUTMOE_EINVAL
    assert lib.lutmoe_dequant(None, 0, 1, P(0x100), None) == N.LUTMOE_EINVAL
    w = _bl4_weights(N)
    w.cols = 100                                   # K not a multiple of 64
    assert lib.lutmoe_dequant(ctypes.byref(w), 0, 1, P(0x100), None) == N.LUTMOE_EINVAL
    w = _bl4_weights(N, codes=0x10004)             # misaligned codes
    assert lib.lutmoe_gemv(ctypes.byref(w), 0, P(0x100), 1, P(0x100), 0, None) == N.LUTMOE_EALIGN
    w = _bl4_weights(N)
    assert lib.lutmoe_gemv(ctypes.byref(w), 5, P(0x100), 1, P(0x100), 0, None) == N.LUTMOE_EINVAL
    assert lib.lutmoe_gemv(ctypes.byref(w), 0, P(0x100), 1, P(0x100), 7, None) == N.LUTMOE_EINVAL
    w.format = 9
    assert lib.lutmoe_dequant(ctypes.byref(w), 0, 1, P(0x100), None) == N.LUTMOE_EINVAL
    # routing
    assert lib.lutmoe_route_topk(P(0x100), 4, 8, 9, 0, 1.0, P(0x100), P(0x100), None) == N.LUTMOE_EINVAL
    assert lib.lutmoe_route_topk(P(0x100), 4, 8, 0, 0, 1.0, P(0x100), P(0x100), None) == N.LUTMOE_EINVAL
    assert lib.lutmoe_permute(None, 4, 2, 8, P(1), P(1), P(1), P(1), None) == N.LUTMOE_EINVAL
    # the general top-k kernel keeps one bit per held logit in 64 bits: E <= 4096
    assert lib.lutmoe_route_topk(P(0x100), 4, 4097, 2, 0, 1.0, P(0x100), P(0x100), None) == N.LUTMOE_EUNSUPPORTED
    assert lib.lutmoe_route_topk(P(0x100), 0, 4097, 2, 0, 1.0, P(0x100), P(0x100), None) == N.LUTMOE_EUNSUPPORTED
    # router gate: H % 8, 16-byte alignment, pointers, T range
    assert lib.lutmoe_router_logits(P(0x100), P(0x100), 2, 100, 8, P(0x100), 0, None) == N.LUTMOE_EINVAL
    assert lib.lutmoe_router_logits(P(0x108), P(0x100), 2, 64, 8, P(0x100), 0, None) == N.LUTMOE_EALIGN
    assert lib.lutmoe_router_logits(P(0x100), None, 2, 64, 8, P(0x100), 0, None) == N.LUTMOE_EINVAL
    assert lib.lutmoe_router_logits(P(0x100), P(0x100), 70000, 64, 8, P(0x100), 0, None) == N.LUTMOE_EINVAL
    assert lib.lutmoe_router_logits(None, None, 0, 64, 8, None, 0, None) == N.LUTMOE_OK
    # fused_lut_gemv: the arguments of lutmoe_ref_gemv
    assert lib.lutmoe_fused_lut_gemv(P(1), P(1), P(1), P(1), P(1), 0, 64, 1, 1, 128, 0, None) == N.LUTMOE_EINVAL
    assert lib.lutmoe_fused_lut_gemv(P(1), P(1), P(1), P(1), P(1), 4, 64, 1, 1, 128, 5, None) == N.LUTMOE_EINVAL
    assert lib.lutmoe_fused_lut_gemv(None, P(1), P(1), P(1), P(1), 4, 64, 1, 1, 128, 0, None) == N.LUTMOE_EINVAL
    assert lib.lutmoe_fused_lut_gemv(P(1), P(1), P(1), P(1), P(1), 4, 64, 0, 1, 128, 0, None) == N.LUTMOE_OK
    # reference-compatible entry points
    assert lib.launch_blocklut_decompress(P(0x100), P(0x100), P(0x100), P(0x100), -1, 128, None) == -1
    assert lib.launch_blocklut_decompress(P(0x100), P(0x100), P(0x100), P(0x100), 16, 0, None) == -1
    assert lib.launch_blocklut_decompress(None, None, None, None, 0, 128, None) == 0
    assert lib.launch_batch_blocklut_decompress(P(1), P(1), P(1), P(1), 2, 1000, 3, 128, None) == -1
    lib.lut_moe_launch_unpack_4bit(P(0x100), 7, None)
    assert b"invalid" in lib.lutmoe_last_error()
    lib.lut_moe_launch_unpack_4bit(P(0x100), 0, None)
    assert lib.lutmoe_last_error() == b""
    lib.launch_lut_gemv_kernel(None, None, None, None, None, 4, 4, 1)
    assert b"invalid" in lib.lutmoe_last_error()
    assert lib.lutmoe_unpack_6bit(P(1), P(1), 6, None) == N.LUTMOE_EINVAL
    assert lib.lutmoe_bl4_encode(P(1), 4, 0, P(1), P(1), None) == N.LUTMOE_EINVAL
    assert lib.lutmoe_bl4_tables_from_f16(P(0x104), P(0x100), 8, None) == N.LUTMOE_EALIGN
    # bit-plane packing: n a multiple of 4
    assert lib.lutmoe_pack_bitplanes(P(1), 6, P(1), None) == N.LUTMOE_EINVAL
    assert lib.lutmoe_pack_bitplanes(None, 8, P(1), None) == N.LUTMOE_EINVAL
    assert lib.lutmoe_pack_bitplanes(None, 0, None, None) == N.LUTMOE_OK
    # REF quantize rules: dtype, rule, entry count, pointers, alignment
    q = lib.lutmoe_ref_quantize
    assert q(P(0x100), 7, P(0x200), 256, 128, 128, 0, P(0x300), P(0x400), None) == N.LUTMOE_EINVAL
    assert q(P(0x100), 0, P(0x200), 256, 128, 128, 2, P(0x300), P(0x400), None) == N.LUTMOE_EINVAL
    assert q(P(0x100), 0, P(0x200), 257, 128, 128, 0, P(0x300), P(0x400), None) == N.LUTMOE_EINVAL
    assert q(P(0x100), 0, P(0x200), 1, 128, 128, 1, P(0x300), P(0x400), None) == N.LUTMOE_EINVAL
    assert q(P(0x100), 0, P(0x200), 256, 128, 0, 0, P(0x300), P(0x400), None) == N.LUTMOE_EINVAL
    assert q(None, 0, P(0x200), 256, 128, 128, 0, P(0x300), P(0x400), None) == N.LUTMOE_EINVAL
    assert q(P(0x102), 1, P(0x200), 256, 128, 128, 0, P(0x300), P(0x400), None) == N.LUTMOE_EALIGN
    assert q(P(0x101), 0, P(0x200), 256, 128, 128, 0, P(0x300), P(0x400), None) == N.LUTMOE_EALIGN
    assert q(None, 0, None, 256, 0, 128, 1, None, None, None) == N.LUTMOE_OK
    # nested plane grouping: n % 64 == 0, tier 2..4, pointers, 4-byte alignment
    assert lib.lutmoe_nested_group_planes(P(0x100), 4, 96, P(0x200), None) == N.LUTMOE_EINVAL
    assert lib.lutmoe_nested_group_planes(P(0x100), 5, 128, P(0x200), None) == N.LUTMOE_EINVAL
    assert lib.lutmoe_nested_group_planes(P(0x100), 1, 128, P(0x200), None) == N.LUTMOE_EINVAL
    assert lib.lutmoe_nested_group_planes(None, 3, 128, P(0x200), None) == N.LUTMOE_EINVAL
    assert lib.lutmoe_nested_group_planes(P(0x102), 3, 128, P(0x200), None) == N.LUTMOE_EALIGN
    assert lib.lutmoe_nested_group_planes(P(0x100), 3, 128, P(0x201), None) == N.LUTMOE_EALIGN
    assert lib.lutmoe_nested_group_planes(None, 2, 0, None, None) == N.LUTMOE_OK
    # 1-D k-means: 1 <= k <= 256, n >= 1, n_iter >= 0, pointers
    assert lib.lutmoe_kmeans_1d(P(1), 10, P(1), 0, 3, P(1), None) == N.LUTMOE_EINVAL
    assert lib.lutmoe_kmeans_1d(P(1), 10, P(1), 257, 3, P(1), None) == N.LUTMOE_EINVAL
    assert lib.lutmoe_kmeans_1d(P(1), 0, P(1), 16, 3, P(1), None) == N.LUTMOE_EINVAL
    assert lib.lutmoe_kmeans_1d(P(1), 10, P(1), 16, -1, P(1), None) == N.LUTMOE_EINVAL
    assert lib.lutmoe_kmeans_1d(P(1), 10, None, 16, 3, P(1), None) == N.LUTMOE_EINVAL
    # tier upgrade: n a multiple of 4, shift even in [0, 6], pointers unless n == 0
    assert lib.lutmoe_merge_bitplane(P(1), P(1), 6, 4, None) == N.LUTMOE_EINVAL
    assert lib.lutmoe_merge_bitplane(P(1), P(1), 8, 5, None) == N.LUTMOE_EINVAL
    assert lib.lutmoe_merge_bitplane(P(1), P(1), 8, 8, None) == N.LUTMOE_EINVAL
    assert lib.lutmoe_merge_bitplane(None, P(1), 8, 4, None) == N.LUTMOE_EINVAL
    assert lib.lutmoe_merge_bitplane(None, None, 0, 4, None) == N.LUTMOE_OK
    # REF codebook stride: 0 (shared) or at least one 256-entry codebook per expert
    w = _bl4_weights(N)
    w.format, w.codebook, w.absmax_per_expert, w.block_size = N.FMT_REF, 0x30000, 256, 128
    w.codebook_stride = 100
    assert lib.lutmoe_dequant(ctypes.byref(w), 0, 1, P(0x100), None) == N.LUTMOE_EINVAL
    w.codebook_stride = -256
    assert lib.lutmoe_dequant(ctypes.byref(w), 0, 1, P(0x100), None) == N.LUTMOE_EINVAL


def test_moe_validation(lib):
    from block_lut_amd import _native as N
    P = ctypes.c_void_p
    ws = P(0x100000)
    args = lambda d, T=4, k=2, out_dtype=0, wsb=1 << 30, path=0: (
        ctypes.byref(d), P(0x1000), P(0x2000), P(0x3000), T, k, P(0x4000), out_dtype, ws, wsb,
        path, None)
    d = _desc(N)
    d.w2.rows = 100                                           # inconsistent shapes
    assert lib.lutmoe_moe_forward(*args(d)) == N.LUTMOE_EINVAL
    d = _desc(N, H=256 + 64, I=100)                           # I % 64
    d.w13.cols = 320
    assert lib.lutmoe_moe_forward(*args(d)) in (N.LUTMOE_EINVAL, N.LUTMOE_EUNSUPPORTED)
    d = _desc(N)
    assert lib.lutmoe_moe_forward(*args(d, k=5)) == N.LUTMOE_EINVAL        # k > E
    assert lib.lutmoe_moe_forward(*args(d, out_dtype=3)) == N.LUTMOE_EINVAL
    assert lib.lutmoe_moe_forward(*args(d, path=3)) == N.LUTMOE_EINVAL
    assert lib.lutmoe_moe_forward(*args(d, wsb=16)) == N.LUTMOE_EWORKSPACE
    d = _desc(N, fmt=N.FMT_NESTED)                            # nested without tier bits
    assert lib.lutmoe_moe_forward(*args(d)) == N.LUTMOE_EINVAL
    d.w13.tier_bits = 1
    d.w2.tier_bits = 1
    d.w2.format = N.FMT_BL4                                   # mixed formats
    assert lib.lutmoe_moe_forward(*args(d)) == N.LUTMOE_EUNSUPPORTED
    d.w2.format = N.FMT_NESTED                                # nested, GEMV forced past its limits
    assert lib.lutmoe_moe_forward(*args(d, T=300, path=1)) == N.LUTMOE_EUNSUPPORTED
    d = _desc(N)
    d.w2.num_experts = 3                                      # fewer than routed + shared
    assert lib.lutmoe_moe_forward(*args(d)) == N.LUTMOE_EINVAL
    d = _desc(N)
    assert lib.lutmoe_moe_forward(*args(d, T=0)) == N.LUTMOE_OK           # empty batch
    assert lib.lutmoe_moe_forward_stages(*args(d)[:11], 0, None) == N.LUTMOE_EINVAL
    assert lib.lutmoe_moe_forward_logits(ctypes.byref(d), P(0x1000), None, 4, 2, 0, 1.0,
                                         P(0x4000), 0, ws, 1 << 30, 0, 7, None) == N.LUTMOE_EINVAL


def test_workspace_size_grows_with_tokens(lib):
    from block_lut_amd import _native as N
    d = _desc(N, H=2048, I=1408, E=64, S=2)
    small = lib.lutmoe_moe_workspace_size(ctypes.byref(d), 1, 6)
    big = lib.lutmoe_moe_workspace_size(ctypes.byref(d), 2048, 6)
    assert 0 < small < big
    # prefill workspace holds act [P][I] bf16 and y [P][H] fp32 for P = T*(k+S)
    assert big >= 2048 * 8 * (1408 * 2 + 2048 * 4)
    assert lib.lutmoe_moe_workspace_size(None, 1, 1) == 0
