"""ctypes binding of liblutmoe.so (the C ABI declared in include/lutmoe.h).

The library is built in-tree by ``block_lut_amd.csrc.build`` (or
``__graft_entry__.build()``).  There is no fallback: if the library is
missing, every entry point raises ``LutMoeNotBuilt``.
"""
from __future__ import annotations

import ctypes
import os
import threading

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liblutmoe.so")

LUTMOE_OK = 0
LUTMOE_EINVAL = -1
LUTMOE_EUNSUPPORTED = -2
LUTMOE_EHIP = -3
LUTMOE_EWORKSPACE = -4
LUTMOE_EALIGN = -5

FMT_REF = 0
FMT_BL4 = 1
FMT_NESTED = 2

QRULE_QUANTIZER = 0
QRULE_MIDPOINTS = 1

STAGE_ROUTE = 1
STAGE_GATE_UP = 2
STAGE_DOWN = 4
STAGE_ALL = 7

DTYPE_BF16 = 0
DTYPE_F32 = 1


class LutMoeNotBuilt(RuntimeError):
    pass


class LutMoeError(RuntimeError):
    def __init__(self, fn: str, code: int, text: str):
        super().__init__(f"{fn} failed: {text} (code {code})")
        self.code = code


class lutmoe_weights(ctypes.Structure):
    _fields_ = [
        ("format", ctypes.c_int32),
        ("num_experts", ctypes.c_int32),
        ("rows", ctypes.c_int32),
        ("cols", ctypes.c_int32),
        ("codes", ctypes.c_void_p),
        ("tables", ctypes.c_void_p),
        ("codebook", ctypes.c_void_p),
        ("tier_bits", ctypes.c_void_p),
        ("absmax_per_expert", ctypes.c_int64),
        ("block_size", ctypes.c_int32),
        ("codebook_stride", ctypes.c_int32),
    ]


class lutmoe_moe_desc(ctypes.Structure):
    _fields_ = [
        ("w13", lutmoe_weights),
        ("w2", lutmoe_weights),
        ("hidden", ctypes.c_int32),
        ("inter", ctypes.c_int32),
        ("num_routed", ctypes.c_int32),
        ("num_shared", ctypes.c_int32),
        ("shared_gate", ctypes.c_void_p),
        ("dense_inter", ctypes.c_int32),
        ("dense_reserved", ctypes.c_int32),
        ("dense_w13", ctypes.c_void_p),
        ("dense_w2", ctypes.c_void_p),
    ]


P = ctypes.c_void_p
I32 = ctypes.c_int
I64 = ctypes.c_int64
F32 = ctypes.c_float
SZ = ctypes.c_size_t
WP = ctypes.POINTER(lutmoe_weights)
DP = ctypes.POINTER(lutmoe_moe_desc)

# name -> (restype, argtypes)
PROTOTYPES = {
    "lutmoe_strerror": (ctypes.c_char_p, [I32]),
    "lutmoe_version": (ctypes.c_char_p, []),
    "lutmoe_last_error": (ctypes.c_char_p, []),
    "launch_blocklut_decompress": (I32, [P, P, P, P, I32, I32, P]),
    "launch_batch_blocklut_decompress": (I32, [P, P, P, P, I32, I32, I32, I32, P]),
    "lut_moe_launch_blocklut_recover": (None, [P, P, P, P, SZ, P]),
    "lut_moe_launch_unpack_4bit": (None, [P, SZ, P]),
    "launch_lut_gemv_kernel": (None, [P, P, P, P, P, I32, I32, I32]),
    "lutmoe_ref_gemv": (I32, [P, P, P, P, P, I32, I32, I32, I32, I32, I32, P]),
    "lutmoe_fused_lut_gemv": (I32, [P, P, P, P, P, I32, I32, I32, I32, I32, I32, P]),
    "lutmoe_router_logits": (I32, [P, P, I32, I32, I32, P, I32, P]),
    "lutmoe_unpack_6bit": (I32, [P, P, I64, P]),
    "lutmoe_merge_bitplane": (I32, [P, P, I64, I32, P]),
    "lutmoe_kmeans_1d": (I32, [P, I64, P, I32, I32, P, P]),
    "lutmoe_pack_bitplanes": (I32, [P, I64, P, P]),
    "lutmoe_nested_group_planes": (I32, [P, I32, I64, P, P]),
    "lutmoe_ref_quantize": (I32, [P, I32, P, I32, I64, I32, I32, P, P, P]),
    "lutmoe_dequant": (I32, [WP, I32, I32, P, P]),
    "lutmoe_gemv": (I32, [WP, I32, P, I32, P, I32, P]),
    "lutmoe_gemv_ex": (I32, [WP, I32, P, I32, I32, P, I32, P]),
    "lutmoe_bl4_tables_from_f16": (I32, [P, P, I64, P]),
    "lutmoe_decode_stream_probe_sink_words": (SZ, [DP, I32, I32]),
    "lutmoe_decode_stream_probe": (I32, [DP, P, I32, I32, P, P]),
    "lutmoe_route_topk": (I32, [P, I32, I32, I32, I32, F32, P, P, P]),
    "lutmoe_permute": (I32, [P, I32, I32, I32, P, P, P, P, P]),
    "lutmoe_moe_workspace_size": (SZ, [DP, I32, I32]),
    "lutmoe_moe_forward": (I32, [DP, P, P, P, I32, I32, P, I32, P, SZ, I32, P]),
    "lutmoe_moe_forward_stages": (I32, [DP, P, P, P, I32, I32, P, I32, P, SZ, I32, I32, P]),
    "lutmoe_moe_forward_logits": (I32, [DP, P, P, I32, I32, I32, F32, P, I32, P, SZ, I32, I32, P]),
    "lutmoe_moe_forward_noalloc": (I32, [DP, P, P, P, I32, I32, P, I32, I32, P]),
    "lutmoe_noalloc_prepare": (I32, []),
    "lutmoe_bl4_encode": (I32, [P, I64, I32, P, P, P]),
    "lutmoe_ref_encode": (I32, [P, P, I64, I32, P, P, P]),
}

_lib = None
_lock = threading.Lock()


def lib():
    """Load liblutmoe.so (raises LutMoeNotBuilt when absent)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise LutMoeNotBuilt(
                    f"{LIB_PATH} is missing: build it with `python -m block_lut_amd.csrc.build` "
                    "(there is no CPU fallback)")
            # torch's HIP runtime first: its libamdhip64 carries the soname
            # (libamdhip64.so.7) the library asks for, so both share one
            # runtime.  Loaded the other way round, the process holds two HIP
            # runtimes and device pointers of one are foreign to the other.
            import torch  # noqa: F401
            h = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in PROTOTYPES.items():
                f = getattr(h, name)
                f.restype = res
                f.argtypes = args
            _lib = h
    return _lib


def check(fn: str, rc: int) -> None:
    if rc != LUTMOE_OK:
        text = lib().lutmoe_strerror(rc).decode()
        if rc == LUTMOE_EHIP:
            detail = lib().lutmoe_last_error().decode()
            if "HIP runtime error: " in detail:
                text = detail[detail.index("HIP runtime error: "):]
        raise LutMoeError(fn, rc, text)


def check_last(fn: str) -> None:
    msg = lib().lutmoe_last_error().decode()
    if msg:
        raise LutMoeError(fn, -1, msg)
