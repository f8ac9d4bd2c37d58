"""GPU parity of the HIP kernels against the CPU oracle (seeded inputs).

Bar: bit-exact for codes, dequantised weights, routing ids and permutations;
GEMV / layer outputs (fp32 accumulation, fp32 output) within max-abs 1e-3
relative to the oracle's float64 result, i.e.
    max|y - y_ref| / max|y_ref| <= 1e-3.
"""
import numpy as np
import pytest

import oracle as O
from lutmoe_testutil import (BL4Expertset, NestedExpertset, RefExpertset, bf16_bits, golden_codebook,
                             rel_excess_bf16, rel_maxabs, to_dev_bf16, to_dev_f16)

pytestmark = pytest.mark.gpu
TOL = 1e-3


def _x(rng, T, K):
    return O.f32_to_bf16(rng.standard_normal((T, K)).astype(np.float32))


# ------------------------------------------------------------------ encoder

@pytest.mark.parametrize("M,K,n_iter", [(16, 768, 50), (64, 2048, 20)])
def test_bl4_encode_bitexact(gpu, M, K, n_iter):
    import torch
    from block_lut_amd import ops
    rng = np.random.default_rng(100 + M)
    w = (rng.standard_normal((M, K)) * 0.02).astype(np.float32)
    w[0, :64] = 0.0                       # degenerate block: all equal
    w[1, :64] = np.repeat(w[1, :16], 4)   # heavy duplicates
    codes, tables = ops.bl4_encode(torch.from_numpy(w).to(gpu), n_iter=n_iter)
    rc, rt = O.bl4_encode(w, n_iter=n_iter)
    torch.cuda.synchronize()
    assert np.array_equal(codes.cpu().numpy(), rc)
    assert np.array_equal(tables.cpu().numpy().view(np.uint16), rt)


# ------------------------------------------------------------------ dequant

def test_bl4_dequant_bitexact(gpu):
    from block_lut_amd import ops
    es = BL4Expertset(3, 96, 1408, seed=1)
    st = es.stack(gpu)
    got = bf16_bits(ops.dequant(st))
    for e in range(3):
        assert np.array_equal(got[e], O.bl4_dequant(es.codes[e], es.tables[e]))
    # table conversion alone: every fp16 pattern (incl. subnormals, inf, nan)
    import torch
    from block_lut_amd.formats import BL4Stack
    allh = np.arange(65536, dtype=np.uint16).reshape(1, 1, 64, 16 * 64)[..., :16 * 64]
    t = allh.reshape(1, 64, 64, 16)
    c = torch.zeros((1, 64, 2048), dtype=torch.uint8, device=gpu)
    st2 = BL4Stack.from_fp16(c, to_dev_f16(t, gpu))
    got_t = bf16_bits(st2.tables)
    assert np.array_equal(got_t, O.bl4_tables_bf16(t))


def test_ref_dequant_bitexact(gpu):
    import torch
    from block_lut_amd import ops
    rng = np.random.default_rng(2)
    cb = golden_codebook()
    for n, bs in ((4096, 128), (1000, 128), (2816 * 64, 128), (777, 64)):
        idx = rng.integers(0, 256, n, dtype=np.uint8)
        nb = -(-n // bs)
        am = O.f32_to_bf16(np.abs(rng.standard_normal(nb)).astype(np.float32) * 0.05)
        got = ops.blocklut_decompress(torch.from_numpy(idx).to(gpu), to_dev_bf16(am, gpu),
                                      to_dev_bf16(cb, gpu), bs)
        assert np.array_equal(bf16_bits(got), O.ref_dequant(idx, am, cb, bs)), (n, bs)
        if bs == 128:
            got2 = ops.blocklut_recover(torch.from_numpy(idx).to(gpu), to_dev_bf16(am, gpu),
                                        to_dev_bf16(cb, gpu))
            assert np.array_equal(bf16_bits(got2), O.ref_dequant(idx, am, cb, bs))


def test_ref_dequant_all_codes_all_scales(gpu):
    """Brute force: every code x a spread of absmax values (incl. zero, subnormal, large)."""
    import torch
    from block_lut_amd import ops
    cb = golden_codebook()
    scales = np.array([0.0, 1e-40, 1e-10, 3e-3, 0.02, 0.5, 1.0, 3.0, 1e4, 3e38], np.float32)
    am = O.f32_to_bf16(scales)
    idx = np.concatenate([np.roll(np.arange(256, dtype=np.uint8), s)[:128] for s in range(0, 20, 2)])
    got = ops.blocklut_decompress(torch.from_numpy(idx).to(gpu), to_dev_bf16(am, gpu),
                                  to_dev_bf16(cb, gpu), 128)
    assert np.array_equal(bf16_bits(got), O.ref_dequant(idx, am, cb, 128))


def test_ref_batch_decompress(gpu):
    import ctypes
    import torch
    from block_lut_amd import _native as N
    rng = np.random.default_rng(3)
    cb = golden_codebook()
    E, n, bs = 4, 5000, 128
    nb = -(-n // bs)
    idx = rng.integers(0, 256, (E, n), dtype=np.uint8)
    am = O.f32_to_bf16(np.abs(rng.standard_normal((E, nb))).astype(np.float32))
    out = torch.empty((E, n), dtype=torch.bfloat16, device=gpu)
    di = torch.from_numpy(idx).to(gpu)
    da = to_dev_bf16(am, gpu)
    dc = to_dev_bf16(cb, gpu)
    rc = N.lib().launch_batch_blocklut_decompress(out.data_ptr(), di.data_ptr(), da.data_ptr(),
                                                  dc.data_ptr(), E, n, nb, bs, None)
    assert rc == 0
    got = bf16_bits(out)
    for e in range(E):
        assert np.array_equal(got[e], O.ref_dequant(idx[e], am[e], cb, bs))


@pytest.mark.parametrize("n", [16, 8190, 8192, 8194, 100002, 5767168])
def test_unpack_4bit_inplace(gpu, n):
    import torch
    from block_lut_amd import ops
    rng = np.random.default_rng(n)
    codes = rng.integers(0, 256, n, dtype=np.uint8)
    packed = (codes[0::2] & 0x0F) | ((codes[1::2] & 0x0F) << 4)
    buf = torch.zeros(n, dtype=torch.uint8, device=gpu)
    buf[: n // 2] = torch.from_numpy(packed.astype(np.uint8)).to(gpu)
    ops.unpack_4bit_(buf, n)
    assert np.array_equal(buf.cpu().numpy(), O.unpack_4bit_ref(packed, n))


def test_unpack_6bit(gpu):
    import torch
    from block_lut_amd import ops
    rng = np.random.default_rng(6)
    n = 4096 * 3
    codes = rng.integers(0, 256, n, dtype=np.uint8)
    packed = O.bitplane_pack_ref(codes)
    got = ops.unpack_6bit(torch.from_numpy(packed).to(gpu), n)
    assert np.array_equal(got.cpu().numpy(), O.unpack_6bit_ref(packed, n))
    assert np.array_equal(got.cpu().numpy(), codes & 0x3F)


@pytest.mark.parametrize("n,off", [(4, 0), (20, 0), (4096 + 12, 0), (1 << 20, 0), (4096, 1), (8200, 3)])
def test_pack_bitplanes(gpu, n, off):
    """Bit-plane packing vs the oracle, bit-exact (odd offsets and sizes take the byte
    path), and the round trip through the GPU unpacks and the tier merges."""
    import torch
    from block_lut_amd import ops
    rng = np.random.default_rng(n * 3 + off)
    codes = rng.integers(0, 256, off + n, dtype=np.uint8)
    dc = torch.from_numpy(codes).to(gpu)[off:]
    got = ops.pack_bitplanes(dc)
    assert np.array_equal(got.cpu().numpy(), O.bitplane_pack_ref(codes[off:]))
    c6 = ops.unpack_6bit(got, n)
    assert np.array_equal(c6.cpu().numpy(), codes[off:] & 0x3F)
    ops.merge_bitplane_(c6, got[n // 2 + n // 4:], 6)
    assert np.array_equal(c6.cpu().numpy(), codes[off:])


@pytest.mark.parametrize("n,off", [(4, 0), (20, 0), (4096 + 12, 0), (1 << 20, 0), (4096, 1), (8200, 3)])
def test_merge_bitplane(gpu, n, off):
    """In-place merge of a 2-bit section at every shift vs the oracle, bit-exact; odd
    offsets take the byte path; the bytes around the codes stay untouched."""
    import torch
    from block_lut_amd import ops
    rng = np.random.default_rng(n + off)
    codes = rng.integers(0, 256, off + n + 16, dtype=np.uint8)
    plane = rng.integers(0, 256, off + n // 4 + 4, dtype=np.uint8)
    for shift in (0, 2, 4, 6):
        dc = torch.from_numpy(codes).to(gpu)
        dp = torch.from_numpy(plane).to(gpu)
        ops.merge_bitplane_(dc[off:off + n], dp[off:off + n // 4], shift)
        got = dc.cpu().numpy()
        assert np.array_equal(got[off:off + n], O.merge_bitplane_ref(codes[off:off + n], plane[off:off + n // 4], shift))
        assert np.array_equal(got[:off], codes[:off]) and np.array_equal(got[off + n:], codes[off + n:])


# --------------------------------------------------------------------- GEMV

@pytest.mark.parametrize("T", [1, 2, 3, 5])
def test_bl4_gemv_c1_shape(gpu, T):
    """Switch-base-8 expert FFN shape: W [3072, 768], 64-weight blocks."""
    import torch
    from block_lut_amd import ops
    es = BL4Expertset(1, 3072, 768, seed=0, n_iter=10)
    st = es.stack(gpu)
    rng = np.random.default_rng(1)
    xb = _x(rng, T, 768)
    y = ops.gemv(st, to_dev_bf16(xb, gpu), 0, out_dtype=torch.float32).cpu().numpy()
    ref = O.bf16_to_f32(xb).astype(np.float64) @ es.deq_f32(0).astype(np.float64).T
    assert rel_maxabs(y, ref) <= TOL


@pytest.mark.parametrize("fmt,T", [("bl4", 1), ("bl4", 3), ("ref", 1), ("ref", 2)])
def test_gemv_fp32_activations(gpu, fmt, T):
    """The switch-base-8 single linear at its configured precision: W [3072, 768] from
    N(0, 0.02) fp32, one (or a few) fp32 N(0, 1) activation rows, fp32 output; BL4 weights
    are the bf16 table entries, REF ones lut_gemv's unrounded cb * absmax products.  The
    fp32 path must see the activations' low mantissa bits: the same rows rounded to bf16
    give a clearly different result."""
    import torch
    from block_lut_amd import ops
    es = (BL4Expertset(1, 3072, 768, seed=0, n_iter=10) if fmt == "bl4" else RefExpertset(1, 3072, 768, seed=0))
    st = es.stack(gpu)
    rng = np.random.default_rng(1)
    x = rng.standard_normal((T, 768)).astype(np.float32)
    y = ops.gemv(st, torch.from_numpy(x).to(gpu), 0, out_dtype=torch.float32).cpu().numpy()
    wf = (es.deq_f32 if fmt == "bl4" else es.gemv_f32)(0).astype(np.float64)
    ref = x.astype(np.float64) @ wf.T
    assert rel_maxabs(y, ref) <= 1e-5
    ref_b = O.bf16_to_f32(O.f32_to_bf16(x)).astype(np.float64) @ wf.T
    assert rel_maxabs(ref_b, ref) > 20 * rel_maxabs(y, ref)


# ------------------------------------------------------------ NestedLUT

def test_nested_dequant_bitexact(gpu):
    """Tier-b dequant of the bit-plane sections, experts at tiers 2, 3, 4."""
    from block_lut_amd import ops
    es = NestedExpertset([2, 3, 4], 96, 640, seed=3)
    got = ops.dequant(es.stack(gpu))
    for e in range(es.E):
        assert np.array_equal(bf16_bits(got[e]), es.deq_bits(e)), f"expert {e} (tier {es.bits[e]})"


def test_nested_grouped_layout_bitexact(gpu):
    """The device order of NestedStack's codes (lutmoe_nested_group_planes)
    equals the oracle's regrouping of the plane sections, at every tier;
    keep_planes=False drops the plane tensors and keeps the codes."""
    import torch
    from block_lut_amd.formats import NestedExpert, NestedStack
    es = NestedExpertset([2, 3, 4], 64, 192, seed=5, n_iter=4)
    st = es.stack(gpu)
    for e, b in enumerate(es.bits):
        want = O.nested_group_planes(es.planes(e), b, es.M, es.K)
        assert np.array_equal(st.codes[e].cpu().numpy(), want), f"tier {b}"
    ex = [NestedExpert(b, torch.from_numpy(es.planes(e)).to(gpu), to_dev_bf16(es.table_bf16(e), gpu))
          for e, b in enumerate(es.bits)]
    st2 = NestedStack(ex, es.M, es.K, keep_planes=False)
    assert all(x.planes is None for x in st2.experts)
    for e in range(es.E):
        assert torch.equal(st2.codes[e], st.codes[e])


@pytest.mark.parametrize("bits,M,K,T", [(2, 2816, 2048, 1), (3, 2048, 1408, 1), (4, 2048, 1408, 2),
                                        (3, 300, 640, 5), (2, 40, 4160, 3)])
def test_nested_gemv(gpu, bits, M, K, T):
    """Single-matrix GEMV (lutmoe_gemv) on a tier-b expert, including K past
    one 2048-column pass and a row count that is not a multiple of 32."""
    import torch
    from block_lut_amd import ops
    es = NestedExpertset([4, bits], M, K, seed=M + K, n_iter=8)
    rng = np.random.default_rng(bits)
    xb = _x(rng, T, K)
    y = ops.gemv(es.stack(gpu), to_dev_bf16(xb, gpu), 1, out_dtype=torch.float32).cpu().numpy()
    ref = O.bf16_to_f32(xb).astype(np.float64) @ es.deq_f32(1).astype(np.float64).T
    assert rel_maxabs(y, ref) <= TOL


@pytest.mark.parametrize("T,path", [(1, 1), (2, 1), (4, 1), (9, 1), (40, 1), (150, 2), (5, 2)])
def test_moe_layer_nested_tiers(gpu, T, path):
    """MoE layer over NestedLUT experts of mixed tiers (decode GEMV and the
    grouped MFMA path): routed experts at tiers 2/3/4 and a tier-4 shared
    expert, against the dense restatement of the tier-b weights.  Decode
    passes: one token (T=1), two tokens with the routing in each wave (T=2),
    two tokens a pass and chunk (T=4, 9), four tokens a pass with one-token
    passes beside them (T=40)."""
    import torch
    from block_lut_amd import ops
    from block_lut_amd.formats import MoEWeights
    E, S, k, H, I = 6, 1, 2, 512, 320
    bits = [2, 3, 4, 2, 3, 4, 4]
    w13 = NestedExpertset(bits, 2 * I, H, seed=40 + T, n_iter=8)
    w2 = NestedExpertset(bits, H, I, seed=41 + T, n_iter=8)
    moe = MoEWeights(w13.stack(gpu), w2.stack(gpu), H, I, E, S)
    rng = np.random.default_rng(T)
    xb = _x(rng, T, H)
    lg = rng.standard_normal((T, E)).astype(np.float32)
    rw, rids = O.route(lg, k)
    out = ops.moe_forward(moe, to_dev_bf16(xb, gpu), torch.from_numpy(rw).to(gpu),
                          torch.from_numpy(rids).to(gpu), out_dtype=torch.float32, path=path)
    ref = O.moe_layer(xb, rids, rw, w13.deq_f32, w2.deq_f32,
                      shared=[(w13.deq_f32(E + s), w2.deq_f32(E + s)) for s in range(S)])
    assert rel_maxabs(out.cpu().numpy(), ref) <= TOL


@pytest.mark.parametrize("M,K,T", [(2816, 2048, 1), (2048, 1408, 1), (300, 640, 3)])
def test_ref_gemv(gpu, M, K, T):
    import torch
    from block_lut_amd import ops
    rng = np.random.default_rng(M + K)
    cb = golden_codebook()
    idx = rng.integers(0, 256, (M, K), dtype=np.uint8)
    nb = -(-M * K // 128)
    am = O.f32_to_bf16(np.abs(rng.standard_normal(nb)).astype(np.float32) * 0.02)
    xb = _x(rng, T, K)
    y = ops.ref_gemv(to_dev_bf16(xb, gpu), torch.from_numpy(idx).to(gpu), to_dev_bf16(cb, gpu),
                     to_dev_bf16(am, gpu), out_dtype=torch.float32).cpu().numpy()
    for t in range(T):
        ref = O.ref_gemv(xb[t], idx, cb, am)
        assert rel_maxabs(y[t], ref) <= TOL


def test_ref_gemv_generic_path(gpu):
    """K not a multiple of 8 and 100-element absmax blocks spanning rows."""
    import torch
    from block_lut_amd import ops
    rng = np.random.default_rng(9)
    cb = golden_codebook()
    M, K, bs = 37, 203, 100
    idx = rng.integers(0, 256, (M, K), dtype=np.uint8)
    nb = -(-M * K // bs)
    am = O.f32_to_bf16(np.abs(rng.standard_normal(nb)).astype(np.float32))
    xb = _x(rng, 1, K)
    y = ops.ref_gemv(to_dev_bf16(xb, gpu), torch.from_numpy(idx).to(gpu), to_dev_bf16(cb, gpu),
                     to_dev_bf16(am, gpu), block_size=bs, out_dtype=torch.float32)
    deq = O.bf16_to_f32(cb)[idx] * O.bf16_to_f32(am)[np.minimum(np.arange(M * K) // bs, nb - 1)].reshape(M, K)
    ref = deq.astype(np.float64) @ O.bf16_to_f32(xb[0]).astype(np.float64)
    assert rel_maxabs(y.cpu().numpy()[0], ref) <= TOL


def test_lut_gemv_reference_signature(gpu):
    """launch_lut_gemv_kernel: fp32 codebook, default stream, bf16 out."""
    import torch
    from block_lut_amd import _native as N
    rng = np.random.default_rng(10)
    cb = golden_codebook()
    M, K = 512, 1024
    idx = rng.integers(0, 256, (M, K), dtype=np.uint8)
    nb = M * K // 128
    am = O.f32_to_bf16(np.abs(rng.standard_normal(nb)).astype(np.float32) * 0.02)
    xb = _x(rng, 1, K)
    di = torch.from_numpy(idx).to(gpu)
    dcb = torch.from_numpy(O.bf16_to_f32(cb)).to(gpu)
    dx, da = to_dev_bf16(xb, gpu), to_dev_bf16(am, gpu)
    out = torch.empty(M, dtype=torch.bfloat16, device=gpu)
    torch.cuda.synchronize()
    N.lib().launch_lut_gemv_kernel(dx.data_ptr(), di.data_ptr(), dcb.data_ptr(), da.data_ptr(),
                                   out.data_ptr(), M, K, nb)
    N.check_last("launch_lut_gemv_kernel")
    torch.cuda.synchronize()
    ref = O.ref_gemv(xb[0], idx, cb, am)
    # bf16 output: one bf16 rounding of the fp32 sum on top of the tolerance
    assert rel_maxabs(O.bf16_to_f32(bf16_bits(out)), ref) <= TOL + 2.0 ** -8


# ------------------------------------------------------------------ routing

@pytest.mark.parametrize("T,E,k,renorm", [(1, 60, 4, False), (37, 64, 6, False), (513, 8, 2, True)])
def test_route_topk(gpu, T, E, k, renorm):
    import torch
    from block_lut_amd import ops
    rng = np.random.default_rng(T * E)
    lg = rng.standard_normal((T, E)).astype(np.float32)
    lg[0, :3] = 1.5                       # a tie: lower expert id first
    w, ids = ops.route_topk(torch.from_numpy(lg).to(gpu), k, renormalize=renorm)
    rw, rids = O.route(lg, k, renormalize=renorm)
    assert np.array_equal(ids.cpu().numpy(), rids)
    np.testing.assert_allclose(w.cpu().numpy(), rw, rtol=2e-6, atol=1e-7)


@pytest.mark.parametrize("E", [40, 100])
def test_route_topk_nan_rows(gpu, E):
    """Rows with fewer finite logits than k: NaN is never selected, and a round with only
    NaN left yields id -1 with weight 0, in the E <= 64 kernel and the general one alike."""
    import torch
    from block_lut_amd import ops
    T, k = 3, 4
    rng = np.random.default_rng(E)
    lg = rng.standard_normal((T, E)).astype(np.float32)
    lg[0, :] = np.nan
    lg[0, [5, E - 1]] = [0.5, 2.0]          # two finite logits of four picks
    lg[1, 3] = np.nan                       # a NaN among finite values
    w, ids = ops.route_topk(torch.from_numpy(lg).to(gpu), k)
    w, ids = w.cpu().numpy(), ids.cpu().numpy()
    assert list(ids[0]) == [E - 1, 5, -1, -1]
    assert np.all(w[0, 2:] == 0)      # (the softmax of a row holding NaN is NaN, as torch's)
    fin = np.where(np.isnan(lg), -np.inf, lg)
    for t in (1, 2):
        assert list(ids[t]) == list(np.argsort(-fin[t], kind="stable")[:k])
        assert 3 not in ids[1]


@pytest.mark.parametrize("T,k,E", [(1, 4, 60), (32, 4, 60), (2048, 8, 66), (300, 2, 8), (1000, 3, 300),
                                   (10, 2, 600)])
def test_permute(gpu, T, k, E):
    import torch
    from block_lut_amd import ops
    rng = np.random.default_rng(T + E)
    ids = np.stack([rng.permutation(E)[:k] for _ in range(T)]).astype(np.int32)
    off, perm, inv, act = [t.cpu().numpy() for t in ops.permute(torch.from_numpy(ids).to(gpu), E)]
    roff, rperm, rinv = O.permute(ids, E)
    assert np.array_equal(off, roff)
    assert np.array_equal(perm, rperm)
    assert np.array_equal(inv, rinv)
    nz = np.nonzero(np.diff(roff))[0]
    assert act[0] == nz.size and np.array_equal(act[1:1 + nz.size], nz)


def test_permute_drops_out_of_range(gpu):
    """Pairs whose expert id is outside [0, E) get inv = -1 and no position; the others keep
    the expert-major, pair-ascending order among themselves."""
    import torch
    from block_lut_amd import ops
    rng = np.random.default_rng(77)
    T, k, E = 700, 3, 10
    ids = rng.integers(-2, E + 2, size=(T, k)).astype(np.int32)
    off, perm, inv, act = [t.cpu().numpy() for t in ops.permute(torch.from_numpy(ids).to(gpu), E)]
    flat = ids.reshape(-1)
    valid = (flat >= 0) & (flat < E)
    assert np.all(inv[~valid] == -1)
    vi = np.nonzero(valid)[0]
    order = vi[np.argsort(flat[vi], kind="stable")]
    assert np.array_equal(perm[:order.size], order)
    assert np.array_equal(inv[order], np.arange(order.size))
    assert np.array_equal(off, np.concatenate([[0], np.cumsum(np.bincount(flat[vi], minlength=E))]))


# --------------------------------------------------------------- MoE layer

def _ref_semantics(w13, w2, T, path):
    """Weights of the reference's REF layer as the oracle sees them: one token takes
    lut_gemv's unrounded (x * cb) * absmax products (vllm_lut/quant_method.py:250-260),
    several tokens the dequantised bf16(cb * absmax) weights and a matmul (:261-277).  The
    grouped MFMA path (path 2) always computes with the dequantised weights."""
    if T == 1 and path != 2:
        return w13.gemv_f32, w2.gemv_f32
    return w13.deq_f32, w2.deq_f32


def _moe_case(fmt, E, S, H, I, seed):
    cls = BL4Expertset if fmt == "bl4" else RefExpertset
    w13 = cls(E + S, 2 * I, H, seed=seed)
    w2 = cls(E + S, H, I, seed=seed + 1)
    return w13, w2


@pytest.mark.parametrize("fmt,T,path", [("bl4", 1, 1), ("bl4", 2, 1), ("bl4", 4, 1), ("bl4", 9, 1),
                                        ("bl4", 40, 1), ("bl4", 200, 2), ("bl4", 5, 2),
                                        ("ref", 1, 1), ("ref", 2, 1), ("ref", 3, 1), ("ref", 9, 1),
                                        ("ref", 150, 2)])
def test_moe_layer(gpu, fmt, T, path):
    import torch
    from block_lut_amd import ops
    from block_lut_amd.formats import MoEWeights
    E, S, k, H, I = 8, 1, 2, 512, 320
    w13, w2 = _moe_case(fmt, E, S, H, I, seed=20 + T)
    moe = MoEWeights(w13.stack(gpu), w2.stack(gpu), H, I, E, S)
    rng = np.random.default_rng(T)
    xb = _x(rng, T, H)
    lg = rng.standard_normal((T, E)).astype(np.float32)
    rw, rids = O.route(lg, k)
    out = ops.moe_forward(moe, to_dev_bf16(xb, gpu), torch.from_numpy(rw).to(gpu),
                          torch.from_numpy(rids).to(gpu), out_dtype=torch.float32, path=path)
    # REF decode follows the reference's lut_gemv (unrounded cb*absmax products),
    # REF prefill its dequant-then-GEMM branch (bf16 weights); BL4 weights are the
    # bf16 table entries on both paths.
    f13, f2 = _ref_semantics(w13, w2, T, path) if fmt == "ref" else (w13.deq_f32, w2.deq_f32)
    ref = O.moe_layer(xb, rids, rw, f13, f2, shared=[(f13(E + s), f2(E + s)) for s in range(S)])
    assert rel_maxabs(out.cpu().numpy(), ref) <= TOL


@pytest.mark.parametrize("fmt,T,path", [("bl4", 1, 1), ("bl4", 2, 1), ("bl4", 3, 1), ("bl4", 3, 2),
                                        ("ref", 1, 1), ("ref", 2, 1), ("ref", 3, 1),
                                        ("nested", 1, 1), ("nested", 3, 1), ("nested", 3, 2)])
def test_moe_layer_repeated_ids(gpu, fmt, T, path):
    """Caller-given ids that list an expert twice for one token: both pairs count, each with
    its weight, as the reference's loop over the k slots adds them (vllm_lut/fast_moe.py:
    58-61).  One token takes the one-token kernels' fallback routing (a slot with two
    positions)."""
    import torch
    from block_lut_amd import ops
    from block_lut_amd.formats import MoEWeights
    E, S, k, H, I = 8, 1, 3, 512, 320
    if fmt == "nested":
        bits = [2, 3, 4, 2, 3, 4, 3, 2, 4]
        w13 = NestedExpertset(bits, 2 * I, H, seed=80 + T, n_iter=8)
        w2 = NestedExpertset(bits, H, I, seed=81 + T, n_iter=8)
    else:
        w13, w2 = _moe_case(fmt, E, S, H, I, seed=70 + T)
    moe = MoEWeights(w13.stack(gpu), w2.stack(gpu), H, I, E, S)
    rng = np.random.default_rng(700 + T)
    xb = _x(rng, T, H)
    rids = np.array([[5, 2, 5], [1, 1, 7], [3, 6, 3]], np.int32)[:T]
    rw = rng.uniform(0.1, 1.0, size=(T, k)).astype(np.float32)
    out = ops.moe_forward(moe, to_dev_bf16(xb, gpu), torch.from_numpy(rw).to(gpu),
                          torch.from_numpy(rids).to(gpu), out_dtype=torch.float32, path=path)
    f13, f2 = _ref_semantics(w13, w2, T, path) if fmt == "ref" else (w13.deq_f32, w2.deq_f32)
    ref = O.moe_layer(xb, rids, rw, f13, f2, shared=[(f13(E + s), f2(E + s)) for s in range(S)])
    assert rel_maxabs(out.cpu().numpy(), ref) <= TOL


@pytest.mark.parametrize("fmt,T", [("bl4", 16), ("bl4", 40), ("ref", 16), ("nested", 16), ("nested", 40)])
def test_moe_layer_skewed_routing(gpu, fmt, T):
    """Decode with one heavily routed expert: every token picks expert 0 plus k-1 others, so
    expert 0 holds T positions while the mean slot holds about 3, and the routing kernel
    cuts its slot into several work chunks (gate/up CTA rows, down y waves)."""
    import torch
    from block_lut_amd import ops
    from block_lut_amd.formats import MoEWeights
    E, S, k, H, I = 24, 0, 4, 256, 192
    if fmt == "nested":
        bits = [2, 3, 4] * (E // 3)
        w13 = NestedExpertset(bits, 2 * I, H, seed=90 + T, n_iter=8)
        w2 = NestedExpertset(bits, H, I, seed=91 + T, n_iter=8)
        f13, f2 = w13.deq_f32, w2.deq_f32
    else:
        w13, w2 = _moe_case(fmt, E, S, H, I, seed=90 + T)
        f13, f2 = _ref_semantics(w13, w2, T, 1) if fmt == "ref" else (w13.deq_f32, w2.deq_f32)
    moe = MoEWeights(w13.stack(gpu), w2.stack(gpu), H, I, E, S)
    rng = np.random.default_rng(900 + T)
    xb = _x(rng, T, H)
    rids = np.stack([np.concatenate([[0], 1 + rng.permutation(E - 1)[:k - 1]]) for _ in range(T)])
    rids = rids.astype(np.int64)
    rw = rng.random((T, k)).astype(np.float32)
    out = ops.moe_forward(moe, to_dev_bf16(xb, gpu), torch.from_numpy(rw).to(gpu),
                          torch.from_numpy(rids).to(gpu), out_dtype=torch.float32, path=1)
    ref = O.moe_layer(xb, rids, rw, f13, f2, shared=[])
    assert rel_maxabs(out.cpu().numpy(), ref) <= TOL


@pytest.mark.parametrize("T,path,out_bf16", [(3, 1, False), (40, 2, False), (40, 2, True)])
def test_moe_layer_max_slots(gpu, T, path, out_bf16):
    """k + shared experts = 16, the entry points' maximum: each token's 16 positions meet in
    the combine kernel (the prefill path's, and the decode path's from three tokens on),
    with some routed pairs dropped (id -1: no position, skipped by the combine).  The
    oracle takes a dropped pair as expert 0 at weight 0, which adds exactly nothing."""
    import torch
    from block_lut_amd import ops
    from block_lut_amd.formats import MoEWeights
    E, S, k, H, I = 24, 4, 12, 256, 192
    w13, w2 = _moe_case("bl4", E, S, H, I, seed=130 + T)
    moe = MoEWeights(w13.stack(gpu), w2.stack(gpu), H, I, E, S)
    rng = np.random.default_rng(1300 + T)
    xb = _x(rng, T, H)
    rids = np.stack([rng.permutation(E)[:k] for _ in range(T)]).astype(np.int32)
    rids[::3, 5] = -1                     # one dropped pair in every third token
    rids[1, [0, 7]] = -1                  # two in token 1
    rw = rng.uniform(0.05, 1.0, size=(T, k)).astype(np.float32)
    out = ops.moe_forward(moe, to_dev_bf16(xb, gpu), torch.from_numpy(rw).to(gpu),
                          torch.from_numpy(rids).to(gpu),
                          out_dtype=torch.bfloat16 if out_bf16 else torch.float32, path=path)
    keep = rids >= 0
    ref = O.moe_layer(xb, np.where(keep, rids, 0), np.where(keep, rw, 0.0).astype(np.float32),
                      w13.deq_f32, w2.deq_f32, shared=[(w13.deq_f32(E + s), w2.deq_f32(E + s)) for s in range(S)])
    if out_bf16:
        assert rel_excess_bf16(O.bf16_to_f32(bf16_bits(out)), ref) <= TOL
    else:
        assert rel_maxabs(out.cpu().numpy(), ref) <= TOL


@pytest.mark.parametrize("fmt", ["bl4", "ref", "nested"])
def test_prefill_skewed_routing_staged(gpu, fmt):
    """Prefill with very uneven tiles: every token picks expert 0 (one tile of 200 positions)
    and three others of a Zipf-like popularity (tiles of a few to ~60 positions), so the
    grouped GEMMs hand tiles out longest first from their launch counters and the tiles of
    at most 64 positions look their tables up in registers (BL4, NestedLUT).  Checked against
    the oracle; then the stages run one by one in one workspace, gate/up and down twice each
    after one routing (the counters are zeroed by the routing and by each launch's last CTA),
    equal to the one-call layer bit for bit."""
    import torch
    from block_lut_amd import _native as N
    from block_lut_amd import ops
    from block_lut_amd.formats import MoEWeights
    E, S, k, H, I, T = 24, 0, 4, 512, 320, 200
    if fmt == "nested":
        bits = [2, 3, 4] * (E // 3)
        w13 = NestedExpertset(bits, 2 * I, H, seed=130, n_iter=8)
        w2 = NestedExpertset(bits, H, I, seed=131, n_iter=8)
        f13, f2 = w13.deq_f32, w2.deq_f32
    else:
        w13, w2 = _moe_case(fmt, E, S, H, I, seed=130)
        f13, f2 = _ref_semantics(w13, w2, T, 2) if fmt == "ref" else (w13.deq_f32, w2.deq_f32)
    moe = MoEWeights(w13.stack(gpu), w2.stack(gpu), H, I, E, S)
    rng = np.random.default_rng(1300)
    xb = _x(rng, T, H)
    p = 1.0 / np.arange(1, E) ** 1.1
    p /= p.sum()
    rids = np.stack([np.concatenate([[0], 1 + rng.choice(E - 1, size=k - 1, replace=False, p=p)])
                     for _ in range(T)]).astype(np.int64)
    rw = rng.random((T, k)).astype(np.float32)
    counts = np.bincount(rids.ravel(), minlength=E)
    assert counts[0] == T and np.sum((counts > 0) & (counts <= 64)) >= E // 2
    args = (moe, to_dev_bf16(xb, gpu), torch.from_numpy(rw).to(gpu), torch.from_numpy(rids).to(gpu))
    full = ops.moe_forward(*args, out_dtype=torch.float32, path=2, workspace=ops.new_workspace(moe, T, k, gpu))
    ref = O.moe_layer(xb, rids, rw, f13, f2, shared=[])
    assert rel_maxabs(full.cpu().numpy(), ref) <= TOL
    ws = ops.new_workspace(moe, T, k, gpu)
    staged = torch.empty_like(full)
    ops.moe_forward(*args, out=staged, path=2, workspace=ws, stages=N.STAGE_ROUTE)
    for _ in range(2):
        ops.moe_forward(*args, out=staged, path=2, workspace=ws, stages=N.STAGE_GATE_UP)
    for _ in range(2):
        staged.zero_()
        ops.moe_forward(*args, out=staged, path=2, workspace=ws, stages=N.STAGE_DOWN)
        torch.cuda.synchronize()
        assert torch.equal(full, staged)


def test_prefill_many_experts(gpu):
    """More experts than the grouped GEMMs keep offsets of in LDS (1,100 routed + shared):
    the kernels read the offsets in place; checked against the oracle."""
    import torch
    from block_lut_amd import ops
    from block_lut_amd.formats import MoEWeights
    from block_lut_amd.formats import BL4Stack
    E, S, k, H, I, T = 1100, 1, 2, 256, 192, 96

    class RandomBL4:
        """Random codes and sorted random fp16 tables (no k-means: 1,101 experts)."""

        def __init__(self, M, K, seed):
            r = np.random.default_rng(seed)
            self.codes = r.integers(0, 256, (E + S, M, K // 2), dtype=np.uint8)
            t = np.sort(r.standard_normal((E + S, M, K // 64, 16)).astype(np.float32) * 0.02, axis=-1)
            self.tables = t.astype(np.float16).view(np.uint16)

        def deq_f32(self, e):
            return O.bf16_to_f32(O.bl4_dequant(self.codes[e], self.tables[e]))

        def stack(self, device):
            return BL4Stack.from_fp16(torch.from_numpy(self.codes).to(device), to_dev_f16(self.tables, device))

    w13, w2 = RandomBL4(2 * I, H, 140), RandomBL4(H, I, 141)
    moe = MoEWeights(w13.stack(gpu), w2.stack(gpu), H, I, E, S)
    rng = np.random.default_rng(1400)
    xb = _x(rng, T, H)
    rids = np.stack([rng.choice(E, size=k, replace=False) for _ in range(T)]).astype(np.int64)
    rids[: T // 2, 0] = 7   # one expert with many positions, the rest with one or none
    rw = rng.random((T, k)).astype(np.float32)
    out = ops.moe_forward(moe, to_dev_bf16(xb, gpu), torch.from_numpy(rw).to(gpu),
                          torch.from_numpy(rids).to(gpu), out_dtype=torch.float32, path=2)
    f13, f2 = w13.deq_f32, w2.deq_f32
    ref = O.moe_layer(xb, rids, rw, f13, f2, shared=[(f13(E + s), f2(E + s)) for s in range(S)])
    assert rel_maxabs(out.cpu().numpy(), ref) <= TOL


@pytest.mark.parametrize("block_size,T,path", [(64, 1, 1), (64, 9, 1), (192, 1, 1), (192, 9, 1), (256, 1, 1),
                                               (256, 9, 1), (64, 40, 2), (192, 40, 2), (256, 300, 2)])
def test_moe_layer_ref_block_sizes(gpu, block_size, T, path):
    """REF with absmax blocks of 64, 192 and 256 columns.  Decode (path 1) follows the
    reference GEMV's (x * cb) * absmax products (a lane's 32 aligned columns share one block;
    T=9 runs the down projection of every active expert in parallel, y + combine); prefill
    (path 2) the reference's dequantise-then-GEMM branch, bf16(cb * absmax) weights, with the
    absmax block of each 64-column K step picked per weight row."""
    import torch
    from block_lut_amd import ops
    from block_lut_amd.formats import MoEWeights
    E, S, k, H, I = 8, 1, 2, 256, 192
    w13 = RefExpertset(E + S, 2 * I, H, seed=30 + block_size, block_size=block_size)
    w2 = RefExpertset(E + S, H, I, seed=31 + block_size, block_size=block_size)
    moe = MoEWeights(w13.stack(gpu), w2.stack(gpu), H, I, E, S)
    rng = np.random.default_rng(block_size + T)
    xb = _x(rng, T, H)
    rw, rids = O.route(rng.standard_normal((T, E)).astype(np.float32), k)
    out = ops.moe_forward(moe, to_dev_bf16(xb, gpu), torch.from_numpy(rw).to(gpu),
                          torch.from_numpy(rids).to(gpu), out_dtype=torch.float32, path=path)
    f13, f2 = _ref_semantics(w13, w2, T, path)
    ref = O.moe_layer(xb, rids, rw, f13, f2, shared=[(f13(E + s), f2(E + s)) for s in range(S)])
    assert rel_maxabs(out.cpu().numpy(), ref) <= TOL


@pytest.mark.parametrize("n,k,n_iter", [(300_000, 256, 4), (5000, 256, 12), (100, 256, 3), (4096, 16, 25)])
def test_train_kmeans_matches_oracle(gpu, n, k, n_iter):
    """Codebook training (LUTQuantizer._train_kmeans) with the Lloyd iterations on the GPU
    vs the oracle restatement (pinned by the reference's golden vectors): same subsample
    and initial pick from the seeded permutations (n > 200k takes the subsample path, n < k
    pads with zeros), the same assignments; means summed in another order, so the bf16
    codebooks agree to one bf16 ulp and almost all entries exactly."""
    from block_lut_amd.quantizer import train_kmeans
    rng = np.random.default_rng(n + k)
    w = (rng.standard_normal(n) * 0.02).astype(np.float32)
    blk = np.abs(np.pad(w, (0, -n % 128)).reshape(-1, 128)).max(axis=1)
    data = (w / np.repeat(np.maximum(blk, 1e-10), 128)[:n]).astype(np.float32)
    import torch
    got = O.f32_to_bf16(train_kmeans(torch.from_numpy(data).to(gpu), k, n_iter, seed=5).float().numpy())
    ref = O.train_kmeans_ref(data, k, n_iter, seed=5)
    gf, rf = O.bf16_to_f32(got), O.bf16_to_f32(ref)
    assert np.all(np.diff(gf) >= 0)
    ulp = np.abs(rf) * 2.0 ** -7 + 1e-30
    assert np.all(np.abs(gf - rf) <= ulp), np.max(np.abs(gf - rf) / ulp)
    assert np.mean(got == ref) >= 0.95


def test_train_nested_codebooks(gpu):
    """LUTQuantizer._train_nested_codebooks: the 64-entry codebook within one bf16 ulp of
    the oracle's k-means, and both 256-entry tables built from it (16 entries by the
    reference's greedy merge in bf16)."""
    import torch
    from block_lut_amd.quantizer import build_mapped_table, greedy_merge, train_nested_codebooks
    rng = np.random.default_rng(33)
    data = np.clip(rng.standard_normal(20000) * 0.3, -1, 1).astype(np.float32)
    m64, m16 = train_nested_codebooks(torch.from_numpy(data).to(gpu), n_iter=10, seed=9)
    assert m64.dtype == torch.bfloat16 and m64.numel() == 256 and m16.numel() == 256
    c64 = m64[:64]
    assert torch.equal(m64, build_mapped_table(c64, 256))
    assert torch.equal(m16, build_mapped_table(greedy_merge(c64, 16), 256))
    ref = O.bf16_to_f32(O.train_kmeans_ref(data, 64, 10, seed=9))
    got = c64.float().numpy()
    assert np.all(np.abs(got - ref) <= np.abs(ref) * 2.0 ** -7 + 1e-30)


@pytest.mark.parametrize("fmt,T", [("bl4", 1), ("bl4", 8), ("bl4", 300), ("ref", 1), ("ref", 300),
                                   ("nested", 4), ("nested", 150)])
def test_moe_layer_graph_replays(gpu, fmt, T):
    """The layer captured in a HIP graph (router logits in, output out, one workspace):
    four replays, each after new inputs were copied into the captured buffers and an eager
    call on other buffers ran in between, every replay bit-identical to the eager layer
    on the same inputs (the decode counters left zero by each call, no stale routing)."""
    import torch
    from block_lut_amd import ops
    from block_lut_amd.formats import MoEWeights
    E, S, k, H, I = 8, 1, 2, 256, 192
    if fmt == "nested":
        w13 = NestedExpertset([2, 3, 4, 4, 3, 2, 4, 3, 2], 2 * I, H, seed=80)
        w2 = NestedExpertset([2, 3, 4, 4, 3, 2, 4, 3, 2], H, I, seed=81)
    else:
        w13, w2 = _moe_case(fmt, E, S, H, I, seed=82)
    moe = MoEWeights(w13.stack(gpu), w2.stack(gpu), H, I, E, S)
    rng = np.random.default_rng(800 + T)
    x = torch.empty((T, H), dtype=torch.bfloat16, device=gpu)
    lg = torch.empty((T, E), dtype=torch.float32, device=gpu)
    out = torch.empty((T, H), dtype=torch.float32, device=gpu)
    ws = ops.new_workspace(moe, T, k, gpu)
    x2, lg2 = torch.empty_like(x), torch.empty_like(lg)
    out2 = torch.empty_like(out)
    ws2 = ops.new_workspace(moe, T, k, gpu)

    def fill(xt, lt):
        xt.copy_(to_dev_bf16(_x(rng, T, H), gpu))
        lt.copy_(torch.from_numpy(rng.standard_normal((T, E)).astype(np.float32)).to(gpu))

    fill(x, lg)
    ops.moe_forward_logits(moe, x, lg, k, out=out, workspace=ws)   # warm-up outside capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        ops.moe_forward_logits(moe, x, lg, k, out=out, workspace=ws)
    for rep in range(4):
        fill(x, lg)
        fill(x2, lg2)
        ops.moe_forward_logits(moe, x2, lg2, k, out=out2, workspace=ws2)   # eager work between replays
        g.replay()
        torch.cuda.synchronize()
        eager = ops.moe_forward_logits(moe, x, lg, k, out_dtype=torch.float32)
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {rep}"


@pytest.mark.parametrize("T,path", [(40, 2), (300, 2), (3, 1)])
def test_moe_layer_ref_short_odd_absmax(gpu, T, path):
    """REF stacks whose absmax rows hold one entry fewer than ceil(M*K/128) (an odd count):
    the last block index is clamped to the last entry, as decompress_blocklut does
    (vllm_lut/quantizer.py:473-474), and prefill takes the register-staged kernel (the
    DMA ring reads absmax in aligned pairs and needs an even count)."""
    import torch
    from block_lut_amd import ops
    from block_lut_amd.formats import MoEWeights
    E, S, k, H, I = 6, 1, 2, 256, 192
    w13 = RefExpertset(E + S, 2 * I, H, seed=70)
    w2 = RefExpertset(E + S, H, I, seed=71)
    for w in (w13, w2):
        w.absmax = np.ascontiguousarray(w.absmax[:, :-1])
        assert w.absmax.shape[1] % 2 == 1
    moe = MoEWeights(w13.stack(gpu), w2.stack(gpu), H, I, E, S)
    rng = np.random.default_rng(700 + T)
    xb = _x(rng, T, H)
    rw, rids = O.route(rng.standard_normal((T, E)).astype(np.float32), k)
    out = ops.moe_forward(moe, to_dev_bf16(xb, gpu), torch.from_numpy(rw).to(gpu),
                          torch.from_numpy(rids).to(gpu), out_dtype=torch.float32, path=path)
    f13, f2 = _ref_semantics(w13, w2, T, path)
    ref = O.moe_layer(xb, rids, rw, f13, f2, shared=[(f13(E + s), f2(E + s)) for s in range(S)])
    assert rel_maxabs(out.cpu().numpy(), ref) <= TOL


@pytest.mark.parametrize("T", [1, 7, 40])
def test_fused_lut_moe_reference_signature(gpu, T):
    """fused_lut_moe(x, topk_ids, topk_weights, w13, w13_absmax, w2, w2_absmax, codebook)
    (vllm_lut/fast_moe.py:30-43) on the reference's REF tensors, also as the torch op
    lutmoe::fused_lut_moe (identical output); decode sizes follow the reference GEMV's
    (x * cb) * absmax products, prefill its dequantise-then-GEMM branch."""
    import torch
    import block_lut_amd.fast_moe as FM
    E, k, H, I = 8, 2, 256, 192
    w13 = RefExpertset(E, 2 * I, H, seed=60)
    w2 = RefExpertset(E, H, I, seed=61)
    rng = np.random.default_rng(600 + T)
    xb = _x(rng, T, H)
    rw, rids = O.route(rng.standard_normal((T, E)).astype(np.float32), k)
    args = (to_dev_bf16(xb, gpu), torch.from_numpy(rids).to(gpu), torch.from_numpy(rw).to(gpu),
            torch.from_numpy(w13.codes).to(gpu), to_dev_bf16(w13.absmax, gpu),
            torch.from_numpy(w2.codes).to(gpu), to_dev_bf16(w2.absmax, gpu), to_dev_bf16(w13.cb, gpu))
    out = FM.fused_lut_moe(*args)
    assert out.dtype == torch.bfloat16 and tuple(out.shape) == (T, H)
    assert torch.equal(torch.ops.lutmoe.fused_lut_moe(*args), out)
    f13, f2 = _ref_semantics(w13, w2, T, 0)
    ref = O.moe_layer(xb, rids, rw, f13, f2)
    # bf16 output: the tolerance adds half an ulp of bf16 relative to max|ref|
    assert rel_maxabs(O.bf16_to_f32(bf16_bits(out)), ref) <= TOL + 2.0 ** -8


@pytest.mark.parametrize("T,path", [(1, 1), (3, 1), (9, 1), (40, 2), (300, 2)])
def test_moe_layer_ref_per_expert_codebook(gpu, T, path):
    """REF experts at different tiers (tier 0 / 1 / 2 codes with the full / first-64 /
    first-16 tables, one codebook row per expert) through decode and prefill, plus per-
    expert dequantisation (bit-exact) and the single-expert GEMV."""
    import torch
    from block_lut_amd import ops
    from block_lut_amd.formats import MoEWeights
    E, S, k, H, I = 8, 1, 2, 256, 192
    tiers = [0, 2, 1, 2, 0, 1, 1, 2, 0]
    w13 = RefExpertset(E + S, 2 * I, H, seed=90, tiers=tiers)
    w2 = RefExpertset(E + S, H, I, seed=91, tiers=tiers)
    moe = MoEWeights(w13.stack(gpu), w2.stack(gpu), H, I, E, S)
    assert moe.w13.codebook_stride == 256
    rng = np.random.default_rng(900 + T)
    xb = _x(rng, T, H)
    rw, rids = O.route(rng.standard_normal((T, E)).astype(np.float32), k)
    out = ops.moe_forward(moe, to_dev_bf16(xb, gpu), torch.from_numpy(rw).to(gpu),
                          torch.from_numpy(rids).to(gpu), out_dtype=torch.float32, path=path)
    f13, f2 = _ref_semantics(w13, w2, T, path)
    ref = O.moe_layer(xb, rids, rw, f13, f2, shared=[(f13(E + s), f2(E + s)) for s in range(S)])
    assert rel_maxabs(out.cpu().numpy(), ref) <= TOL
    if T == 1:
        deq = bf16_bits(ops.dequant(moe.w2, 2, 5))
        for j in range(5):
            assert np.array_equal(deq[j].reshape(-1), O.ref_dequant(w2.codes[2 + j], w2.absmax[2 + j], w2.cbs[2 + j]))
        for e in (1, 5):
            xa = _x(rng, 2, I)
            y = ops.gemv(moe.w2, to_dev_bf16(xa, gpu), expert=e, out_dtype=torch.float32)
            assert rel_maxabs(y.cpu().numpy(), O.bf16_to_f32(xa) @ w2.gemv_f32(e).T) <= TOL


@pytest.mark.parametrize("fmt,T,path,renorm,E", [("bl4", 1, 1, False, 12), ("bl4", 3, 1, True, 12),
                                                 ("bl4", 32, 1, False, 12), ("bl4", 40, 2, False, 12),
                                                 ("bl4", 300, 2, True, 12), ("bl4", 1, 1, True, 130),
                                                 ("bl4", 2, 1, True, 130), ("bl4", 5, 2, False, 130),
                                                 ("ref", 1, 1, False, 12), ("ref", 1, 1, True, 130),
                                                 ("ref", 3, 1, True, 12)])
def test_moe_layer_from_logits(gpu, fmt, T, path, renorm, E):
    """Block forward from router logits (routing inside the layer) vs oracle routing + layer;
    E = 130 puts several logits on one lane of the in-kernel top-k (and, for one token, routes
    in the routing kernel before the one-token down kernels)."""
    import torch
    from block_lut_amd import ops
    from block_lut_amd.formats import MoEWeights
    S, k, H, I = 2, 3, 256, 192
    w13, w2 = _moe_case(fmt, E, S, H, I, seed=70 + T)
    moe = MoEWeights(w13.stack(gpu), w2.stack(gpu), H, I, E, S)
    rng = np.random.default_rng(700 + T)
    xb = _x(rng, T, H)
    lg = rng.standard_normal((T, E)).astype(np.float32)
    out = ops.moe_forward_logits(moe, to_dev_bf16(xb, gpu), torch.from_numpy(lg).to(gpu), k,
                                 renormalize=renorm, scaling=1.0, out_dtype=torch.float32, path=path)
    rw, rids = O.route(lg, k, renormalize=renorm)
    f13, f2 = _ref_semantics(w13, w2, T, path) if fmt == "ref" else (w13.deq_f32, w2.deq_f32)
    ref = O.moe_layer(xb, rids, rw, f13, f2, shared=[(f13(E + s), f2(E + s)) for s in range(S)])
    assert rel_maxabs(out.cpu().numpy(), ref) <= TOL


@pytest.mark.parametrize("T,E,renorm", [(1, 12, False), (2, 12, True), (1, 60, False), (2, 60, False)])
def test_moe_layer_from_logits_ties(gpu, T, E, renorm):
    """Decode routing on logits with many exact ties, -0.0 next to +0.0 and a -inf:
    the in-kernel top-k must pick the lower expert id on every tie, as the oracle
    (and torch.topk on the reference's softmax) does, so any other choice changes
    the experts and the output."""
    import torch
    from block_lut_amd import ops
    from block_lut_amd.formats import MoEWeights
    S, k, H, I = 1, 4, 256, 192
    w13, w2 = _moe_case("bl4", E, S, H, I, seed=90 + T + E)
    moe = MoEWeights(w13.stack(gpu), w2.stack(gpu), H, I, E, S)
    rng = np.random.default_rng(900 + T + E)
    xb = _x(rng, T, H)
    lg = (np.round(rng.standard_normal((T, E)) * 1.5) / 2).astype(np.float32)   # few distinct values
    lg[0, 1] = -0.0
    lg[0, 2] = 0.0
    lg[0, 3] = np.float32(lg.max())          # a tie at the top
    lg[-1, 0] = -np.inf
    out = ops.moe_forward_logits(moe, to_dev_bf16(xb, gpu), torch.from_numpy(lg).to(gpu), k,
                                 renormalize=renorm, scaling=1.0, out_dtype=torch.float32, path=1)
    rw, rids = O.route(lg, k, renormalize=renorm)
    ref = O.moe_layer(xb, rids, rw, w13.deq_f32, w2.deq_f32,
                      shared=[(w13.deq_f32(E + s), w2.deq_f32(E + s)) for s in range(S)])
    assert rel_maxabs(out.cpu().numpy(), ref) <= TOL


@pytest.mark.parametrize("fmt,T", [("bl4", 1), ("bl4", 2), ("bl4", 9), ("ref", 1), ("nested", 1)])
def test_moe_layer_decode_staged_equals_full(gpu, fmt, T):
    """The decode layer run stage by stage (routing + gate/up, then down + combine, in one
    workspace) equals the one-call layer bit for bit, and the oracle; the one-token
    stream probe (the layer's weight loads alone, for the HBM floor) runs through the C
    ABI with the same grid and leaves one word per CTA."""
    import ctypes
    import torch
    from block_lut_amd import _native as N
    from block_lut_amd import ops
    from block_lut_amd.formats import MoEWeights
    E, S, k, H, I = 8, 1, 2, 512, 320
    if fmt == "nested":
        bits = [2, 3, 4, 2, 3, 4, 3, 2, 4]
        w13 = NestedExpertset(bits, 2 * I, H, seed=91, n_iter=8)
        w2 = NestedExpertset(bits, H, I, seed=92, n_iter=8)
    else:
        w13, w2 = _moe_case(fmt, E, S, H, I, seed=21 + T)
    moe = MoEWeights(w13.stack(gpu), w2.stack(gpu), H, I, E, S)
    rng = np.random.default_rng(T)
    xb = _x(rng, T, H)
    rw, rids = O.route(rng.standard_normal((T, E)).astype(np.float32), k)
    args = (moe, to_dev_bf16(xb, gpu), torch.from_numpy(rw).to(gpu), torch.from_numpy(rids).to(gpu))
    full = ops.moe_forward(*args, out_dtype=torch.float32, path=1, workspace=ops.new_workspace(moe, T, k, gpu))
    ws = ops.new_workspace(moe, T, k, gpu)
    staged = torch.empty_like(full)
    ops.moe_forward(*args, out=staged, path=1, workspace=ws, stages=N.STAGE_ROUTE | N.STAGE_GATE_UP)
    ops.moe_forward(*args, out=staged, path=1, workspace=ws, stages=N.STAGE_DOWN)
    assert torch.equal(full, staged)
    f13, f2 = _ref_semantics(w13, w2, T, 1) if fmt == "ref" else (w13.deq_f32, w2.deq_f32)
    ref = O.moe_layer(xb, rids, rw, f13, f2, shared=[(f13(E + s), f2(E + s)) for s in range(S)])
    assert rel_maxabs(full.cpu().numpy(), ref) <= TOL
    if fmt == "bl4" and T == 1:
        d = moe.desc()
        slot_ids = torch.tensor(list(rids[0]) + [E + s for s in range(S)], dtype=torch.int32, device=gpu)
        for which in (1, 2, 3):
            n = N.lib().lutmoe_decode_stream_probe_sink_words(ctypes.byref(d), k, which)
            assert n == ((I + 7) // 8 * (k + S) if which & 1 else 0) + (H // 4 if which & 2 else 0)
            sink = torch.full((n + 1,), -7, dtype=torch.int32, device=gpu)
            N.check("lutmoe_decode_stream_probe",
                    N.lib().lutmoe_decode_stream_probe(ctypes.byref(d), slot_ids.data_ptr(), k, which,
                                                       sink.data_ptr(), None))
            torch.cuda.synchronize()
            got = sink.cpu().numpy()
            assert got[n] == -7 and not np.any(got[:n] == -7)


@pytest.mark.parametrize("T", [1, 2, 5])
def test_ref_decode_follows_reference_branch(gpu, T):
    """REF decode picks the reference's branch by token count (vllm_lut/quant_method.py:
    250-277): one token takes lut_gemv's unrounded (x * cb) * absmax products, several tokens
    the dequantised bf16(cb * absmax) weights.  The layer must sit much closer to its own
    branch's oracle than to the other branch's (the two differ by the bf16 rounding of
    every weight, about 1e-3 of the output's range)."""
    import torch
    from block_lut_amd import ops
    from block_lut_amd.formats import MoEWeights
    E, S, k, H, I = 8, 0, 2, 512, 320
    w13, w2 = _moe_case("ref", E, S, H, I, seed=123 + T)
    moe = MoEWeights(w13.stack(gpu), w2.stack(gpu), H, I, E, S)
    rng = np.random.default_rng(40 + T)
    xb = _x(rng, T, H)
    rw, rids = O.route(rng.standard_normal((T, E)).astype(np.float32), k)
    out = ops.moe_forward(moe, to_dev_bf16(xb, gpu), torch.from_numpy(rw).to(gpu),
                          torch.from_numpy(rids).to(gpu), out_dtype=torch.float32, path=1).cpu().numpy()
    gemv = O.moe_layer(xb, rids, rw, w13.gemv_f32, w2.gemv_f32)
    deq = O.moe_layer(xb, rids, rw, w13.deq_f32, w2.deq_f32)
    own, other = (gemv, deq) if T == 1 else (deq, gemv)
    e_own, e_other = rel_maxabs(out, own), rel_maxabs(out, other)
    assert e_own <= TOL
    assert e_own < 0.25 * e_other, (e_own, e_other)


def test_moe_layer_qwen_decode_full_shape(gpu):
    """Full Qwen1.5-MoE layer shape (H2048 I1408 E60 top-4), T=1, 8 and 32, BL4 weights from the
    GPU encoder; the oracle dequantises the touched experts on the host from the encoder's
    codes and fp16 codebooks."""
    import torch
    from block_lut_amd import ops
    from block_lut_amd.formats import BL4Stack, MoEWeights
    H, I, E, k = 2048, 1408, 60, 4
    g = torch.Generator(device="cpu").manual_seed(5)
    w13 = (torch.randn((E, 2 * I, H), generator=g) * 0.02).to(gpu)
    c13, t13 = ops.bl4_encode(w13, n_iter=4)
    del w13
    w2 = (torch.randn((E, H, I), generator=g) * 0.02).to(gpu)
    c2, t2 = ops.bl4_encode(w2, n_iter=4)
    del w2
    moe = MoEWeights(BL4Stack.from_fp16(c13, t13), BL4Stack.from_fp16(c2, t2), H, I, E, 0)
    d13, d2 = {}, {}

    def host13(e):
        if e not in d13:
            d13[e] = O.bl4_dequant_f32(c13[e].cpu().numpy(), t13[e].cpu().numpy().view(np.uint16))
        return d13[e]

    def host2(e):
        if e not in d2:
            d2[e] = O.bl4_dequant_f32(c2[e].cpu().numpy(), t2[e].cpu().numpy().view(np.uint16))
        return d2[e]

    for T in (1, 8, 32):
        rng = np.random.default_rng(T)
        xb = _x(rng, T, H)
        lg = rng.standard_normal((T, E)).astype(np.float32)
        out = ops.moe_forward_logits(moe, to_dev_bf16(xb, gpu), torch.from_numpy(lg).to(gpu), k,
                                     out_dtype=torch.float32).cpu().numpy()
        rw, rids = O.route(lg, k)
        ref = O.moe_layer(xb, rids, rw, host13, host2)
        assert rel_maxabs(out, ref) <= TOL, T


@pytest.mark.parametrize("n,block_size,sorted_cb", [(128 * 300 + 77, 128, True), (5000, 64, False),
                                                    (4097, 100, True), (1, 128, True)])
def test_ref_encode_bit_exact(gpu, n, block_size, sorted_cb):
    """GPU REF encoder (encode_lut) vs the oracle's restatement of encode_blocklut_kernel:
    codes and bf16 absmax bit-identical, with a short last block, an all-zero block, weights
    on exact midpoints between entries (first index wins) and an unsorted codebook."""
    import torch
    from block_lut_amd import fast_encode, ops
    rng = np.random.default_rng(n + block_size)
    cb = rng.uniform(-1, 1, 256).astype(np.float32)
    if sorted_cb:
        cb = np.sort(cb)
    w = rng.standard_normal(n).astype(np.float32) * 0.02
    if n > 3 * block_size:
        w[block_size:2 * block_size] = 0.0                     # all-zero block
        s = np.sort(cb)
        m = ((s[100:120] + s[101:121]) / 2).astype(np.float32)  # midpoints, absmax 1
        w[2 * block_size:2 * block_size + 20] = m
        w[2 * block_size + 20] = 1.0
    wb = O.f32_to_bf16(w)
    wt = torch.from_numpy(wb.view(np.int16)).view(torch.bfloat16).to(gpu)
    codes, am = ops.ref_encode(wt, torch.from_numpy(cb).to(gpu), block_size)
    ic, ia = O.ref_encode_fast(wb, cb, block_size)
    assert np.array_equal(codes.cpu().numpy(), ic)
    assert np.array_equal(am.view(torch.int16).cpu().numpy().view(np.uint16), ia)
    c2, a2 = fast_encode.encode_lut(wt, torch.from_numpy(cb).to(gpu), block_size)
    assert torch.equal(c2, codes.cpu()) and torch.equal(a2, am.cpu())


def test_ref_quantize_rule_on_golden_vectors(gpu):
    """LUTQuantizer.quantize's rule on the GPU reproduces the vectors written from the
    reference itself (tests/golden/quantizer.npz: fp32 weights, a padded tail with an
    all-zero block, bf16 weights normalised in bf16) bit for bit, through both the
    function and the LUTQuantizer class."""
    import os
    import torch
    from block_lut_amd.quantizer import LUTQuantizer, quantize
    qv = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "quantizer.npz"),
                 allow_pickle=False)
    cbb = golden_codebook()
    cb = torch.from_numpy(cbb.view(np.int16)).view(torch.bfloat16)
    for key, bf16 in (("q_f32", False), ("q_pad", False), ("q_bf16", True)):
        w = qv[f"{key}_w"]
        wt = (torch.from_numpy(w.view(np.int16)).view(torch.bfloat16) if bf16 else torch.from_numpy(w)).to(gpu)
        codes, am = quantize(wt, cb, 128)
        assert np.array_equal(codes.cpu().numpy(), qv[f"{key}_idx"]), key
        assert np.array_equal(am.view(torch.int16).cpu().numpy().view(np.uint16), qv[f"{key}_absmax"]), key
        r = LUTQuantizer("BLOCKLUT", device=str(gpu)).quantize(wt, cb)
        assert np.array_equal(r["indices"].numpy(), qv[f"{key}_idx"]), key


@pytest.mark.parametrize("n,block_size,k,bf16", [(128 * 37 + 51, 128, 256, True), (4096, 128, 40, False),
                                                 (1000, 100, 256, False)])
def test_ref_quantize_rules_bitexact(gpu, n, block_size, k, bf16):
    """Both extra REF rules against the oracle, codes and bf16 absmax bit-identical:
    'quantizer' (normalised in the weights' dtype, first nearest of an unsorted codebook)
    and 'midpoints' (the offload runtime's searchsorted over an ascending codebook of k
    entries); an all-zero block, weights on exact midpoints, a short last block."""
    import torch
    from block_lut_amd.quantizer import quantize
    rng = np.random.default_rng(n + k)
    cb = np.sort(rng.uniform(-1, 1, k).astype(np.float32))
    w = rng.standard_normal(n).astype(np.float32) * 0.02
    w[block_size:2 * block_size] = 0.0
    mid = ((cb[:-1] + cb[1:]) / np.float32(2)).astype(np.float32)
    w[2 * block_size:2 * block_size + 20] = mid[5:25]
    w[2 * block_size + 20] = 1.0
    if bf16:
        w = O.bf16_to_f32(O.f32_to_bf16(w))
        wt = torch.from_numpy(O.f32_to_bf16(w).view(np.int16)).view(torch.bfloat16).to(gpu)
    else:
        wt = torch.from_numpy(w).to(gpu)
    cbq = O.f32_to_bf16(cb[rng.permutation(k)])          # unsorted bf16 codebook
    c1, a1 = quantize(wt, torch.from_numpy(cbq.view(np.int16)).view(torch.bfloat16).to(gpu), block_size)
    i1, b1 = O.ref_quantize(w, np.pad(cbq, (0, 0)), block_size, input_is_bf16=bf16)
    assert np.array_equal(c1.cpu().numpy(), i1)
    assert np.array_equal(a1.view(torch.int16).cpu().numpy().view(np.uint16), b1)
    c2, a2 = quantize(wt, torch.from_numpy(cb).to(gpu), block_size, rule="midpoints")
    i2, b2 = O.ref_encode_midpoints(w, cb, block_size)
    assert np.array_equal(c2.cpu().numpy(), i2)
    assert np.array_equal(a2.view(torch.int16).cpu().numpy().view(np.uint16), b2)


def test_lut_quantizer_train_quantize_decompress(gpu, tmp_path):
    """LUTQuantizer end to end on the GPU: train a BLOCKLUT codebook (sorted bf16 [256]),
    quantize (codes = the golden-pinned oracle rule on that codebook), decompress (the
    oracle's dequantisation), save / load round trip; the LUT code type normalises by one
    global absmax; NESTEDLUT also builds its two 256-entry tables."""
    import torch
    from block_lut_amd.quantizer import LUTQuantizer
    rng = np.random.default_rng(77)
    w = torch.from_numpy((rng.standard_normal((4, 64, 96)) * 0.02).astype(np.float32))
    q = LUTQuantizer("BLOCKLUT", device=str(gpu))
    q.train(w.to(gpu), n_iter=10, seed=5)
    cb = q.lut_codebook
    assert cb.dtype == torch.bfloat16 and cb.numel() == 256
    assert torch.all(cb.float()[1:] >= cb.float()[:-1])
    wb = w[1].to(torch.bfloat16)
    r = q.quantize(wb.to(gpu))
    cbb = cb.view(torch.int16).numpy().view(np.uint16)
    i, a = O.ref_quantize(O.bf16_to_f32(wb.view(torch.int16).numpy().view(np.uint16)), cbb, 128,
                          input_is_bf16=True)
    assert np.array_equal(r["indices"].numpy(), i) and np.array_equal(
        r["absmax"].view(torch.int16).numpy().view(np.uint16), a)
    d = q.decompress(r["indices"], r["absmax"], r["codebook"], out_shape=(64, 96))
    assert np.array_equal(d.view(torch.int16).cpu().numpy().view(np.uint16).reshape(-1), O.ref_dequant(i, a, cbb))
    q.save(str(tmp_path))
    q2 = LUTQuantizer("BLOCKLUT", device=str(gpu))
    assert q2.load(str(tmp_path)) and torch.equal(q2.lut_codebook, cb)
    g = LUTQuantizer("LUT", device=str(gpu))
    rg = g.quantize(w[2].to(gpu), cb)
    assert rg["absmax"].numel() == 1
    ig, ag = O.ref_quantize(w[2].numpy().reshape(-1), cbb, w[2].numel())
    assert np.array_equal(rg["indices"].numpy(), ig)
    nq = LUTQuantizer("NESTEDLUT", device=str(gpu))
    nq.train(w.to(gpu), n_iter=5, seed=2)
    assert nq.nested_mapped64.numel() == 256 and nq.nested_mapped16.numel() == 256
    assert torch.unique(nq.nested_mapped16).numel() <= 16


def test_ref_encode_expert_size_roundtrip(gpu):
    """A whole Qwen W13 expert (5.77 M weights) encoded on the GPU: sampled blocks match the
    oracle, and the GPU dequantisation of the result is within the codebook's resolution."""
    import torch
    from block_lut_amd import ops
    from block_lut_amd.formats import RefStack
    M, K = 2816, 2048
    g = torch.Generator(device=gpu).manual_seed(9)
    w = (torch.randn((M, K), generator=g, device=gpu) * 0.02).to(torch.bfloat16)
    cb = torch.sort(torch.randn(256, generator=g, device=gpu) * 0.5).values
    cb = cb / cb.abs().max()
    codes, am = ops.ref_encode(w, cb, 128)
    wb = w.view(torch.int16).cpu().numpy().view(np.uint16).reshape(-1)
    rng = np.random.default_rng(9)
    for b in rng.choice(M * K // 128, 40, replace=False):
        ic, ia = O.ref_encode_fast(wb[b * 128:(b + 1) * 128], cb.cpu().numpy(), 128)
        assert np.array_equal(codes[b * 128:(b + 1) * 128].cpu().numpy(), ic)
        assert am[b].view(torch.int16).item() & 0xffff == int(ia[0])
    st = RefStack(codes.view(1, M, K), am.view(1, -1), cb.to(torch.bfloat16), 128)
    deq = ops.dequant(st, 0, 1)[0].float()
    err = (deq - w.float()).abs().max().item()
    # nearest-entry error: half the widest gap of the (bf16-stored) codebook, plus bf16
    # rounding of the entries, the absmax and the product, times the largest absmax
    # (w / absmax lies in [-1, 1]: beyond the outermost entries the whole distance counts)
    cbs = cb.to(torch.bfloat16).float().cpu().numpy()
    worst = max(np.diff(cbs).max() / 2, 1.0 - cbs.max(), cbs.min() + 1.0)
    bound = (worst + 3 * 2.0 ** -8) * float(am.float().max())
    assert err <= bound * 1.01, (err, bound)


def test_checkpoint_loaders(gpu, tmp_path):
    """The reference's on-disk layouts -> device stacks: convert_checkpoint.py tensors
    (flattened uint8 codes, `<name>.absmax`, `model._lut_codebook`) and convert_lut.py GGUF
    files (BLOCKLUT8 blobs [codes | absmax]; nested files as bit-plane sections read at
    tiers 0/1/2 with the full / mapped64 / mapped16 tables).  Codes, absmax and tables
    arrive bit-exact (dequantisation equal to the oracle's), and a layer built from the
    converted tensors matches the oracle."""
    import torch
    from block_lut_amd import checkpoint as C
    from block_lut_amd import ops
    from lutmoe_testutil import GGUF_BLOCKLUT8_TEST_ID, write_gguf
    E, H, I = 4, 256, 128
    rng = np.random.default_rng(77)
    cb = golden_codebook()
    q = {}
    for e in range(E):
        for p, shape in (("gate", (I, H)), ("up", (I, H)), ("down", (H, I))):
            w = (rng.standard_normal(shape) * 0.02).astype(np.float32)
            q[C.expert_key(0, e, p)] = O.ref_quantize(w, cb, 128)

    def bf16_t(bits):
        return torch.from_numpy(np.asarray(bits, np.uint16).view(np.int16)).view(torch.bfloat16)

    def deq_check(stack, codes_of, table_bits):
        for e in range(E):
            got = bf16_bits(ops.dequant(stack, e, 1)[0]).reshape(-1)
            c, a = codes_of(e)
            assert np.array_equal(got, O.ref_dequant(c, a, table_bits, 128))

    def w13_of(e, mask=0xFF):
        g, u = q[C.expert_key(0, e, "gate")], q[C.expert_key(0, e, "up")]
        return np.concatenate([g[0], u[0]]) & mask, np.concatenate([g[1], u[1]])

    def w2_of(e, mask=0xFF):
        d = q[C.expert_key(0, e, "down")]
        return d[0] & mask, d[1]

    # convert_checkpoint.py layout
    td = {"model._lut_codebook": bf16_t(cb)}
    for k, (idx, am) in q.items():
        td[k] = torch.from_numpy(idx.copy())
        td[k + ".absmax"] = bf16_t(am)
    lay = C.load_converted_layer(td, 0, E, H, I, device=gpu)
    deq_check(lay.w13, w13_of, cb)
    deq_check(lay.w2, w2_of, cb)
    T = 40
    xb = _x(rng, T, H)
    rw, rids = O.route(rng.standard_normal((T, E)).astype(np.float32), 2)
    out = ops.moe_forward(lay, to_dev_bf16(xb, gpu), torch.from_numpy(rw).to(gpu),
                          torch.from_numpy(rids).to(gpu), out_dtype=torch.float32, path=2).cpu().numpy()
    deq = lambda f: (lambda e: O.bf16_to_f32(O.ref_dequant(*f(e), cb, 128)))
    ref = O.moe_layer(xb, rids, rw, lambda e: deq(w13_of)(e).reshape(2 * I, H),
                      lambda e: deq(w2_of)(e).reshape(H, I))
    assert rel_maxabs(out, ref) <= TOL

    # GGUF, plain and nested
    for nested in (False, True):
        tens = []
        for k, (idx, am) in q.items():
            body = O.bitplane_pack_ref(idx) if nested else idx
            tens.append((k, (idx.size,), GGUF_BLOCKLUT8_TEST_ID, np.concatenate([body, am.view(np.uint8)]).tobytes()))
        kv = [("lut-moe.enabled", True), ("lut-moe.block_size", 128), ("lut-moe.k", 256),
              ("lut-moe.nested_lut", nested), ("lut-moe.lut_table", cb.tolist())]
        if nested:
            kv += [("lut-moe.lut_mapped64", cb[:64].tolist()), ("lut-moe.lut_mapped16", cb[:16].tolist())]
        path = str(tmp_path / f"m{int(nested)}.gguf")
        write_gguf(path, kv, tens)
        g = C.read_gguf(path)
        for tier in ((0, 1, 2) if nested else (0,)):
            mask, tab = {0: (0xFF, cb), 1: (0x3F, cb[:64]), 2: (0x0F, cb[:16])}[tier]
            tab256 = np.full(256, tab[-1], np.uint16)
            tab256[:tab.size] = tab
            lay = C.load_gguf_layer(g, 0, E, H, I, tier=tier, device=gpu)
            for e in range(E):
                c13, a13 = w13_of(e, mask)
                assert np.array_equal(lay.w13.codes[e].cpu().numpy().reshape(-1), c13)
                assert np.array_equal(bf16_bits(lay.w13.absmax[e]).reshape(-1), a13)
            deq_check(lay.w13, lambda e: w13_of(e, mask), tab256)
            deq_check(lay.w2, lambda e: w2_of(e, mask), tab256)


def test_gguf_tier_upgrade(gpu, tmp_path):
    """Experts of a nested GGUF file loaded at mixed tiers (one codebook row per expert),
    then promoted in place (2 -> 1, 2 -> 0, 1 -> 0) from the sections they lack: codes
    and codebooks equal a fresh load at the new tiers, the two layers give identical
    outputs on the decode and prefill paths, and those match the oracle.  A layer loaded
    at one tier keeps one shared codebook while every expert moves together."""
    import torch
    from block_lut_amd import checkpoint as C
    from block_lut_amd import ops
    from lutmoe_testutil import GGUF_BLOCKLUT8_TEST_ID, TIER_MASK, tier_tables, write_gguf
    E, H, I, k = 6, 256, 128, 2
    rng = np.random.default_rng(78)
    cb = golden_codebook()
    tabs = tier_tables(cb)
    q, tens = {}, []
    for e in range(E):
        for p, shape in (("gate", (I, H)), ("up", (I, H)), ("down", (H, I))):
            w = (rng.standard_normal(shape) * 0.02).astype(np.float32)
            idx, am = O.ref_quantize(w, cb, 128)
            key = C.expert_key(0, e, p)
            q[key] = (idx, am)
            tens.append((key, (idx.size,), GGUF_BLOCKLUT8_TEST_ID,
                         np.concatenate([O.bitplane_pack_ref(idx), am.view(np.uint8)]).tobytes()))
    kv = [("lut-moe.enabled", True), ("lut-moe.block_size", 128), ("lut-moe.k", 256),
          ("lut-moe.nested_lut", True), ("lut-moe.lut_table", cb.tolist()),
          ("lut-moe.lut_mapped64", cb[:64].tolist()), ("lut-moe.lut_mapped16", cb[:16].tolist())]
    path = str(tmp_path / "tiers.gguf")
    write_gguf(path, kv, tens)
    g = C.read_gguf(path)

    def parts(e):
        return [q[C.expert_key(0, e, p)] for p in ("gate", "up", "down")]

    def check(lay, tiers):
        for e, t in enumerate(tiers):
            (gi, ga), (ui, ua), (di, da) = parts(e)
            assert np.array_equal(lay.w13.codes[e].cpu().numpy().reshape(-1), np.concatenate([gi, ui]) & TIER_MASK[t])
            assert np.array_equal(lay.w2.codes[e].cpu().numpy().reshape(-1), di & TIER_MASK[t])
            for st in (lay.w13, lay.w2):
                row = st.codebook if st.codebook_stride == 0 else st.codebook[e]
                assert np.array_equal(bf16_bits(row).reshape(-1), tabs[t])

    def oracle_out(tiers, xb, rids, rw, gemv):
        def mat(e, which):
            (gi, ga), (ui, ua), (di, da) = parts(e)
            c, a, shape = ((np.concatenate([gi, ui]), np.concatenate([ga, ua]), (2 * I, H)) if which == 13
                           else (di, da, (H, I)))
            c = c & TIER_MASK[tiers[e]]
            tab = O.bf16_to_f32(tabs[tiers[e]])
            if gemv:
                am = O.bf16_to_f32(a)
                return (tab[c] * am[np.arange(c.size) // 128]).astype(np.float32).reshape(shape)
            return O.bf16_to_f32(O.ref_dequant(c, a, tabs[tiers[e]], 128)).reshape(shape)
        return O.moe_layer(xb, rids, rw, lambda e: mat(e, 13), lambda e: mat(e, 2))

    def run(lay, xb, rids, rw, path):
        return ops.moe_forward(lay, to_dev_bf16(xb, gpu), torch.from_numpy(rw).to(gpu),
                               torch.from_numpy(rids).to(gpu), out_dtype=torch.float32, path=path)

    lay = C.load_gguf_layer(g, 0, E, H, I, tier=[2, 1, 0, 2, 2, 1], device=gpu)
    assert lay.w13.codebook_stride == 256
    check(lay, [2, 1, 0, 2, 2, 1])
    C.upgrade_gguf_experts(lay, g, 0, [0, 1], 1)
    C.upgrade_gguf_experts(lay, g, 0, [3, 5], 0)
    now = [1, 1, 0, 0, 2, 0]
    assert lay.w13.tiers == now
    check(lay, now)
    fresh = C.load_gguf_layer(g, 0, E, H, I, tier=now, device=gpu)
    for T, path in ((1, 1), (5, 1), (40, 2)):
        xb = _x(rng, T, H)
        rw, rids = O.route(rng.standard_normal((T, E)).astype(np.float32), k)
        a, b = run(lay, xb, rids, rw, path), run(fresh, xb, rids, rw, path)
        assert torch.equal(a, b)
        # one decode token: lut_gemv's products; several tokens: the dequantised weights
        assert rel_maxabs(a.cpu().numpy(), oracle_out(now, xb, rids, rw, T == 1 and path == 1)) <= TOL

    lay2 = C.load_gguf_layer(g, 0, E, H, I, tier=2, device=gpu)
    assert lay2.w13.codebook_stride == 0
    C.upgrade_gguf_experts(lay2, g, 0, range(E), 1)
    assert lay2.w13.codebook_stride == 0
    check(lay2, [1] * E)
    C.upgrade_gguf_experts(lay2, g, 0, [2], 0)
    assert lay2.w13.codebook_stride == 256
    check(lay2, [1, 1, 0, 1, 1, 1])
    xb = _x(rng, 3, H)
    rw, rids = O.route(rng.standard_normal((3, E)).astype(np.float32), k)
    assert rel_maxabs(run(lay2, xb, rids, rw, 1).cpu().numpy(),
                      oracle_out([1, 1, 0, 1, 1, 1], xb, rids, rw, False)) <= TOL


@pytest.mark.parametrize("fmt", ["bl4", "ref", "nested"])
def test_prefill_deepseek_shape(gpu, fmt):
    """Grouped MFMA prefill at the DeepSeek-V2-Lite expert shape (H2048 I1408): 8 routed
    experts top-2 + 1 shared, T=512, so tiles of 256 rows (shared expert), about 128-row
    routed tiles and the tail split all occur; every format's ring loader at full K.  The
    oracle dequantises the experts on the host from their codes."""
    import torch
    from block_lut_amd import ops
    from block_lut_amd.formats import MoEWeights
    from gpu_weights import DevBL4, DevNested, DevRef
    H, I, E, S, k, T = 2048, 1408, 8, 1, 2, 512
    g = torch.Generator(device=gpu).manual_seed(31)

    def stack(M, K):
        if fmt == "bl4":
            return DevBL4(E + S, M, K, g, gpu)
        if fmt == "ref":
            return DevRef(E + S, M, K, g, gpu)
        return DevNested([[2, 3, 4][e % 3] for e in range(E + S)], M, K, g, gpu)

    w13, w2 = stack(2 * I, H), stack(H, I)
    moe = MoEWeights(w13.stack, w2.stack, H, I, E, S)
    rng = np.random.default_rng(512)
    xb = _x(rng, T, H)
    lg = rng.standard_normal((T, E)).astype(np.float32)
    rw, rids = O.route(lg, k)
    out = ops.moe_forward(moe, to_dev_bf16(xb, gpu), torch.from_numpy(rw).to(gpu),
                          torch.from_numpy(rids).to(gpu), out_dtype=torch.float32, path=2).cpu().numpy()
    ref = O.moe_layer(xb, rids, rw, w13.host, w2.host,
                      shared=[(w13.host(E + s), w2.host(E + s)) for s in range(S)])
    assert rel_maxabs(out, ref) <= TOL


def test_moe_layer_mixtral_shape(gpu):
    """Mixtral-8x7B layer shape (H4096 I14336, 8 experts top-2 with renormalisation): K spans
    two (W13) and seven (W2) 2048-column decode chunks, and the MFMA path runs 112 n-tiles per
    expert.  Decode T=1 and T=3 from logits, prefill T=64 from ids on 3 experts; the oracle
    dequantises the touched experts on the host from their codes."""
    import torch
    from block_lut_amd import ops
    from block_lut_amd.formats import MoEWeights
    from gpu_weights import DevBL4
    H, I, E, k = 4096, 14336, 8, 2
    g = torch.Generator(device=gpu).manual_seed(14)
    w13 = DevBL4(E, 2 * I, H, g, gpu)
    w2 = DevBL4(E, H, I, g, gpu)
    moe = MoEWeights(w13.stack, w2.stack, H, I, E, 0)
    for T in (1, 3):
        rng = np.random.default_rng(140 + T)
        xb = _x(rng, T, H)
        lg = rng.standard_normal((T, E)).astype(np.float32)
        out = ops.moe_forward_logits(moe, to_dev_bf16(xb, gpu), torch.from_numpy(lg).to(gpu), k,
                                     renormalize=True, out_dtype=torch.float32, path=1).cpu().numpy()
        rw, rids = O.route(lg, k, renormalize=True)
        ref = O.moe_layer(xb, rids, rw, w13.host, w2.host)
        assert rel_maxabs(out, ref) <= TOL, T
    T = 64
    rng = np.random.default_rng(164)
    xb = _x(rng, T, H)
    rids = np.stack([rng.choice([0, 3, 5], size=k, replace=False) for _ in range(T)]).astype(np.int32)
    rw = rng.dirichlet(np.ones(k), size=T).astype(np.float32)
    out = ops.moe_forward(moe, to_dev_bf16(xb, gpu), torch.from_numpy(rw).to(gpu),
                          torch.from_numpy(rids).to(gpu), out_dtype=torch.float32, path=2).cpu().numpy()
    ref = O.moe_layer(xb, rids, rw, w13.host, w2.host)
    assert rel_maxabs(out, ref) <= TOL


@pytest.mark.parametrize("T,k", [(1, 1), (1, 2), (2, 2), (3, 2), (20, 2), (40, 2)])
def test_moe_layer_two_chunk_rows(gpu, T, k):
    """Decode where both projections span two 2048-column chunks (H = 4096, I = 2304): one and
    two tokens (the one-token down kernel over both chunks, with one or two active experts),
    two-token passes (T = 3) and four-token passes (T = 20, ten positions per expert, and
    T = 40 on the forced GEMV path: the interleaved code-dword lane map of the 8-row loop)
    against the oracle on host-dequantised weights."""
    import torch
    from block_lut_amd import ops
    from block_lut_amd.formats import MoEWeights
    from gpu_weights import DevBL4
    E, S, H, I = 4, 0, 4096, 2304
    g = torch.Generator(device=gpu).manual_seed(230 + 10 * T + k)
    w13 = DevBL4(E, 2 * I, H, g, gpu)
    w2 = DevBL4(E, H, I, g, gpu)
    moe = MoEWeights(w13.stack, w2.stack, H, I, E, S)
    rng = np.random.default_rng(2300 + T)
    xb = _x(rng, T, H)
    lg = rng.standard_normal((T, E)).astype(np.float32)
    rw, rids = O.route(lg, k)
    out = ops.moe_forward(moe, to_dev_bf16(xb, gpu), torch.from_numpy(rw).to(gpu),
                          torch.from_numpy(rids).to(gpu), out_dtype=torch.float32, path=1)
    ref = O.moe_layer(xb, rids, rw, w13.host, w2.host)
    assert rel_maxabs(out.cpu().numpy(), ref) <= TOL


def _sigmoid_gate(xb, gate_bits):
    z = O.bf16_to_f32(xb).astype(np.float64) @ O.bf16_to_f32(gate_bits).astype(np.float64)
    return 1.0 / (1.0 + np.exp(-z))


@pytest.mark.parametrize("fmt,T,path,logits", [("bl4", 1, 1, True), ("bl4", 2, 1, False), ("bl4", 5, 1, True),
                                               ("bl4", 5, 1, False), ("bl4", 70, 2, True),
                                               ("ref", 1, 1, False), ("ref", 4, 1, True), ("ref", 40, 2, False)])
def test_moe_layer_qwen_gated_shared_expert(gpu, fmt, T, path, logits):
    """Qwen1.5-MoE's shared expert (customized/qwen.py:40-43, 99-100): one MLP with 4x the
    routed intermediate size, split into 4 slots of I, each token's slots weighted by
    sigmoid(x . shared_expert_gate).  The oracle runs the unsplit shared MLP and the gate in
    float64; decode with routing in registers (T <= 2), in the routing kernel (T = 4, 5),
    from ids and from logits, and the MFMA path."""
    import torch
    from block_lut_amd import ops
    from block_lut_amd.formats import (BL4Stack, MoEWeights, RefStack, split_shared_bl4,
                                       split_shared_ref)
    E, k, H, I, m = 8, 2, 512, 256, 4
    rng = np.random.default_rng(300 + T)
    if fmt == "bl4":
        routed13 = BL4Expertset(E, 2 * I, H, seed=31 + T, n_iter=8)
        routed2 = BL4Expertset(E, H, I, seed=32 + T, n_iter=8)
        sh13 = BL4Expertset(1, 2 * m * I, H, seed=33 + T, n_iter=8)
        sh2 = BL4Expertset(1, H, m * I, seed=34 + T, n_iter=8)
        c13, t13, c2, t2 = split_shared_bl4(torch.from_numpy(sh13.codes[0]), torch.from_numpy(sh13.tables[0]),
                                            torch.from_numpy(sh2.codes[0]), torch.from_numpy(sh2.tables[0]), I)
        w13 = BL4Stack.from_fp16(torch.cat([torch.from_numpy(routed13.codes), c13]).to(gpu),
                                 to_dev_f16(np.concatenate([routed13.tables, t13.numpy()]), gpu))
        w2 = BL4Stack.from_fp16(torch.cat([torch.from_numpy(routed2.codes), c2]).to(gpu),
                                to_dev_f16(np.concatenate([routed2.tables, t2.numpy()]), gpu))
        sh_w13, sh_w2 = sh13.deq_f32(0), sh2.deq_f32(0)
    else:
        routed13 = RefExpertset(E, 2 * I, H, seed=31 + T)
        routed2 = RefExpertset(E, H, I, seed=32 + T)
        sh13 = RefExpertset(1, 2 * m * I, H, seed=33 + T)
        sh2 = RefExpertset(1, H, m * I, seed=34 + T)
        c13, a13, c2, a2 = split_shared_ref(torch.from_numpy(sh13.codes[0]), torch.from_numpy(sh13.absmax[0].view(np.int16)),
                                            torch.from_numpy(sh2.codes[0]), torch.from_numpy(sh2.absmax[0].view(np.int16)), I)
        cb = to_dev_bf16(routed13.cb, gpu)
        w13 = RefStack(torch.cat([torch.from_numpy(routed13.codes), c13]).to(gpu),
                       torch.cat([torch.from_numpy(routed13.absmax.view(np.int16)), a13]).to(gpu).view(torch.bfloat16),
                       cb, 128)
        w2 = RefStack(torch.cat([torch.from_numpy(routed2.codes), c2]).to(gpu),
                      torch.cat([torch.from_numpy(routed2.absmax.view(np.int16)), a2]).to(gpu).view(torch.bfloat16),
                      cb, 128)
        sem13, sem2 = _ref_semantics(sh13, sh2, T, path)
        sh_w13, sh_w2 = sem13(0), sem2(0)
    gate = O.f32_to_bf16((rng.standard_normal(H) * 0.05).astype(np.float32))
    moe = MoEWeights(w13, w2, H, I, E, m, shared_gate=to_dev_bf16(gate, gpu))
    xb = _x(rng, T, H)
    lg = rng.standard_normal((T, E)).astype(np.float32)
    rw, rids = O.route(lg, k)
    if logits:
        out = ops.moe_forward_logits(moe, to_dev_bf16(xb, gpu), torch.from_numpy(lg).to(gpu), k,
                                     out_dtype=torch.float32, path=path)
    else:
        out = ops.moe_forward(moe, to_dev_bf16(xb, gpu), torch.from_numpy(rw).to(gpu),
                              torch.from_numpy(rids).to(gpu), out_dtype=torch.float32, path=path)
    f13, f2 = _ref_semantics(routed13, routed2, T, path) if fmt == "ref" else (routed13.deq_f32, routed2.deq_f32)
    sw = _sigmoid_gate(xb, gate)
    assert sw.mean() < 0.85     # the gate moves the shared expert's weight well away from 1
    ref = O.moe_layer(xb, rids, rw, f13, f2, shared=[(sh_w13, sh_w2)], shared_w=sw)
    assert rel_maxabs(out.cpu().numpy(), ref) <= TOL


def test_moe_layer_paths_agree(gpu):
    """GEMV and MFMA paths on the same inputs (both fp32 accumulation)."""
    import torch
    from block_lut_amd import ops
    from block_lut_amd.formats import MoEWeights
    E, S, k, H, I, T = 8, 0, 2, 512, 320, 16
    w13, w2 = _moe_case("bl4", E, S, H, I, seed=5)
    moe = MoEWeights(w13.stack(gpu), w2.stack(gpu), H, I, E, S)
    rng = np.random.default_rng(55)
    xb = _x(rng, T, H)
    rw, rids = O.route(rng.standard_normal((T, E)).astype(np.float32), k)
    args = (moe, to_dev_bf16(xb, gpu), torch.from_numpy(rw).to(gpu), torch.from_numpy(rids).to(gpu))
    a = ops.moe_forward(*args, out_dtype=torch.float32, path=1).cpu().numpy()
    b = ops.moe_forward(*args, out_dtype=torch.float32, path=2).cpu().numpy()
    assert rel_maxabs(a, b) <= TOL


# ------------------------------------------------ dense bf16 shared expert

def dense_shared_weights(gpu, Is, H, seed):
    """A dense bf16 shared expert (N(0, 0.02) on the device) and its float32 host copy."""
    import torch
    g = torch.Generator(device=gpu).manual_seed(seed)
    w13 = (torch.randn((2 * Is, H), generator=g, device=gpu) * 0.02).to(torch.bfloat16)
    w2 = (torch.randn((H, Is), generator=g, device=gpu) * 0.02).to(torch.bfloat16)

    def host(t):
        return O.bf16_to_f32(t.view(torch.int16).cpu().numpy().view(np.uint16))
    return w13, w2, host(w13), host(w2)


@pytest.mark.parametrize("T,path,gated,logits", [(1, 1, False, True), (1, 1, True, False), (3, 1, True, True),
                                                 (9, 1, False, False), (32, 1, True, False), (5, 2, True, False),
                                                 (300, 2, False, True)])
def test_moe_layer_dense_shared_expert(gpu, T, path, gated, logits):
    """A shared expert kept in dense bf16 beside the LUT experts (and a LUT shared slot):
    every token adds w * W2s . bf16(silu(Wg x) * (Wu x)), w = 1 or sigmoid(x . g) (which
    then weighs the LUT shared slot too), against the oracle, on the GEMV (decode) and MFMA
    (prefill) paths; the stages run one by one give the one-call result bit for bit."""
    import torch
    from block_lut_amd import _native as N
    from block_lut_amd import ops
    from block_lut_amd.formats import MoEWeights
    E, S, k, H, I, Is = 8, 1, 2, 512, 320, 640
    w13, w2 = _moe_case("bl4", E, S, H, I, seed=600 + T)
    d13, d2, h13, h2 = dense_shared_weights(gpu, Is, H, 601 + T)
    rng = np.random.default_rng(602 + T)
    gate = O.f32_to_bf16((rng.standard_normal(H) * 0.05).astype(np.float32)) if gated else None
    moe = MoEWeights(w13.stack(gpu), w2.stack(gpu), H, I, E, S, dense_shared=(d13, d2),
                     shared_gate=None if gate is None else to_dev_bf16(gate, gpu))
    xb = _x(rng, T, H)
    lg = rng.standard_normal((T, E)).astype(np.float32)
    rw, rids = O.route(lg, k)
    x = to_dev_bf16(xb, gpu)
    if logits:
        out = ops.moe_forward_logits(moe, x, torch.from_numpy(lg).to(gpu), k, out_dtype=torch.float32, path=path)
    else:
        args = (moe, x, torch.from_numpy(rw).to(gpu), torch.from_numpy(rids).to(gpu))
        out = ops.moe_forward(*args, out_dtype=torch.float32, path=path)
        ws = ops.new_workspace(moe, T, k, gpu)
        staged = torch.empty_like(out)
        ops.moe_forward(*args, out=staged, path=path, workspace=ws, stages=N.STAGE_ROUTE | N.STAGE_GATE_UP)
        ops.moe_forward(*args, out=staged, path=path, workspace=ws, stages=N.STAGE_DOWN)
        assert torch.equal(out, staged)
    sw = _sigmoid_gate(xb, gate) if gated else None
    shared = [(w13.deq_f32(E + s), w2.deq_f32(E + s)) for s in range(S)] + [(h13, h2)]
    ref = O.moe_layer(xb, rids, rw, w13.deq_f32, w2.deq_f32, shared=shared, shared_w=sw)
    assert rel_maxabs(out.cpu().numpy(), ref) <= TOL
    # the dense expert moves the result well past the bar: dropping it fails
    ref_wo = O.moe_layer(xb, rids, rw, w13.deq_f32, w2.deq_f32, shared=shared[:S], shared_w=sw)
    assert rel_maxabs(ref_wo, ref) > 50 * TOL
