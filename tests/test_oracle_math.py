"""The oracle pinned by what the mathematics fixes: independent library
routines (torch casts and matmuls, scipy softmax, argsort), brute force on
tiny inputs, closed forms and invariants.  CPU only."""
import numpy as np
import pytest

import oracle as O


# ----------------------------------------------------------------- rounding

def test_f32_to_bf16_matches_torch_on_all_patterns_of_a_sweep():
    import torch
    rng = np.random.default_rng(0)
    u = rng.integers(0, 2 ** 32, 2_000_000, dtype=np.uint64).astype(np.uint32)
    x = u.view(np.float32)
    x = x[~np.isnan(x)]
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(O.f32_to_bf16(x), ref)
    assert np.array_equal(O.c_f32_to_bf16(x), ref)


def test_f32_to_f16_c_matches_numpy():
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.standard_normal(300000).astype(np.float32) * s
                        for s in (1e-9, 1e-7, 6e-5, 1e-3, 0.02, 1.0, 3e4, 7e4)])
    x = np.concatenate([x, np.float32([0.0, -0.0, np.inf, -np.inf, 65504, 65520, 65519.99,
                                       2 ** -24, 2 ** -25, 3 * 2 ** -26])])
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(O.c_f32_to_f16(x), ref)


def test_f16_bf16_table_conversion_all_patterns():
    import torch
    h = np.arange(65536, dtype=np.uint16)
    ok = ~np.isnan(h.view(np.float16))
    ref = torch.from_numpy(h.view(np.float16)).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(O.bl4_tables_bf16(h)[ok], ref[ok])


# ------------------------------------------------------------------- REF

def test_ref_dequant_brute_force_vs_torch_bf16_mul():
    """All 256 codes x a spread of absmax values; torch's bf16 multiply is the
    independent reference (quantizer.py:349)."""
    import torch
    cb = O.f32_to_bf16(np.linspace(-1, 1, 256, dtype=np.float32))
    scales = np.float32([0.0, 1e-40, 1e-10, 3e-3, 0.02, 0.5, 1.0, 3.0, 1e4, 3e38])
    am = O.f32_to_bf16(scales)
    idx = np.tile(np.arange(256, dtype=np.uint8), 10)
    bs = 256
    got = O.ref_dequant(idx, am, cb, bs)
    tcb = torch.from_numpy(cb.view(np.int16)).view(torch.bfloat16)
    tam = torch.from_numpy(am.view(np.int16)).view(torch.bfloat16)
    ref = (tcb[torch.from_numpy(idx).long()] * tam[torch.arange(idx.size) // bs])
    assert np.array_equal(got, ref.view(torch.int16).numpy().view(np.uint16))


def test_ref_dequant_clamps_block_index():
    cb = O.f32_to_bf16(np.linspace(-1, 1, 256, dtype=np.float32))
    am = O.f32_to_bf16(np.float32([1.0, 2.0]))
    idx = np.full(1000, 255, np.uint8)
    out = O.bf16_to_f32(O.ref_dequant(idx, am, cb, 128))
    assert np.all(out[:128] == 1.0) and np.all(out[128:] == 2.0)


def test_ref_gemv_vs_torch_matmul():
    import torch
    rng = np.random.default_rng(2)
    M, K = 70, 384
    idx = rng.integers(0, 256, (M, K), dtype=np.uint8)
    cb = O.f32_to_bf16(rng.standard_normal(256).astype(np.float32))
    am = O.f32_to_bf16(np.abs(rng.standard_normal(M * K // 128)).astype(np.float32))
    x = O.f32_to_bf16(rng.standard_normal(K).astype(np.float32))
    W = torch.from_numpy(O.bf16_to_f32(cb)[idx].astype(np.float64)) * \
        torch.from_numpy(np.repeat(O.bf16_to_f32(am).astype(np.float64), 128).reshape(M, K))
    ref = (W @ torch.from_numpy(O.bf16_to_f32(x).astype(np.float64))).numpy()
    got = O.ref_gemv(x, idx, cb, am)
    assert np.abs(got - ref).max() <= 1e-6 * np.abs(ref).max()


def test_ref_encode_fast_equals_golden_pinned_quantize_on_bf16_codebooks():
    """With an fp32 codebook holding bf16 values and bf16 weights, the fast encoder's rule
    (fp32 absmax and division, first nearest entry) is the quantizer's fp32 branch, which the
    reference's own outputs pin (test_oracle_golden)."""
    rng = np.random.default_rng(21)
    cb_bf16 = O.f32_to_bf16(np.sort(rng.standard_normal(256).astype(np.float32)))
    w = O.f32_to_bf16(rng.standard_normal(128 * 37 + 51).astype(np.float32) * 0.02)
    idx, am = O.ref_encode_fast(w, O.bf16_to_f32(cb_bf16), 128)
    idx2, am2 = O.ref_quantize(O.bf16_to_f32(w), cb_bf16, 128)
    assert np.array_equal(idx, idx2) and np.array_equal(am, am2)


def test_ref_encode_fast_argmin_ties_and_zero_block():
    """Every index is a nearest entry of w / absmax (fp32), ties go to the first index
    (exact midpoints of a non-uniform codebook, and duplicated entries), an all-zero block
    keeps absmax 1e-10 and maps to the entry nearest 0; an unsorted codebook is scanned
    whole."""
    cb = np.sort(np.random.default_rng(3).uniform(-1, 1, 256)).astype(np.float32)
    cb[10] = cb[11]                                   # duplicated entry: index 10 wins
    mids = ((cb[20:40] + cb[21:41]) / 2).astype(np.float32)
    # weights equal to the midpoints (absmax 1: include +-1 so w / absmax == w)
    w = np.concatenate([mids, np.float32([1.0, -1.0, cb[11], 0.5])])
    wb = O.f32_to_bf16(w)
    idx, am = O.ref_encode_fast(wb, cb, 64)
    v = O.bf16_to_f32(wb) / np.float32(1.0)
    d = np.abs(v[:, None] - cb[None, :])
    first = np.array([np.flatnonzero(row == row.min())[0] for row in d])
    assert np.array_equal(idx, first)
    assert idx[w.size - 2] == 10 or abs(O.bf16_to_f32(wb)[w.size - 2] - cb[10]) > 0
    zi, zam = O.ref_encode_fast(np.zeros(64, np.uint16), cb, 64)
    assert np.all(zi == np.abs(cb).argmin())
    assert zam[0] == O.f32_to_bf16(np.float32(1e-10))
    perm = np.random.default_rng(4).permutation(256)
    pi, _ = O.ref_encode_fast(wb, cb[perm], 64)
    assert np.array_equal(cb[perm][pi], cb[first])


def test_ref_encode_midpoints_nearest_and_lower_on_midpoints():
    """The offload encoder's searchsorted rule: every index is a nearest entry of
    w / absmax (brute force over the sorted codebook) except within one fp32 ulp of a
    midpoint, where the fp32 midpoint decides; a value exactly on an fp32 midpoint takes
    the lower entry; absmax is at least fp32(1e-12) (an all-zero block maps to the entry
    nearest 0); the zero-padded tail block gives the same codes as the block alone; a
    codebook shorter than 256 indexes only its own entries."""
    rng = np.random.default_rng(31)
    cb = np.sort(rng.standard_normal(256).astype(np.float32) * 0.4)
    w = rng.standard_normal(128 * 9 + 77).astype(np.float32) * 0.02
    idx, am = O.ref_encode_midpoints(w, cb, 128)
    blocks = np.concatenate([w, np.zeros(128 * 10 - w.size, np.float32)]).reshape(10, 128)
    amax = np.maximum(np.abs(blocks).max(1), np.float32(1e-12))
    assert np.array_equal(am, O.f32_to_bf16(amax))
    v = (blocks / amax[:, None]).astype(np.float32).reshape(-1)[:w.size]
    d = np.abs(v[:, None].astype(np.float64) - cb[None, :].astype(np.float64))
    mid = ((cb[:-1] + cb[1:]) / np.float32(2)).astype(np.float32)
    near_mid = np.abs(v[:, None] - mid[None, :]).min(1) <= np.spacing(np.abs(v)) * 2
    ok = d[np.arange(v.size), idx] <= d.min(1) * (1 + 1e-12)
    assert np.all(ok | near_mid) and ok.mean() > 0.99
    # exactly on midpoints (absmax 1 via a +-1 weight): the lower entry
    on = np.concatenate([mid[40:80], np.float32([1.0, -1.0])])
    oi, _ = O.ref_encode_midpoints(on, cb, 128)
    assert np.array_equal(oi[:40], np.arange(40, 80))
    zi, zam = O.ref_encode_midpoints(np.zeros(128, np.float32), cb, 128)
    assert np.all(zi == np.abs(cb).argmin()) and zam[0] == O.f32_to_bf16(np.float32(1e-12))
    ti, _ = O.ref_encode_midpoints(w[128 * 9:], cb, 128)
    assert np.array_equal(ti, idx[128 * 9:])
    si, _ = O.ref_encode_midpoints(w, cb[::16], 128)
    assert si.max() <= 15


def test_bitplane_pack_roundtrip_all_codes():
    codes = np.tile(np.arange(256, dtype=np.uint8), 4)
    packed = O.bitplane_pack_ref(codes)
    n = codes.size
    assert packed.size == n // 2 + n // 4 + n // 4
    assert np.array_equal(O.unpack_4bit_ref(packed, n), codes & 0x0F)
    assert np.array_equal(O.unpack_6bit_ref(packed, n), codes & 0x3F)
    # even element in the low nibble (model_offload.py:755)
    assert packed[0] == (codes[0] & 15) | ((codes[1] & 15) << 4)


def test_merge_bitplane_rebuilds_codes_from_sections():
    """A tier upgrade by merging sections: the low nibble (tier 2) plus the mid section at
    bit 4 equals the reference's 6-bit unpack (tier 1), plus the high section at bit 6 the
    original codes (tier 0), for every code value in shuffled order.  The fields replace
    what the target bits held (a planted wrong bit there is overwritten) and a second
    merge changes nothing; code 4i+j takes bits 2j..2j+1 of plane byte i."""
    rng = np.random.default_rng(12)
    codes = rng.permutation(np.tile(np.arange(256, dtype=np.uint8), 8))
    n = codes.size
    packed = O.bitplane_pack_ref(codes)
    mid, high = packed[n // 2:n // 2 + n // 4], packed[n // 2 + n // 4:]
    c4 = O.unpack_4bit_ref(packed, n)
    c6 = O.merge_bitplane_ref(c4, mid, 4)
    assert np.array_equal(c6, O.unpack_6bit_ref(packed, n))
    c8 = O.merge_bitplane_ref(c6, high, 6)
    assert np.array_equal(c8, codes)
    assert np.array_equal(O.merge_bitplane_ref(c8, high, 6), codes)
    noisy = (c4 | (rng.integers(0, 4, n, dtype=np.uint8) << 4)).astype(np.uint8)
    assert np.array_equal(O.merge_bitplane_ref(noisy, mid, 4), c6)
    assert list(O.merge_bitplane_ref(np.zeros(4, np.uint8), np.array([0b11100100], np.uint8), 0)) == [0, 1, 2, 3]
    lo = O.merge_bitplane_ref(O.merge_bitplane_ref(np.zeros(n, np.uint8), mid, 0), high, 2)
    assert np.array_equal(lo, (codes >> 4) & 0x0F)


# ------------------------------------------------------------------- BL4

def _bl4(w, n_iter=30):
    p, t = O.bl4_encode(w, n_iter=n_iter)
    return O.bl4_unpack(p), O.f16_to_f32(t)


def test_bl4_codes_are_argmin_of_stored_tables():
    rng = np.random.default_rng(3)
    w = (rng.standard_normal((32, 256)) * 0.02).astype(np.float32)
    codes, tab = _bl4(w)
    M, K = w.shape
    t = tab.reshape(M, K // 64, 16)
    for r in range(M):
        for b in range(K // 64):
            x = w[r, 64 * b: 64 * b + 64]
            d = np.abs(x[:, None] - t[r, b][None, :])
            assert np.array_equal(codes[r, 64 * b: 64 * b + 64], d.argmin(axis=1))


def test_bl4_tables_sorted_and_fp16():
    rng = np.random.default_rng(4)
    w = (rng.standard_normal((16, 128)) * 0.02).astype(np.float32)
    _, t = O.bl4_encode(w)
    v = O.f16_to_f32(t)
    assert np.all(np.diff(v, axis=-1) >= 0)


def test_bl4_exact_when_block_has_at_most_16_values():
    """Brute force: a block with <= 16 distinct values is reproduced to fp16."""
    rng = np.random.default_rng(5)
    for nvals in (1, 2, 5, 16):
        vals = (rng.standard_normal(nvals) * 0.02).astype(np.float32)
        w = rng.choice(vals, size=(1, 64)).astype(np.float32)
        codes, tab = _bl4(w)
        rec = tab.reshape(16)[codes[0]]
        assert np.array_equal(rec, w[0].astype(np.float16).astype(np.float32)), nvals


def test_bl4_quality_close_to_sklearn_kmeans():
    from sklearn.cluster import KMeans
    rng = np.random.default_rng(6)
    w = (rng.standard_normal((4, 256)) * 0.02).astype(np.float32)
    codes, tab = _bl4(w, 50)
    rec = np.take_along_axis(tab.reshape(4, 4, 16), codes.reshape(4, 4, 64), axis=2).reshape(4, 256)
    ours = ((rec - w) ** 2).sum()
    sk = 0.0
    for blk in w.reshape(-1, 64):
        km = KMeans(16, n_init=4, random_state=0).fit(blk[:, None])
        sk += ((km.cluster_centers_[km.labels_, 0] - blk) ** 2).sum()
    assert ours <= 1.6 * sk


def test_bl4_pack_roundtrip_and_dequant_closed_form():
    rng = np.random.default_rng(7)
    codes = rng.integers(0, 16, (3, 128), dtype=np.uint8)
    assert np.array_equal(O.bl4_unpack(O.bl4_pack(codes)), codes)
    tables = O.f32_to_f16(rng.standard_normal((3, 2, 16)).astype(np.float32))
    deq = O.bl4_dequant(O.bl4_pack(codes), tables)
    for r in range(3):
        for c in range(128):
            v = O.f16_to_f32(tables[r, c // 64, codes[r, c]])
            assert deq[r, c] == O.f32_to_bf16(np.float32([v]))[0]


# --------------------------------------------------------------- nested

def test_nested_tiers_refine_and_use_low_bits():
    rng = np.random.default_rng(8)
    w = (rng.standard_normal((16, 256)) * 0.02).astype(np.float32)
    codes, t2, t3, t4 = O.nested_encode(w, n_iter=30)
    errs = []
    for b, t in ((2, t2), (3, t3), (4, t4)):
        rec = O.bf16_to_f32(O.nested_dequant(codes, t, b))
        errs.append(((rec - w) ** 2).mean())
        # tier-b reconstruction depends only on the low b bits
        alt = codes ^ (np.uint8(0xF0) if b == 4 else np.uint8((0xF << b) & 0xF))
        assert np.array_equal(O.nested_dequant(alt, t, b), O.nested_dequant(codes, t, b))
    assert errs[0] > errs[1] > errs[2]
    # descent: the level-2 cell is the argmin over T2
    f2 = O.f16_to_f32(t2).reshape(16, 4, 4)
    for r in range(4):
        for blk in range(4):
            x = w[r, 64 * blk: 64 * blk + 64]
            assert np.array_equal(codes[r, 64 * blk: 64 * blk + 64] & 3,
                                  np.abs(x[:, None] - f2[r, blk][None]).argmin(1))


def test_nested_planes_roundtrip_and_prefix():
    rng = np.random.default_rng(9)
    codes = rng.integers(0, 16, (4, 128), dtype=np.uint8)
    pl = O.nested_pack_planes(codes)
    assert pl["p01"].shape == (4, 32) and pl["p2"].shape == (4, 16)
    for b in (2, 3, 4):
        assert np.array_equal(O.nested_unpack_planes(pl, b), codes & ((1 << b) - 1))


def test_nested_grouped_layout_by_brute_force():
    """Device order of the nested codes: weight i's tier-b code read straight from
    the grouped bytes by the layout rule (group i // 32 at 4b bytes; in the
    group, weight j = n + 8q: its 2-bit field at bits 4n + 2(q % 2) of word q // 2,
    its bit 2 / bit 3 at bit 4n + q of words 2 / 3) equals the plane sections'
    code; ungrouping restores the sections."""
    rng = np.random.default_rng(21)
    M, K = 3, 128
    codes = rng.integers(0, 16, (M, K), dtype=np.uint8)
    pl = O.nested_pack_planes(codes)
    for b in (2, 3, 4):
        buf = np.concatenate([pl["p01"].reshape(-1)] +
                             [pl[p].reshape(-1) for p, bit in (("p2", 2), ("p3", 3)) if b > bit])
        g = O.nested_group_planes(buf, b, M, K)
        assert g.size == M * K * b // 8
        flat = codes.reshape(-1)
        for i in range(M * K):
            grp = g[(i // 32) * 4 * b: (i // 32 + 1) * 4 * b]
            word = [int.from_bytes(grp[4 * w: 4 * w + 4].tobytes(), "little") for w in range(b)]
            j = i % 32
            n, q = j % 8, j // 8
            c = (word[q // 2] >> (4 * n + 2 * (q % 2))) & 3
            if b >= 3:
                c |= ((word[2] >> (4 * n + q)) & 1) << 2
            if b >= 4:
                c |= ((word[3] >> (4 * n + q)) & 1) << 3
            assert c == flat[i] & ((1 << b) - 1), (b, i)
        back = O.nested_ungroup(g, b, M, K)
        ref = O.nested_planes_split(buf, b, M, K)
        assert sorted(back) == sorted(ref)
        for name in ref:
            assert np.array_equal(back[name], ref[name])


def test_nested_exact_with_four_values_at_tier2():
    rng = np.random.default_rng(10)
    vals = (rng.standard_normal(4) * 0.02).astype(np.float32)
    w = rng.choice(vals, size=(1, 64)).astype(np.float32)
    codes, t2, _, _ = O.nested_encode(w, n_iter=20)
    rec = O.f16_to_f32(t2).reshape(4)[codes[0] & 3]
    assert np.array_equal(rec, w[0].astype(np.float16).astype(np.float32))


# ---------------------------------------------------------- routing/permute

def test_route_vs_scipy_softmax_and_argsort():
    from scipy.special import softmax
    rng = np.random.default_rng(11)
    lg = rng.standard_normal((50, 60)).astype(np.float32)
    lg[3, [5, 9, 40]] = 2.5           # ties: lower id first
    w, ids = O.route(lg, 4)
    p = softmax(lg.astype(np.float64), axis=1)
    for t in range(50):
        order = sorted(range(60), key=lambda e: (-lg[t, e], e))[:4]
        assert list(ids[t]) == order
        np.testing.assert_allclose(w[t], p[t, order], rtol=1e-6)
    assert list(ids[3][:3]) == [5, 9, 40]
    wr, _ = O.route(lg, 4, renormalize=True)
    np.testing.assert_allclose(wr.sum(1), 1.0, rtol=1e-6)


def test_permute_brute_force():
    rng = np.random.default_rng(12)
    T, k, E = 37, 3, 9
    ids = np.stack([rng.permutation(E)[:k] for _ in range(T)]).astype(np.int32)
    off, perm, inv = O.permute(ids, E)
    order = [t * k + s for e in range(E) for t in range(T) for s in range(k) if ids[t, s] == e]
    assert list(perm) == order
    assert np.array_equal(inv[perm], np.arange(T * k))
    assert np.array_equal(np.diff(off), np.bincount(ids.reshape(-1), minlength=E))


@pytest.mark.parametrize("repeats", [False, True])
def test_moe_layer_loop_vs_dense_restatement(repeats):
    """The per-expert grouping of oracle.moe_layer against a dense sum over all experts
    weighted by sum_k w[t,k] [ids[t,k] == e].  With repeats, tokens list an expert twice
    (ids the caller passes): both pairs count, as the reference's loop over the k slots
    adds each (vllm_lut/fast_moe.py:58-61)."""
    rng = np.random.default_rng(13)
    T, H, I, E, k = 9, 64, 32, 5, 2
    x = O.f32_to_bf16(rng.standard_normal((T, H)).astype(np.float32))
    W13 = [(rng.standard_normal((2 * I, H)) * 0.1).astype(np.float32) for _ in range(E)]
    W2 = [(rng.standard_normal((H, I)) * 0.1).astype(np.float32) for _ in range(E)]
    w, ids = O.route(rng.standard_normal((T, E)).astype(np.float32), k)
    if repeats:
        ids[::2, 1] = ids[::2, 0]   # every other token: its first expert twice
    got = O.moe_layer(x, ids, w, W13.__getitem__, W2.__getitem__)
    xf = O.bf16_to_f32(x).astype(np.float64)
    dense = np.zeros((T, H))
    for e in range(E):
        gu = xf @ W13[e].astype(np.float64).T
        g, u = gu[:, :I].astype(np.float32), gu[:, I:].astype(np.float32)
        a = O.bf16_to_f32(O.f32_to_bf16(g / (1 + np.exp(-g)) * u)).astype(np.float64)
        y = a @ W2[e].astype(np.float64).T
        gate = (w.astype(np.float64) * (ids == e)).sum(1)
        dense += gate[:, None] * y
    np.testing.assert_allclose(got, dense, rtol=1e-9, atol=1e-12)


def test_moe_layer_swiglu_pinned_by_torch():
    """oracle.moe_layer against the reference's own torch formulation of one expert
    (vllm_lut/moe_layer.py:332-340: gate_up = F.linear(x, W13); gate, up = chunk(2);
    F.silu(gate) * up; F.linear(act, W2)) in float64, with gate rows and up rows drawn
    from different distributions (a gate/up swap, a missing SiLU or a SiLU on the up half
    fails), routed weights applied per slot and a shared expert with weight 1."""
    import torch
    import torch.nn.functional as F
    rng = np.random.default_rng(31)
    T, H, I, E, k = 7, 64, 32, 4, 2
    x = O.f32_to_bf16(rng.standard_normal((T, H)).astype(np.float32))
    W13 = [np.concatenate([(rng.standard_normal((I, H)) * 0.3 + 0.05),      # gate rows [0, I)
                           (rng.standard_normal((I, H)) * 0.1 - 0.02)]).astype(np.float32)  # up rows
           for _ in range(E + 1)]
    W2 = [(rng.standard_normal((H, I)) * 0.1).astype(np.float32) for _ in range(E + 1)]
    w, ids = O.route(rng.standard_normal((T, E)).astype(np.float32), k)
    got = O.moe_layer(x, ids, w, W13.__getitem__, W2.__getitem__, shared=[(W13[E], W2[E])],
                      act_round_bf16=False)
    xt = torch.from_numpy(O.bf16_to_f32(x).astype(np.float64))

    def expert(e, rows):
        gate, up = F.linear(xt[rows], torch.from_numpy(W13[e].astype(np.float64))).chunk(2, dim=-1)
        return F.linear(F.silu(gate) * up, torch.from_numpy(W2[e].astype(np.float64)))

    ref = torch.zeros((T, H), dtype=torch.float64)
    for e in range(E):
        for s in range(k):
            m = torch.from_numpy(ids[:, s] == e)
            if m.any():
                ref[m] += expert(e, m) * torch.from_numpy(w[:, s].astype(np.float64))[m, None]
    ref += expert(E, torch.ones(T, dtype=torch.bool))

    def rel(a, b):   # the oracle's SwiGLU runs in fp32, torch's here in float64
        return np.abs(a - b).max() / np.abs(b).max()

    assert rel(got, ref.numpy()) <= 1e-6
    # the check can fail: swapping the gate and up halves moves the result by O(1)
    swapped = [np.concatenate([m[I:], m[:I]]) for m in W13]
    bad = O.moe_layer(x, ids, w, swapped.__getitem__, W2.__getitem__, shared=[(swapped[E], W2[E])],
                      act_round_bf16=False)
    assert rel(bad, ref.numpy()) > 0.05
    # the per-token shared weights (Qwen's sigmoid gate) scale only the shared expert
    sw = rng.random(T)
    got2 = O.moe_layer(x, ids, w, W13.__getitem__, W2.__getitem__, shared=[(W13[E], W2[E])],
                       act_round_bf16=False, shared_w=sw)
    ref2 = ref - expert(E, torch.ones(T, dtype=torch.bool)) * (1 - torch.from_numpy(sw))[:, None]
    assert rel(got2, ref2.numpy()) <= 1e-6
    # a subset of W2's rows gives those output columns
    cols = np.array([3, 17, 40])
    got3 = O.moe_layer(x, ids, w, W13.__getitem__, lambda e: W2[e][cols], act_round_bf16=False)
    full = O.moe_layer(x, ids, w, W13.__getitem__, W2.__getitem__, act_round_bf16=False)
    np.testing.assert_allclose(got3, full[:, cols], rtol=1e-12, atol=1e-15)


def test_moe_layer_float32_blas_within_1e5_of_float64():
    """The float32 host-BLAS mode of oracle.moe_layer (the full-shape prefill checks: the
    down projection's product in float32) at a prefill-like depth (K = 2048 and 1408) stays
    within 1e-5 relative max-abs of the float64 mode, 100 times inside the 1e-3 bar."""
    rng = np.random.default_rng(41)
    T, H, I, E, k = 48, 2048, 1408, 3, 2
    x = O.f32_to_bf16(rng.standard_normal((T, H)).astype(np.float32))
    W13 = [(rng.standard_normal((2 * I, H)) * 0.02).astype(np.float32) for _ in range(E)]
    W2 = [(rng.standard_normal((H, I)) * 0.02).astype(np.float32) for _ in range(E)]
    w, ids = O.route(rng.standard_normal((T, E)).astype(np.float32), k)
    f64 = O.moe_layer(x, ids, w, W13.__getitem__, W2.__getitem__)
    f32 = O.moe_layer(x, ids, w, W13.__getitem__, W2.__getitem__, blas_dtype=np.float32)
    assert np.abs(f32 - f64).max() / np.abs(f64).max() <= 1e-5


def test_fast_host_dequant_matches_oracle():
    """bl4_dequant_f32 / nested_dequant_f32 (the vectorised host dequantisers of the
    full-shape GPU tests) equal bl4_dequant / nested_dequant, including every fp16 table
    pattern class (zero, subnormal, inf, NaN) and more rows than one gather chunk; the
    bit-plane section split of a device buffer gives back the codes."""
    rng = np.random.default_rng(32)
    M, K = 1030, 128
    p = rng.integers(0, 256, (M, K // 2), dtype=np.uint8)
    t = rng.integers(0, 65536, (M, K // 64, 16), dtype=np.uint16)
    t[0, 0, :6] = [0, 1, 0x3ff, 0x7c00, 0x7e00, 0xfc01]
    got = O.bl4_dequant_f32(p, t, row_chunk=256)
    ref = O.bf16_to_f32(O.bl4_dequant(p, t))
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    for b in (2, 3, 4):
        c = rng.integers(0, 16, (M, K), dtype=np.uint8)
        tb = rng.integers(0, 65536, (M, K // 64, 1 << b), dtype=np.uint16)
        got = O.nested_dequant_f32(c, tb, b, row_chunk=300)
        ref = O.bf16_to_f32(O.nested_dequant(c, tb, b))
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), b
        pl = O.nested_pack_planes(c)
        buf = np.concatenate([pl["p01"].reshape(-1)] + [pl[n].reshape(-1) for n in ("p2", "p3")][: b - 2])
        back = O.nested_unpack_planes(O.nested_planes_split(buf, b, M, K), b)
        assert np.array_equal(back, c & ((1 << b) - 1)), b


def test_cpu_baseline_dequant_matches_oracle():
    import torch
    from oracle.cpu_baseline import bl4_dequant_torch
    rng = np.random.default_rng(14)
    codes = rng.integers(0, 256, (8, 64), dtype=np.uint8)
    tab16 = O.f32_to_f16(rng.standard_normal((8, 2, 16)).astype(np.float32))
    tb = torch.from_numpy(O.bl4_tables_bf16(tab16).view(np.int16)).view(torch.bfloat16)
    got = bl4_dequant_torch(torch.from_numpy(codes), tb).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, O.bl4_dequant(codes, tab16))


def test_product_nested_table_helpers_match_the_oracle():
    """block_lut_amd.quantizer.greedy_merge / build_mapped_table (host code of the product)
    against the oracle's restatements, which the reference's golden vectors pin; the
    merge's effective rule (the first two entries, every step) on unsorted input too."""
    import torch
    from block_lut_amd.quantizer import build_mapped_table, greedy_merge
    rng = np.random.default_rng(21)
    for n, tk in ((64, 16), (40, 7), (16, 16)):
        c = rng.standard_normal(n).astype(np.float32)
        got = greedy_merge(torch.from_numpy(c), tk).numpy()
        assert np.array_equal(got, O.greedy_merge_ref(c, tk))
    for k in (16, 64, 100, 256):
        c = np.sort(rng.standard_normal(k)).astype(np.float32)
        got = build_mapped_table(torch.from_numpy(c), 256).view(torch.int16).numpy().view(np.uint16)
        assert np.array_equal(got, O.build_mapped_table_ref(c, 256))
