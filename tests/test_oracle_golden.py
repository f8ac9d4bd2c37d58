"""The oracle pinned against vectors written from the reference itself
(tests/golden/make_golden.py) and against the reference's shipped codebook
tables.  CPU only."""
import os

import numpy as np
import pytest

import oracle as O

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module")
def qv():
    return np.load(os.path.join(GOLDEN, "quantizer.npz"), allow_pickle=False)


@pytest.fixture(scope="module")
def cbk():
    return np.load(os.path.join(GOLDEN, "codebooks.npz"), allow_pickle=False)


# ----------------------------------------------------- LUTQuantizer.quantize

def test_ref_quantize_f32(qv, cbk):
    idx, am = O.ref_quantize(qv["q_f32_w"], cbk["qwen_blocklut_256_bf16"], 128)
    assert np.array_equal(idx, qv["q_f32_idx"])
    assert np.array_equal(am, qv["q_f32_absmax"])


def test_ref_quantize_padded_tail_and_zero_block(qv, cbk):
    idx, am = O.ref_quantize(qv["q_pad_w"], cbk["qwen_blocklut_256_bf16"], 128)
    assert idx.size == qv["q_pad_w"].size
    assert np.array_equal(idx, qv["q_pad_idx"])
    assert np.array_equal(am, qv["q_pad_absmax"])


def test_ref_quantize_bf16_input(qv, cbk):
    w = O.bf16_to_f32(qv["q_bf16_w"])
    idx, am = O.ref_quantize(w, cbk["qwen_blocklut_256_bf16"], 128, input_is_bf16=True)
    assert np.array_equal(idx, qv["q_bf16_idx"])
    assert np.array_equal(am, qv["q_bf16_absmax"])


def test_ref_quantize_bf16_path_matters(qv, cbk):
    """The fp32-normalisation restatement must NOT reproduce the bf16 vectors:
    a dropped bf16 rounding of x/absmax would be caught."""
    w = O.bf16_to_f32(qv["q_bf16_w"])
    idx, _ = O.ref_quantize(w, cbk["qwen_blocklut_256_bf16"], 128, input_is_bf16=False)
    assert not np.array_equal(idx, qv["q_bf16_idx"])


# --------------------------------------------------- training / merging

@pytest.mark.parametrize("seed,k,it", [(0, 16, 5), (3, 64, 8)])
def test_train_kmeans(qv, seed, k, it):
    got = O.train_kmeans_ref(qv["km_data"], k, it, seed)
    assert np.array_equal(got, qv[f"km_s{seed}_k{k}_it{it}"])


def test_train_kmeans_subsample_path(qv):
    import sys
    sys.path.insert(0, GOLDEN)
    from make_golden import km_big_data
    got = O.train_kmeans_ref(km_big_data(), 16, 3, 11)
    assert np.array_equal(got, qv["km_big_s11_k16_it3"])


def test_greedy_merge(qv):
    got = O.greedy_merge_ref(qv["gm_in"], 16)
    np.testing.assert_array_equal(got, qv["gm_out"])


def test_build_mapped_table_closed_form():
    c = np.sort(np.random.default_rng(0).standard_normal(64).astype(np.float32))
    t = O.build_mapped_table_ref(c, 256)
    assert t.size == 256
    assert np.array_equal(t, O.f32_to_bf16(np.tile(c, 4)))
    c16 = c[:16]
    t16 = O.build_mapped_table_ref(c16, 256)
    assert float(O.bf16_to_f32(t16)[17]) == float(O.bf16_to_f32(O.f32_to_bf16(c16[1:2]))[0])


# ------------------------------------------------- shipped nested tables

def test_nested_prefix_pad_matches_shipped_qwen_tables(cbk):
    """models/qwen/nested_lut_mapped{16,64}.npy = bf16(pad(sorted blocklut_256[:K]))
    (llama-cpp-port/scripts/convert_lut.py:113-140)."""
    full, m64, m16 = O.nested_tables_prefix_pad(np.sort(cbk["qwen_blocklut_256_f32"]))
    assert np.array_equal(m16, cbk["qwen_nested_lut_mapped16_u16"])
    assert np.array_equal(m64, cbk["qwen_nested_lut_mapped64_u16"])
    assert np.array_equal(full, O.f32_to_bf16(np.sort(cbk["qwen_blocklut_256_f32"])))


def test_nested_merge_map_matches_shipped_deepseek_tables(cbk):
    """models/deepseek/nested_lut_mapped{16,64}.npy = bf16(C_K[map256toK])
    (evaluation/generate_nested_lut.py:93-176)."""
    for K in (16, 64):
        got = O.nested_tables_merge_map(cbk[f"deepseek_nested_lut_{K}_f32"],
                                        cbk[f"deepseek_nested_map_256to{K}_u8"])
        assert np.array_equal(got, cbk[f"deepseek_nested_lut_mapped{K}_u16"])
        # the merge maps are monotone (a nested, order-preserving merge)
        assert np.all(np.diff(cbk[f"deepseek_nested_map_256to{K}_u8"].astype(int)) >= 0)


def test_prefix_pad_would_not_match_deepseek(cbk):
    """A mix-up of the two shipped constructions is caught."""
    _, _, m16 = O.nested_tables_prefix_pad(np.sort(cbk["deepseek_blocklut_256_f32"]))
    assert not np.array_equal(m16, cbk["deepseek_nested_lut_mapped16_u16"])


def test_tier_dequant_uses_shipped_tables(cbk):
    """REF tier reconstruction: tier 2 reads the low nibble, tier 1 six bits, each
    through its shipped 256-entry table (model_topology.cpp:597-619)."""
    rng = np.random.default_rng(1)
    n = 1024
    codes = rng.integers(0, 256, n, dtype=np.uint8)
    packed = O.bitplane_pack_ref(codes)
    am = O.f32_to_bf16(np.abs(rng.standard_normal(n // 128)).astype(np.float32))
    t16 = cbk["qwen_nested_lut_mapped16_u16"]
    t64 = cbk["qwen_nested_lut_mapped64_u16"]
    full = O.f32_to_bf16(np.sort(cbk["qwen_blocklut_256_f32"]))
    assert np.array_equal(O.ref_tier_dequant(packed, am, t16, n, 2), O.ref_dequant(codes & 0x0F, am, t16))
    assert np.array_equal(O.ref_tier_dequant(packed, am, t64, n, 1), O.ref_dequant(codes & 0x3F, am, t64))
    assert np.array_equal(O.ref_tier_dequant(packed, am, full, n, 0), O.ref_dequant(codes, am, full))
