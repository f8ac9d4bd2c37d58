"""Merge-map nested tables (quantizer.merge_map / merge_map_tables, the procedure of
evaluation/generate_nested_lut.py:93-176) on the host, pinned by the reference's shipped
DeepSeek tables and by the invariants of a weighted greedy merge.  CPU only."""
import os

import numpy as np
import torch

import oracle as O
from block_lut_amd import quantizer as Q

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _shipped():
    return np.load(os.path.join(GOLDEN, "codebooks.npz"), allow_pickle=False)


def test_shipped_deepseek_tables_follow_the_mapping_rule():
    """models/deepseek/nested_lut_{64,16}.npy with nested_map_256to{64,16}.npy: under the
    reference's mapping (a merged-away index maps to the first survivor at or right of
    it) the survivors are the last index of each run of equal map values, and every
    merged centroid lies inside its group [s_r, s_(r+1)) of the sorted 256 centroids,
    as a weighted mean must; grouping by the runs themselves (a left-walking map) does
    not fit the shipped values."""
    d = _shipped()
    c = np.sort(d["deepseek_blocklut_256_f32"])
    for K in (64, 16):
        m = d[f"deepseek_nested_map_256to{K}_u8"].astype(int)
        lut = d[f"deepseek_nested_lut_{K}_f32"]
        assert np.all(np.diff(m) >= 0) and m[0] == 0 and m[-1] == K - 1
        ends = [i for i in range(256) if i == 255 or m[i + 1] != m[i]]
        starts = [i for i in range(256) if i == 0 or m[i - 1] != m[i]]
        inside = []
        for r in range(K):
            # the last survivor sits somewhere in the last run
            g = c[ends[r]:ends[r + 1]] if r + 1 < K else c[ends[r - 1] + 1:]
            inside.append(g.min() <= lut[r] <= g.max())
        assert all(inside), [r for r, ok in enumerate(inside) if not ok]
        runs = [c[starts[r]:(starts[r + 1] if r + 1 < K else 256)] for r in range(K)]
        assert sum(g.min() <= lut[r] <= g.max() for r, g in enumerate(runs)) < K // 2


def test_merge_map_invariants():
    """Random centroids and counts: weights sum, the weighted sum is kept, each merged
    centroid is the weighted mean of its group [s_r, s_(r+1)) with the survivors read off
    the map as run ends (the last run holds the last survivor), sizes; target >= K is the
    identity."""
    rng = np.random.default_rng(7)
    c = np.sort(rng.standard_normal(256)).astype(np.float32)
    w = rng.integers(1, 500, 256)
    for K in (64, 16, 3):
        lut, cnt, mp = Q.merge_map(c, w, K)
        assert lut.size == K and cnt.sum() == w.sum() and mp.size == 256
        ends = [i for i in range(256) if i == 255 or mp[i + 1] != mp[i]]
        assert len(ends) == K and np.all(np.diff(mp.astype(int)) >= 0)
        # survivors 0 .. K-2 are the first K-1 run ends; the last one lies in the last run
        for r in range(K - 2):
            g = slice(ends[r], ends[r + 1])
            mean = (c[g].astype(np.float64) * w[g]).sum() / w[g].sum()
            assert abs(mean - lut[r]) <= 1e-6 * max(1.0, abs(mean)), (K, r)
            assert cnt[r] == w[g].sum()
        tot = (c.astype(np.float64) * w).sum()
        assert abs((lut.astype(np.float64) * cnt).sum() - tot) <= 1e-5 * np.abs(c * w).sum()
    lut, cnt, mp = Q.merge_map(c[:10], w[:10], 12)
    assert np.array_equal(mp, np.arange(10)) and np.array_equal(lut, c[:10])


def test_merge_map_takes_the_cheapest_adjacent_pair_first():
    """One merge: the pair with the smallest w_a w_b (c_a - c_b)^2 / (w_a + w_b), the lower
    index on equal costs (a planted tie between two identical pairs)."""
    rng = np.random.default_rng(9)
    c = np.sort(rng.standard_normal(40)).astype(np.float64)
    w = rng.integers(1, 50, 40).astype(np.float64)
    cost = w[:-1] * w[1:] * (c[:-1] - c[1:]) ** 2 / (w[:-1] + w[1:])
    a = int(np.argmin(cost))
    lut, _, mp = Q.merge_map(c, w, 39)
    assert mp[a + 1] != mp[a] and lut.size == 39
    assert abs(lut[a] - (w[a] * c[a] + w[a + 1] * c[a + 1]) / (w[a] + w[a + 1])) < 1e-6
    t = np.array([0.0, 1.0, 5.0, 6.0, 10.0])
    tw = np.ones(5)
    lut, _, _ = Q.merge_map(t, tw, 4)
    assert np.allclose(lut, [0.5, 5.0, 6.0, 10.0])


def test_merge_map_tables_and_counts():
    """merge_map_tables' mapped table is the merge-map rule the shipped mapped tables pin
    (oracle.nested_tables_merge_map); cluster_counts is the nearest-centroid histogram."""
    rng = np.random.default_rng(11)
    c = np.sort(rng.standard_normal(256)).astype(np.float32)
    data = torch.from_numpy(rng.standard_normal(20000).astype(np.float32))
    cnt = Q.cluster_counts(data, torch.from_numpy(c))
    near = np.abs(data.numpy()[:, None] - c[None, :]).argmin(1)
    assert np.array_equal(cnt, np.bincount(near, minlength=256))
    t = Q.merge_map_tables(c, cnt, ks=(64, 16))
    for K in (64, 16):
        assert np.array_equal(t[K]["mapped"], O.nested_tables_merge_map(t[K]["lut"], t[K]["map"]))
