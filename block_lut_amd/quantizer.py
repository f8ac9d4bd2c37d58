"""Codebook training and REF encoding behind the reference's LUTQuantizer
(vllm_lut/quantizer.py: `LUTQuantizer`, :30-396; `_train_kmeans`, :120-178).

`train_kmeans(data, k, n_iter)` returns the sorted bf16[k] codebook on the host, as the
reference stores `lut_codebook`.  Subsampling (more than `max_samples` values: a random
subset, :142-147) and the initial pick (k random samples, zeros when there are fewer,
:150-156) use torch's permutation generator, seeded like the reference's; the Lloyd
iterations (:158-173) run on the GPU (`lutmoe_kmeans_1d`); the sort and the bf16 store
(:176-177) follow.  There is no CPU path.
"""
from __future__ import annotations

import os
from typing import Dict, Optional, Tuple

import numpy as np
import torch

from . import _native as N
from .formats import _dev, _stream

__all__ = ["train_kmeans", "greedy_merge", "build_mapped_table", "train_nested_codebooks", "quantize",
           "LUTQuantizer", "cluster_counts", "merge_map", "merge_map_tables"]


def train_kmeans(data: torch.Tensor, k: int = 256, n_iter: int = 20, max_samples: int = 200000,
                 seed: Optional[int] = None, device=None) -> torch.Tensor:
    """1-D k-means codebook of `data` (any shape; flattened), bf16 [k] sorted, on the host.

    `seed` seeds a private permutation generator (the same stream as the reference's
    after `torch.manual_seed(seed)`); None draws from torch's default generator.  The
    training samples live on `device` (default: `data`'s device, which must be a GPU)."""
    dev = torch.device(device) if device is not None else data.device
    if dev.type != "cuda":
        raise ValueError("train_kmeans runs on the GPU: pass a device tensor or device='cuda'")
    if not 1 <= k <= 256:
        raise ValueError("k must be in [1, 256]")
    x = data.reshape(-1).to(dev, torch.float32)
    gen = torch.Generator().manual_seed(int(seed)) if seed is not None else None
    n_total = x.numel()
    if n_total == 0:
        raise ValueError("no training data")
    if n_total > max_samples:
        sub = torch.randperm(n_total, generator=gen)[:max_samples]
        train = x[sub.to(dev)].contiguous()
    else:
        train = x.contiguous()
    n = train.numel()
    n_init = min(k, n)
    pick = torch.randperm(n, generator=gen)[:n_init]
    cent = torch.zeros(k, dtype=torch.float32, device=dev)
    cent[:n_init] = train[pick.to(dev)]
    asg = torch.empty(n, dtype=torch.int32, device=dev)
    _dev(train, torch.float32, "train")
    N.check("lutmoe_kmeans_1d", N.lib().lutmoe_kmeans_1d(train.data_ptr(), n, cent.data_ptr(), k, int(n_iter),
                                                         asg.data_ptr(), _stream()))
    cent, _ = torch.sort(cent)
    return cent.to(torch.bfloat16).cpu()


def greedy_merge(centroids: torch.Tensor, target_k: int) -> torch.Tensor:
    """LUTQuantizer._greedy_merge (vllm_lut/quantizer.py:202-221), in the dtype of
    `centroids`, on the host.  The reference looks for the closest pair in |c_a - c_b|
    plus eye * inf; off the diagonal that sum is NaN (0 * inf), and torch's argmin returns
    the first NaN, i.e. the pair (0, 1).  Its effective rule, kept here: while more than
    `target_k` entries remain, the first entry becomes the mean of the first two and the
    second is dropped; the result is sorted."""
    c = centroids.detach().cpu().clone()
    while c.numel() > target_k:
        c = torch.cat([((c[0] + c[1]) / 2).reshape(1), c[2:]])
    return torch.sort(c).values


def build_mapped_table(centroids: torch.Tensor, table_size: int = 256) -> torch.Tensor:
    """LUTQuantizer._build_mapped_table (vllm_lut/quantizer.py:223-236): the centroids
    repeated to `table_size` entries (then the first `table_size % k` once more), bf16,
    on the host."""
    c = centroids.detach().cpu()
    k = c.numel()
    if table_size < k:
        raise ValueError("table_size must be at least the number of centroids")
    parts = [c.repeat(table_size // k)]
    if table_size % k:
        parts.append(c[:table_size % k])
    return torch.cat(parts).to(torch.bfloat16)


def train_nested_codebooks(data: torch.Tensor, n_iter: int = 20, seed: Optional[int] = None,
                           device=None):
    """LUTQuantizer._train_nested_codebooks (vllm_lut/quantizer.py:180-200): a 64-entry
    codebook trained like the full one (`train_kmeans`, bf16), 16 entries derived from it
    by `greedy_merge` (in bf16, as the reference's bf16 codebook), and both as 256-entry
    tables.  Returns (mapped64, mapped16), bf16 [256] each, on the host."""
    c64 = train_kmeans(data, 64, n_iter, seed=seed, device=device)
    c16 = greedy_merge(c64, 16)
    return build_mapped_table(c64, 256), build_mapped_table(c16, 256)


_RULES = {"quantizer": N.QRULE_QUANTIZER, "midpoints": N.QRULE_MIDPOINTS}


def quantize(weight: torch.Tensor, codebook: torch.Tensor, block_size: int = 128,
             rule: str = "quantizer") -> Tuple[torch.Tensor, torch.Tensor]:
    """REF codes of `weight` (bf16 or fp32, any shape, flattened) on the GPU: uint8 [N]
    codes and bf16 [ceil(N / block_size)] absmax, device tensors, no host sync.

    rule "quantizer": LUTQuantizer.quantize (vllm_lut/quantizer.py:242-306): normalisation
        in the weights' dtype, code = first nearest entry of `codebook` (bf16 or fp32, any
        order, at most 256 entries).
    rule "midpoints": the offload runtime's encoder (runtime/model_offload.py:897-907):
        fp32 normalisation, code = np.searchsorted over the midpoints of `codebook`, which
        must be ascending (the runtime sorts its table first)."""
    if rule not in _RULES:
        raise ValueError(f"rule must be one of {sorted(_RULES)}")
    w = weight.reshape(-1)
    if w.dtype not in (torch.bfloat16, torch.float32):
        w = w.float()
    w = _dev(w.contiguous(), w.dtype, "weight")
    cb = codebook.reshape(-1).to(w.device, torch.float32).contiguous()
    k = cb.numel()
    if not 1 <= k <= 256:
        raise ValueError("the codebook holds 1..256 entries")
    if rule == "midpoints" and bool((cb[1:] < cb[:-1]).any()):
        raise ValueError("rule 'midpoints' needs an ascending codebook")
    n = w.numel()
    nb = -(-n // block_size) if n else 0
    codes = torch.empty(n, dtype=torch.uint8, device=w.device)
    absmax = torch.empty(nb, dtype=torch.bfloat16, device=w.device)
    dt = N.DTYPE_BF16 if w.dtype == torch.bfloat16 else N.DTYPE_F32
    N.check("lutmoe_ref_quantize",
            N.lib().lutmoe_ref_quantize(w.data_ptr(), dt, cb.data_ptr(), k, n, block_size, _RULES[rule],
                                        codes.data_ptr(), absmax.data_ptr(), _stream()))
    return codes, absmax


class LUTQuantizer:
    """vllm_lut/quantizer.py:30-396 with the GPU doing the work: `train` (block
    normalisation, then the k-means of `train_kmeans`; NESTEDLUT also the nested
    tables), `quantize` (the REF codes of one weight tensor, `quantize(rule="quantizer")`),
    `decompress` (the REF dequantisation kernel) and `save` / `load` of the codebooks.
    Results of `quantize` are host tensors, as the reference returns them."""

    def __init__(self, code_type: str = "BLOCKLUT", block_size: int = 128, lut_size: int = 256,
                 device: str = "cuda"):
        if code_type not in ("LUT", "BLOCKLUT", "NESTEDLUT"):
            raise ValueError(f"Unsupported code_type: {code_type}")
        self.code_type = code_type
        self.block_size = block_size
        self.lut_size = lut_size
        self.device = device
        self.lut_codebook: Optional[torch.Tensor] = None       # [256] bf16
        self.nested_mapped64: Optional[torch.Tensor] = None    # [256] bf16
        self.nested_mapped16: Optional[torch.Tensor] = None    # [256] bf16

    def _normalised(self, flat: torch.Tensor) -> torch.Tensor:
        """Block normalisation of quantizer.py:86-104 in the tensor's dtype."""
        n = flat.numel()
        nb = -(-n // self.block_size)
        if nb * self.block_size != n:
            flat = torch.cat([flat, flat.new_zeros(nb * self.block_size - n)])
        blocks = flat.view(-1, self.block_size)
        am = blocks.abs().amax(dim=1, keepdim=True).clamp(min=1e-10)
        return (blocks / am).reshape(-1)

    @torch.no_grad()
    def train(self, expert_weights: torch.Tensor, n_iter: int = 50, seed: Optional[int] = None) -> None:
        """Codebook(s) from expert weights [E, rows, cols] or any shape (quantizer.py:65-114)."""
        flat = expert_weights.reshape(-1).to(self.device)
        data = flat if self.code_type == "LUT" else self._normalised(flat)
        self.lut_codebook = train_kmeans(data, self.lut_size, n_iter, seed=seed)
        if self.code_type == "NESTEDLUT":
            self.nested_mapped64, self.nested_mapped16 = train_nested_codebooks(data, n_iter, seed=seed)

    @torch.no_grad()
    def quantize(self, weight: torch.Tensor, codebook: Optional[torch.Tensor] = None) -> Dict[str, torch.Tensor]:
        """{'indices': uint8 [N], 'absmax': bf16 [nb], 'codebook': bf16 [256]} on the host
        (quantizer.py:242-306; the LUT code type normalises by one global absmax)."""
        if codebook is None:
            codebook = self.lut_codebook
        if codebook is None:
            raise RuntimeError("LUT codebook not trained or loaded. Call train() or load() first.")
        w = weight.to(self.device)
        bs = self.block_size if self.code_type != "LUT" else max(1, w.numel())
        codes, absmax = quantize(w, codebook.to(torch.bfloat16), bs, rule="quantizer")
        return {"indices": codes.cpu(), "absmax": absmax.cpu(), "codebook": codebook.to(torch.bfloat16).cpu()}

    @torch.no_grad()
    def decompress(self, indices: torch.Tensor, absmax: torch.Tensor, codebook: torch.Tensor,
                   out_shape: Optional[Tuple[int, ...]] = None) -> torch.Tensor:
        """bf16(codebook[index] * absmax[block]) on the GPU (quantizer.py:312-353); one
        absmax entry scales every weight, as for the LUT code type."""
        from .decompress import decompress_blocklut
        dev = torch.device(self.device)
        out = decompress_blocklut(indices.to(dev).reshape(-1), absmax.to(dev, torch.bfloat16).reshape(-1),
                                  codebook.to(dev, torch.bfloat16), self.block_size)
        return out.reshape(out_shape) if out_shape is not None else out

    def save(self, path: str) -> None:
        """The codebooks as .npy files with the reference's names (quantizer.py:359-371),
        holding their float32 values (numpy has no bf16; `load` restores the bf16 values)."""
        os.makedirs(path, exist_ok=True)
        for t, name in ((self.lut_codebook, "blocklut_256.npy"), (self.nested_mapped64, "nested_lut_mapped64.npy"),
                        (self.nested_mapped16, "nested_lut_mapped16.npy")):
            if t is not None:
                np.save(os.path.join(path, name), t.float().cpu().numpy())

    def load(self, path: str) -> bool:
        """quantizer.py:373-396: blocklut_256.npy (or full256.npy) and the optional nested
        tables, as bf16.  False when no codebook file is there."""
        for name in ("blocklut_256.npy", "full256.npy"):
            f = os.path.join(path, name)
            if os.path.exists(f):
                self.lut_codebook = torch.from_numpy(np.load(f, allow_pickle=False)).to(torch.bfloat16)
                break
        else:
            return False
        for attr, name in (("nested_mapped64", "nested_lut_mapped64.npy"),
                           ("nested_mapped16", "nested_lut_mapped16.npy")):
            f = os.path.join(path, name)
            if os.path.exists(f):
                setattr(self, attr, torch.from_numpy(np.load(f, allow_pickle=False)).to(torch.bfloat16))
        return True


# ---------------------------------------------------------------- merge-map nested tables
# evaluation/generate_nested_lut.py:93-176, 264-269: the 256 sorted centroids are merged
# greedily into K of them (adjacent pairs, cheapest weighted-MSE increase first), and the
# tier-K table is indexed by the full 8-bit code through a 256 -> K map.

def cluster_counts(data: torch.Tensor, centroids: torch.Tensor) -> np.ndarray:
    """Samples per centroid (nearest of the ascending `centroids`, the lower one on a
    midpoint), counted on `data`'s device: the weights of generate_nested_lut.py:68-85."""
    c = centroids.reshape(-1).to(data.device, torch.float32)
    mid = (c[:-1] + c[1:]) * 0.5
    idx = torch.bucketize(data.reshape(-1).float(), mid)
    return torch.bincount(idx, minlength=c.numel()).cpu().numpy().astype(np.int64)


def merge_map(centroids, counts, target_k: int):
    """generate_nested_lut.greedy_merge (:93-176) on the host.  Returns (merged centroids
    float32 [K'], their counts int64 [K'], map uint8 [K] original index -> merged index).

    The reference's effective rules, kept because its shipped tables follow them:
      * the candidate adjacent pairs live in a priority queue ordered by (cost, left index,
        right index), cost = w_a w_b (c_a - c_b)^2 / (w_a + w_b) in float64; a popped pair
        is taken when both ends are alive and adjacent, so a pair whose left end grew since
        it was queued can still be taken at its old cost;
      * the right end merges into the left (weighted mean, summed weight); the left keeps
        its index;
      * a merged-away index maps to the first surviving index at or to its right (the
        last survivor if none), i.e. to the group after the one that absorbed it."""
    import heapq
    c = np.asarray(centroids, np.float64).reshape(-1).copy()
    w = np.asarray(counts, np.float64).reshape(-1).copy()
    K = c.size
    if target_k >= K:
        return c.astype(np.float32), w.astype(np.int64), np.arange(K, dtype=np.uint8)
    alive = np.ones(K, bool)
    right = np.arange(1, K + 1)        # next alive index (K = none)
    left = np.arange(-1, K - 1)        # previous alive index (-1 = none)

    def cost(a, b):
        return w[a] * w[b] * (c[a] - c[b]) ** 2 / (w[a] + w[b])

    queue = [(cost(a, a + 1), a, a + 1) for a in range(K - 1)]
    heapq.heapify(queue)
    for _ in range(K - target_k):
        while queue:
            _, a, b = heapq.heappop(queue)
            if alive[a] and alive[b] and right[a] == b:
                break
        else:
            break
        c[a] = (w[a] * c[a] + w[b] * c[b]) / (w[a] + w[b])
        w[a] += w[b]
        alive[b] = False
        right[a] = right[b]
        if right[a] < K:
            left[right[a]] = a
        if left[a] >= 0 and alive[left[a]]:
            heapq.heappush(queue, (cost(left[a], a), left[a], a))
        if right[a] < K and alive[right[a]]:
            heapq.heappush(queue, (cost(a, right[a]), a, right[a]))
    surv = np.flatnonzero(alive)
    rank = np.searchsorted(surv, np.arange(K))                 # first survivor at or right of i
    mapping = np.where(rank < surv.size, rank, surv.size - 1)
    # none at or right of i: the nearest to its left (the last survivor)
    return c[surv].astype(np.float32), w[surv].astype(np.int64), mapping.astype(np.uint8)


def merge_map_tables(centroids, counts, ks=(64, 16)) -> Dict[int, Dict[str, np.ndarray]]:
    """For each K in `ks`: {'lut': float32 [K], 'map': uint8 [256], 'mapped': bf16 bits
    uint16 [256] = bf16(lut[map])}, the nested_lut_K / nested_map_256toK /
    nested_lut_mappedK files of generate_nested_lut.py:264-269, from the 256 ascending
    centroids and their counts."""
    out = {}
    for k in ks:
        lut, _, mp = merge_map(centroids, counts, k)
        mapped = torch.from_numpy(lut[mp.astype(np.int64)]).to(torch.bfloat16).view(torch.int16).numpy()
        out[k] = {"lut": lut, "map": mp, "mapped": mapped.view(np.uint16)}
    return out
