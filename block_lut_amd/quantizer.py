"""Codebook training behind the reference's LUTQuantizer
(vllm_lut/quantizer.py: `LUTQuantizer._train_kmeans`, :120-178).

`train_kmeans(data, k, n_iter)` returns the sorted bf16[k] codebook on the host, as the
reference stores `lut_codebook`.  Subsampling (more than `max_samples` values: a random
subset, :142-147) and the initial pick (k random samples, zeros when there are fewer,
:150-156) use torch's permutation generator, seeded like the reference's; the Lloyd
iterations (:158-173) run on the GPU (`lutmoe_kmeans_1d`); the sort and the bf16 store
(:176-177) follow.  There is no CPU path.
"""
from __future__ import annotations

from typing import Optional

import torch

from . import _native as N
from .formats import _dev, _stream

__all__ = ["train_kmeans", "greedy_merge", "build_mapped_table", "train_nested_codebooks"]


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
