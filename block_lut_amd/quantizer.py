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

__all__ = ["train_kmeans"]


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
