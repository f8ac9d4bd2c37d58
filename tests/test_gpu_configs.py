"""The configured workloads, each run whole on the GPU at its own shape and checked
against the float64 oracle (the Qwen decode layer at T = 1 / 8 / 32 is in
test_gpu_parity.py).

Weights are random stacks in their wire formats (tests/gpu_weights.py); the oracle
dequantises them on the host from the codes.  Every token row of every output is
checked (Mixtral: every token on 384 sampled output columns, which keeps the host
copy of its down projection small); the prefill-sized oracles run their matrix
down projections in float32 host BLAS (relative error near 1e-6; the gate/up products, rounded to bf16, stay float64).  Bar as in
test_gpu_parity.py: max|y - y_ref| / max|y_ref| <= 1e-3, fp32 output.
"""
import numpy as np
import pytest

import oracle as O
from gpu_weights import DevBL4, DevNested
from lutmoe_testutil import rel_maxabs, to_dev_bf16

pytestmark = pytest.mark.gpu
TOL = 1e-3


def _x(rng, T, K):
    return O.f32_to_bf16(rng.standard_normal((T, K)).astype(np.float32))


def test_config_deepseek_v2_lite_prefill(gpu):
    """DeepSeek-V2-Lite-shaped layer prefill: H2048, I1408, 64 routed experts top-6 plus 2
    always-on shared experts, all BL4; 2048 tokens of N(0,1) bf16 activations and N(0,1)
    router logits; the block forward from logits (GPU top-k, permutation, grouped MFMA
    LUT-GEMMs, combine)."""
    import torch
    from block_lut_amd import ops
    from block_lut_amd.formats import MoEWeights
    H, I, E, S, k, T = 2048, 1408, 64, 2, 6, 2048
    g = torch.Generator(device=gpu).manual_seed(2048)
    w13 = DevBL4(E + S, 2 * I, H, g, gpu)
    w2 = DevBL4(E + S, H, I, g, gpu)
    moe = MoEWeights(w13.stack, w2.stack, H, I, E, S)
    rng = np.random.default_rng(3)
    xb = _x(rng, T, H)
    lg = rng.standard_normal((T, E)).astype(np.float32)
    out = ops.moe_forward_logits(moe, to_dev_bf16(xb, gpu), torch.from_numpy(lg).to(gpu), k,
                                 out_dtype=torch.float32).cpu().numpy()
    assert np.isfinite(out).all()
    rw, rids = O.route(lg, k)
    ref = O.moe_layer(xb, rids, rw, w13.host, w2.host,
                      shared=[(w13.host(E + s), w2.host(E + s)) for s in range(S)], blas_dtype=np.float32)
    assert rel_maxabs(out, ref) <= TOL


def test_config_mixtral_layer(gpu):
    """One Mixtral-8x7B-shaped layer (H4096, I14336, 8 experts top-2 with renormalisation,
    BL4, 1.41 GB resident): decode B=1 (grouped LUT-GEMV) and B=64 (grouped MFMA with the
    down projection's K split in two), prefill 4096 tokens; every token row checked on 384
    sampled output columns."""
    import torch
    from block_lut_amd import ops
    from block_lut_amd.formats import MoEWeights
    H, I, E, k = 4096, 14336, 8, 2
    g = torch.Generator(device=gpu).manual_seed(8)
    w13 = DevBL4(E, 2 * I, H, g, gpu)
    w2 = DevBL4(E, H, I, g, gpu)
    moe = MoEWeights(w13.stack, w2.stack, H, I, E, 0)
    rng = np.random.default_rng(87)
    cols = np.unique(np.concatenate([[0, 1, 255, 256, H - 1], rng.choice(H, 379, replace=False)]))
    for T in (1, 64, 4096):
        xb = _x(rng, T, H)
        lg = rng.standard_normal((T, E)).astype(np.float32)
        out = ops.moe_forward_logits(moe, to_dev_bf16(xb, gpu), torch.from_numpy(lg).to(gpu), k,
                                     renormalize=True, out_dtype=torch.float32).cpu().numpy()
        assert np.isfinite(out).all(), T
        rw, rids = O.route(lg, k, renormalize=True)
        ref = O.moe_layer(xb, rids, rw, w13.host, lambda e: w2.host(e, rows=cols), blas_dtype=np.float32)
        assert rel_maxabs(out[:, cols], ref) <= TOL, T


@pytest.mark.parametrize("T", [16, 1024])
def test_config_nested_tiers_qwen(gpu, T):
    """NestedLUT tiers on the Qwen1.5-MoE shape (H2048, I1408, 60 experts top-4): 20 experts
    each at 2, 3 and 4 bits (seeded permutation); expert popularity p_e ~ rank^-1.1 (Zipf,
    seeded ranks) with Gumbel-top-4 routing (logits = log p_e + Gumbel noise, so the layer's
    own softmax / top-k makes the selection).  Decode T=16 and prefill T=1024, every token
    checked."""
    import torch
    from block_lut_amd import ops
    from block_lut_amd.formats import MoEWeights
    H, I, E, k = 2048, 1408, 60, 4
    rng = np.random.default_rng(2024)
    bits = np.array([2] * 20 + [3] * 20 + [4] * 20)[rng.permutation(E)]
    rank = rng.permutation(E) + 1
    p = rank.astype(np.float64) ** -1.1
    logp = np.log(p / p.sum())
    g = torch.Generator(device=gpu).manual_seed(11)
    w13 = DevNested(bits, 2 * I, H, g, gpu)
    w2 = DevNested(bits, H, I, g, gpu)
    moe = MoEWeights(w13.stack, w2.stack, H, I, E, 0)
    rng = np.random.default_rng(T)
    xb = _x(rng, T, H)
    lg = (logp[None, :] + rng.gumbel(size=(T, E))).astype(np.float32)
    out = ops.moe_forward_logits(moe, to_dev_bf16(xb, gpu), torch.from_numpy(lg).to(gpu), k,
                                 out_dtype=torch.float32).cpu().numpy()
    assert np.isfinite(out).all()
    rw, rids = O.route(lg, k)
    counts = np.bincount(rids.reshape(-1), minlength=E)
    assert counts.max() >= 2 * counts[counts > 0].mean()   # the routing is skewed
    ref = O.moe_layer(xb, rids, rw, w13.host, w2.host, blas_dtype=np.float32)
    assert rel_maxabs(out, ref) <= TOL


@pytest.mark.parametrize("model,T", [("deepseek", 1), ("deepseek", 2048), ("qwen", 1), ("qwen", 8),
                                     ("qwen", 1024)])
def test_config_dense_shared_expert(gpu, model, T):
    """The model shapes with their shared experts kept in dense bf16, as the reference keeps
    them (vllm_lut/moe_layer.py:186-200, 348-353): DeepSeek-V2-Lite's two shared experts
    as one 2816-wide bf16 MLP of weight 1 beside 64 routed BL4 experts top-6; Qwen1.5-MoE's
    5632-wide shared expert with its sigmoid(x . g) gate beside 60 routed experts top-4.
    Decode and prefill sizes, every token checked."""
    import torch
    from block_lut_amd import ops
    from block_lut_amd.formats import MoEWeights
    from test_gpu_parity import _sigmoid_gate, dense_shared_weights
    H, I = 2048, 1408
    E, k, Is = (64, 6, 2816) if model == "deepseek" else (60, 4, 5632)
    g = torch.Generator(device=gpu).manual_seed(77 + T)
    w13 = DevBL4(E, 2 * I, H, g, gpu)
    w2 = DevBL4(E, H, I, g, gpu)
    d13, d2, h13, h2 = dense_shared_weights(gpu, Is, H, 78)
    rng = np.random.default_rng(79 + T)
    gate = O.f32_to_bf16((rng.standard_normal(H) * 0.05).astype(np.float32)) if model == "qwen" else None
    moe = MoEWeights(w13.stack, w2.stack, H, I, E, 0, dense_shared=(d13, d2),
                     shared_gate=None if gate is None else to_dev_bf16(gate, gpu))
    xb = _x(rng, T, H)
    lg = rng.standard_normal((T, E)).astype(np.float32)
    out = ops.moe_forward_logits(moe, to_dev_bf16(xb, gpu), torch.from_numpy(lg).to(gpu), k,
                                 out_dtype=torch.float32).cpu().numpy()
    assert np.isfinite(out).all()
    rw, rids = O.route(lg, k)
    sw = None if gate is None else _sigmoid_gate(xb, gate)
    ref = O.moe_layer(xb, rids, rw, w13.host, w2.host, shared=[(h13, h2)], shared_w=sw,
                      blas_dtype=np.float32)
    assert rel_maxabs(out, ref) <= TOL
