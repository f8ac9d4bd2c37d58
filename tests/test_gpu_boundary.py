"""The drop-in Python boundary on the GPU: the entry points a caller of the
reference's vLLM plugin uses, each checked against the oracle.

  LUTConfig -> get_quant_method -> create_weights -> process_weights_after_loading
      (reading blocklut_256.npy and lut_absmax.npz written with the reference's
      names and keys, vllm_lut/quant_method.py:169-224) -> apply at T = 1 / 5 / 40
  LUTMoELayer.forward in both router modes, and the router kernel itself
  LUTMoEExpertWrapper.forward / get_weight
  lut_gemv.lut_gemv and torch.ops.lutmoe.lut_gemv
  fused_kernel.fused_lut_gemv
  decompress.decompress_blocklut, LutDecompressor, torch.ops.lutmoe.blocklut_decompress
"""
import numpy as np
import pytest

import oracle as O
from lutmoe_testutil import (BL4Expertset, RefExpertset, bf16_bits, golden_codebook, rel_excess_bf16,
                             rel_maxabs, to_dev_bf16)

pytestmark = pytest.mark.gpu
TOL = 1e-3


def _x(rng, T, K):
    return O.f32_to_bf16(rng.standard_normal((T, K)).astype(np.float32))


def test_quant_method_ref_dropin(gpu, tmp_path):
    import torch
    from block_lut_amd.quant_method import LUTConfig, LUTFusedMoEMethod
    E, H, I, k, L = 6, 512, 256, 2, 3
    w13 = RefExpertset(E, 2 * I, H, seed=501)
    w2 = RefExpertset(E, H, I, seed=502)
    cb = golden_codebook()
    np.save(tmp_path / "blocklut_256.npy", O.bf16_to_f32(cb))
    keys = {}
    half = w13.absmax.shape[1] // 2
    for e in range(E):
        a13 = O.bf16_to_f32(w13.absmax[e])
        keys[f"model.layers.{L}.mlp.experts.{e}.gate_proj.weight"] = a13[:half]
        keys[f"model.layers.{L}.mlp.experts.{e}.up_proj.weight"] = a13[half:]
        keys[f"model.layers.{L}.mlp.experts.{e}.down_proj.weight"] = O.bf16_to_f32(w2.absmax[e])
    keys[f"model.layers.{L}.mlp.shared_expert.gate_proj.weight"] = np.zeros(4, np.float32)  # skipped
    np.savez(tmp_path / "lut_absmax.npz", **keys)

    layer = torch.nn.Module()
    layer.is_routed_experts = True
    cfg = LUTConfig.from_config({"quant_method": "lut", "code_type": "BLOCKLUT",
                                 "lut_path": str(tmp_path), "block_size": 128})
    assert cfg.get_name() == "lut"
    method = cfg.get_quant_method(layer)
    assert isinstance(method, LUTFusedMoEMethod)
    method.create_weights(layer, E, H, I, torch.bfloat16, device=gpu)
    assert tuple(layer.w13_weight.shape) == (E, 2 * I, H) and layer.w13_weight.dtype == torch.uint8
    assert tuple(layer.w2_absmax.shape) == (E, H * I // 128)
    layer.w13_weight.data.copy_(torch.from_numpy(w13.codes))
    layer.w2_weight.data.copy_(torch.from_numpy(w2.codes))
    method.process_weights_after_loading(layer)
    assert np.array_equal(bf16_bits(layer._codebook), cb)
    assert np.array_equal(bf16_bits(layer.w13_absmax), w13.absmax)
    assert np.array_equal(bf16_bits(layer.w2_absmax), w2.absmax)
    rng = np.random.default_rng(50)
    for T in (1, 5, 40):
        xb = _x(rng, T, H)
        rw, rids = O.route(rng.standard_normal((T, E)).astype(np.float32), k)
        out = method.apply(layer, to_dev_bf16(xb, gpu), torch.from_numpy(rw).to(gpu).to(torch.bfloat16),
                           torch.from_numpy(rids.astype(np.int64)).to(gpu))
        assert out.dtype == torch.bfloat16 and tuple(out.shape) == (T, H)
        # the weights reach the layer as bf16, as the router hands them over
        rwb = O.bf16_to_f32(O.f32_to_bf16(rw))
        # one token: lut_gemv's products (quant_method.py:250-260); more: dequantised weights
        f13, f2 = (w13.gemv_f32, w2.gemv_f32) if T == 1 else (w13.deq_f32, w2.deq_f32)
        ref = O.moe_layer(xb, rids, rwb, f13, f2)
        assert rel_excess_bf16(O.bf16_to_f32(bf16_bits(out)), ref) <= TOL, T


def test_quant_method_bl4_dropin(gpu):
    import torch
    from block_lut_amd.quant_method import LUTConfig
    E, H, I, k = 5, 512, 192, 2
    w13 = BL4Expertset(E, 2 * I, H, seed=511, n_iter=8)
    w2 = BL4Expertset(E, H, I, seed=512, n_iter=8)
    layer = torch.nn.Module()
    layer.is_routed_experts = True
    cfg = LUTConfig(code_type="BLOCKLUT", code_bits=4, codebook_scope="block")
    method = cfg.get_quant_method(layer)
    method.create_weights(layer, E, H, I, torch.bfloat16, device=gpu)
    layer.w13_weight.data.copy_(torch.from_numpy(w13.codes))
    layer.w2_weight.data.copy_(torch.from_numpy(w2.codes))
    layer.w13_codebooks.data.copy_(torch.from_numpy(w13.tables.view(np.float16)))
    layer.w2_codebooks.data.copy_(torch.from_numpy(w2.tables.view(np.float16)))
    method.process_weights_after_loading(layer)
    rng = np.random.default_rng(51)
    for T in (1, 7, 64):
        xb = _x(rng, T, H)
        rw, rids = O.route(rng.standard_normal((T, E)).astype(np.float32), k)
        out = method.apply(layer, to_dev_bf16(xb, gpu), torch.from_numpy(rw).to(gpu),
                           torch.from_numpy(rids).to(gpu))
        ref = O.moe_layer(xb, rids, rw, w13.deq_f32, w2.deq_f32)
        assert rel_excess_bf16(O.bf16_to_f32(bf16_bits(out)), ref) <= TOL, T


@pytest.mark.parametrize("T,round_bf16", [(1, False), (1, True), (7, False), (33, True)])
def test_router_logits_kernel(gpu, T, round_bf16):
    """x . gate^T with fp32 accumulation (MoEGate) or rounded to bf16 (the vLLM layer's
    bf16 gate linear): against float64 sums, and bf16 values within one bf16 step of
    the float64 sum rounded."""
    import torch
    from block_lut_amd import ops
    H, E = 2048, 60
    rng = np.random.default_rng(T + 7 * round_bf16)
    xb = _x(rng, T, H)
    gb = O.f32_to_bf16((rng.standard_normal((E, H)) * 0.02).astype(np.float32))
    got = ops.router_logits(to_dev_bf16(xb, gpu), to_dev_bf16(gb, gpu), round_bf16=round_bf16).cpu().numpy()
    ref = O.bf16_to_f32(xb).astype(np.float64) @ O.bf16_to_f32(gb).astype(np.float64).T
    if round_bf16:
        assert np.array_equal(got, O.bf16_to_f32(O.f32_to_bf16(got)))   # bf16 values
        rb = O.bf16_to_f32(O.f32_to_bf16(ref.astype(np.float32))).astype(np.float64)
        ulp = np.abs(rb) * 2.0 ** -7 + 1e-30
        assert np.all(np.abs(got - rb) <= ulp)
        assert np.mean(got == rb) > 0.99
    else:
        assert np.abs(got - ref).max() <= 1e-5 * np.abs(ref).max()


@pytest.mark.parametrize("router_dtype,T", [("bf16", 1), ("bf16", 6), ("bf16", 100), ("f32", 1), ("f32", 6),
                                            ("f32", 100)])
def test_lut_moe_layer_forward(gpu, router_dtype, T):
    """LUTMoELayer.forward: router (gate kernel up to 64 tokens, torch's GEMM above), top-k,
    fused layer, against the oracle routing the float64 logits.  bf16 mode: the reference's
    vLLM layer (bf16 logits, top-k weights cast to bf16); f32 mode: DeepSeek's MoEGate."""
    import torch
    from block_lut_amd.formats import MoEWeights
    from block_lut_amd.moe_layer import LUTMoELayer
    E, S, k, H, I = 8, 1, 2, 512, 256
    w13 = BL4Expertset(E + S, 2 * I, H, seed=521 + T, n_iter=8)
    w2 = BL4Expertset(E + S, H, I, seed=522 + T, n_iter=8)
    moe = MoEWeights(w13.stack(gpu), w2.stack(gpu), H, I, E, S)
    rng = np.random.default_rng(520 + T)
    gb = O.f32_to_bf16((rng.standard_normal((E, H)) * 0.05).astype(np.float32))
    dt = torch.bfloat16 if router_dtype == "bf16" else torch.float32
    layer = LUTMoELayer(moe, to_dev_bf16(gb, gpu), k, router_dtype=dt)
    xb = _x(rng, T, H)
    out = layer(to_dev_bf16(xb, gpu))
    assert out.dtype == torch.bfloat16 and tuple(out.shape) == (T, H)
    lg = O.bf16_to_f32(xb).astype(np.float64) @ O.bf16_to_f32(gb).astype(np.float64).T
    if router_dtype == "bf16":
        lg = O.bf16_to_f32(O.f32_to_bf16(lg.astype(np.float32)))
    # tokens whose k-th and (k+1)-th logits are a few roundings apart route the same way
    # whatever the summation order (bf16 mode: 4 bf16 steps; f32 mode: 1e-4)
    srt = np.sort(lg, axis=1)[:, ::-1]
    gap = srt[:, k - 1] - srt[:, k]
    clear = gap > (4 * 2.0 ** -7 * np.abs(srt[:, k - 1]) + 1e-6 if router_dtype == "bf16" else 1e-4)
    assert clear.mean() >= 0.75
    rw, rids = O.route(lg.astype(np.float32), k)
    if router_dtype == "bf16":
        rw = O.bf16_to_f32(O.f32_to_bf16(rw))
    ref = O.moe_layer(xb, rids, rw, w13.deq_f32, w2.deq_f32,
                      shared=[(w13.deq_f32(E + s), w2.deq_f32(E + s)) for s in range(S)])
    got = O.bf16_to_f32(bf16_bits(out))
    assert rel_excess_bf16(got[clear], ref[clear]) <= TOL


def test_expert_wrapper(gpu):
    """LUTMoEExpertWrapper: get_weight dequantises one expert bit-exactly, forward runs the
    fused GEMV for a few tokens and the dequantised matmul above."""
    import torch
    from block_lut_amd.moe_layer import LUTMoEExpertWrapper
    E, H, I = 3, 512, 256
    w13 = BL4Expertset(E, 2 * I, H, seed=531, n_iter=8)
    w2 = BL4Expertset(E, H, I, seed=532, n_iter=8)
    ex = LUTMoEExpertWrapper(w13.stack(gpu), w2.stack(gpu), 2)
    assert np.array_equal(bf16_bits(ex.get_weight("w13")), O.bl4_dequant(w13.codes[2], w13.tables[2]))
    rng = np.random.default_rng(53)
    for T in (1, 3, 20):
        xb = _x(rng, T, H)
        y = ex(to_dev_bf16(xb, gpu), "w13")
        ref = O.bf16_to_f32(xb).astype(np.float64) @ w13.deq_f32(2).astype(np.float64).T
        # forward returns bf16 (one rounding); the matmul path also sums in bf16 GEMM order
        assert rel_excess_bf16(O.bf16_to_f32(bf16_bits(y)), ref) <= TOL, T


@pytest.mark.parametrize("M,K,T", [(2816, 2048, 1), (300, 640, 1), (300, 640, 3)])
def test_lut_gemv_wrappers(gpu, M, K, T):
    """lut_gemv.lut_gemv (cuda_lut_gemv.py:153-169) and torch.ops.lutmoe.lut_gemv: bf16 out,
    the reference's (x * cb) * absmax products."""
    import torch
    from block_lut_amd.lut_gemv import lut_gemv
    rng = np.random.default_rng(M + K + T)
    cb = golden_codebook()
    idx = rng.integers(0, 256, (M, K), dtype=np.uint8)
    nb = -(-M * K // 128)
    am = O.f32_to_bf16(np.abs(rng.standard_normal(nb)).astype(np.float32) * 0.02)
    xb = _x(rng, T, K)
    args = (to_dev_bf16(xb[0] if T == 1 else xb, gpu), torch.from_numpy(idx).to(gpu), to_dev_bf16(cb, gpu),
            to_dev_bf16(am, gpu))
    y = lut_gemv(*args)
    assert y.dtype == torch.bfloat16 and tuple(y.shape) == ((M,) if T == 1 else (T, M))
    assert torch.equal(torch.ops.lutmoe.lut_gemv(*args), y)
    got = O.bf16_to_f32(bf16_bits(y)).reshape(T, M)
    for t in range(T):
        assert rel_excess_bf16(got[t], O.ref_gemv(xb[t], idx, cb, am)) <= TOL


@pytest.mark.parametrize("M,K,T,bs", [(2816, 2048, 1, 128), (2048, 1408, 2, 128), (37, 203, 1, 100)])
def test_fused_lut_gemv(gpu, M, K, T, bs):
    """fused_kernel.fused_lut_gemv (vllm_lut/fused_kernel.py:13-46): the dequantised bf16
    weights bf16(cb * absmax) times the input; much closer to that oracle than to
    lut_gemv's unrounded products (the two differ by the weights' bf16 rounding)."""
    import torch
    from block_lut_amd.fused_kernel import fused_lut_gemv
    from block_lut_amd import ops
    rng = np.random.default_rng(M + T + bs)
    cb = golden_codebook()
    idx = rng.integers(0, 256, (M, K), dtype=np.uint8)
    nb = -(-M * K // bs)
    am = O.f32_to_bf16(np.abs(rng.standard_normal(nb)).astype(np.float32) * 0.02 + 0.01)
    xb = _x(rng, T, K)
    args = (torch.from_numpy(idx).to(gpu), to_dev_bf16(cb, gpu), to_dev_bf16(am, gpu))
    y = fused_lut_gemv(to_dev_bf16(xb[0] if T == 1 else xb, gpu), *args, block_size=bs)
    assert y.dtype == torch.bfloat16 and tuple(y.shape) == ((M,) if T == 1 else (T, M))
    deq = O.bf16_to_f32(O.ref_dequant(idx.reshape(-1), am, cb, bs)).reshape(M, K).astype(np.float64)
    blk = np.minimum(np.arange(M * K) // bs, nb - 1)
    raw = (O.bf16_to_f32(cb)[idx.reshape(-1)].astype(np.float64) * O.bf16_to_f32(am)[blk]).reshape(M, K)
    xf = O.bf16_to_f32(xb).astype(np.float64)
    got = O.bf16_to_f32(bf16_bits(y)).reshape(T, M)
    assert rel_excess_bf16(got, xf @ deq.T) <= TOL
    # fp32 output separates the two weight rules clearly
    y32 = ops.ref_gemv(to_dev_bf16(xb, gpu), *args, block_size=bs, out_dtype=torch.float32,
                       dequantised=True).cpu().numpy()
    e_own, e_other = rel_maxabs(y32, xf @ deq.T), rel_maxabs(y32, xf @ raw.T)
    assert e_own <= 1e-5 and e_own < 0.1 * e_other, (e_own, e_other)


def test_decompress_wrappers(gpu):
    """decompress_blocklut (quantizer.py:449-477, including the clamped last block),
    LutDecompressor.decompress (build_lut_kernel.py:88-139) and
    torch.ops.lutmoe.blocklut_decompress: bit-exact against the oracle."""
    import torch
    from block_lut_amd.decompress import LutDecompressor, decompress_blocklut
    rng = np.random.default_rng(61)
    cb = golden_codebook()
    n = 128 * 50 + 37
    idx = rng.integers(0, 256, n, dtype=np.uint8)
    am = O.f32_to_bf16(np.abs(rng.standard_normal(-(-n // 128))).astype(np.float32))
    di, da, dc = torch.from_numpy(idx).to(gpu), to_dev_bf16(am, gpu), to_dev_bf16(cb, gpu)
    ref = O.ref_dequant(idx, am, cb, 128)
    assert np.array_equal(bf16_bits(decompress_blocklut(di, da, dc, 128)), ref)
    assert np.array_equal(bf16_bits(LutDecompressor().decompress(di, da, dc, 128)), ref)
    assert np.array_equal(bf16_bits(torch.ops.lutmoe.blocklut_decompress(di, da, dc, 128)), ref)
    # fewer absmax entries than blocks: the block index clamps to the last entry
    short = am[:10]
    assert np.array_equal(bf16_bits(decompress_blocklut(di, to_dev_bf16(short, gpu), dc, 128)),
                          O.ref_dequant(idx, short, cb, 128))


@pytest.mark.parametrize("router_dtype,T", [("bf16", 1), ("f32", 6), ("bf16", 80)])
def test_lut_moe_layer_dense_shared_expert(gpu, router_dtype, T):
    """LUTMoELayer over LUT routed experts and a shared expert kept in dense bf16 with
    Qwen's sigmoid gate (the layout of the reference's Qwen2MoE block: bf16 shared MLP and
    gate beside the LUT experts, customized/qwen.py:40-43, 96-100), bf16 output against the
    oracle within one bf16 ulp of its rounding plus the bar."""
    import torch
    from block_lut_amd.formats import MoEWeights
    from block_lut_amd.moe_layer import LUTMoELayer
    from test_gpu_parity import _sigmoid_gate, dense_shared_weights
    E, k, H, I, Is = 8, 2, 512, 256, 512
    w13 = BL4Expertset(E, 2 * I, H, seed=541 + T, n_iter=8)
    w2 = BL4Expertset(E, H, I, seed=542 + T, n_iter=8)
    d13, d2, h13, h2 = dense_shared_weights(gpu, Is, H, 543 + T)
    rng = np.random.default_rng(540 + T)
    gate = O.f32_to_bf16((rng.standard_normal(H) * 0.05).astype(np.float32))
    moe = MoEWeights(w13.stack(gpu), w2.stack(gpu), H, I, E, 0, dense_shared=(d13, d2),
                     shared_gate=to_dev_bf16(gate, gpu))
    gb = O.f32_to_bf16((rng.standard_normal((E, H)) * 0.05).astype(np.float32))
    dt = torch.bfloat16 if router_dtype == "bf16" else torch.float32
    layer = LUTMoELayer(moe, to_dev_bf16(gb, gpu), k, router_dtype=dt)
    xb = _x(rng, T, H)
    out = layer(to_dev_bf16(xb, gpu))
    lg = O.bf16_to_f32(xb).astype(np.float64) @ O.bf16_to_f32(gb).astype(np.float64).T
    if router_dtype == "bf16":
        lg = O.bf16_to_f32(O.f32_to_bf16(lg.astype(np.float32)))
    srt = np.sort(lg, axis=1)[:, ::-1]
    gap = srt[:, k - 1] - srt[:, k]
    clear = gap > (4 * 2.0 ** -7 * np.abs(srt[:, k - 1]) + 1e-6 if router_dtype == "bf16" else 1e-4)
    rw, rids = O.route(lg.astype(np.float32), k)
    if router_dtype == "bf16":
        rw = O.bf16_to_f32(O.f32_to_bf16(rw))
    ref = O.moe_layer(xb, rids, rw, w13.deq_f32, w2.deq_f32, shared=[(h13, h2)], shared_w=_sigmoid_gate(xb, gate))
    got = O.bf16_to_f32(bf16_bits(out))
    assert clear.any()
    assert rel_excess_bf16(got[clear], ref[clear]) <= TOL
