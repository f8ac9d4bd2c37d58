"""Host-side interface mirror (no GPU): config surface, argument checks that
fire before any device work, and the no-fallback guarantees."""
import ast
import os
import subprocess
import sys

import numpy as np
import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_lut_config_surface():
    from block_lut_amd.quant_method import LUTConfig, LUTFusedMoEMethod
    assert LUTConfig.get_name() == "lut"
    assert torch.bfloat16 in LUTConfig.get_supported_act_dtypes()
    assert LUTConfig.get_config_filenames() == []
    c = LUTConfig.from_config({"quant_method": "lut", "code_type": "NESTEDLUT",
                               "lut_path": "/nonexistent"})
    assert c.code_type == "NESTEDLUT" and c.lut_path == "/nonexistent" and c.format == "ref"
    c4 = LUTConfig(code_bits=4, codebook_scope="block")
    assert c4.format == "bl4"
    with pytest.raises(ValueError):
        LUTConfig(code_type="GPTQ")
    with pytest.raises(ValueError):
        LUTConfig(code_bits=4, codebook_scope="global")

    class Experts(torch.nn.Module):
        is_routed_experts = True

    class Other(torch.nn.Module):
        pass

    assert isinstance(c.get_quant_method(Experts(), "x"), LUTFusedMoEMethod)
    assert c.get_quant_method(Other(), "x") is None


def test_vllm_config_validation():
    from block_lut_amd.config import LUT_MoE_vLLMConfig
    LUT_MoE_vLLMConfig(code_type="NESTEDLUT", lut_tier=2)
    with pytest.raises(ValueError):
        LUT_MoE_vLLMConfig(code_type="X")
    with pytest.raises(ValueError):
        LUT_MoE_vLLMConfig(lut_tier=3)


def test_create_weights_shapes_cpu_device():
    """create_weights registers the reference's parameter set (quant_method.py:117-163)."""
    from block_lut_amd.quant_method import LUTConfig, LUTFusedMoEMethod
    layer = torch.nn.Module()
    m = LUTFusedMoEMethod(LUTConfig())
    m.create_weights(layer, 4, 256, 128, torch.bfloat16, device="cpu", weight_loader=None)
    assert layer.w13_weight.shape == (4, 256, 256) and layer.w13_weight.dtype == torch.uint8
    assert layer.w2_weight.shape == (4, 256, 128)
    assert layer.w13_absmax.shape == (4, 256 * 256 // 128)
    assert layer._codebook.shape == (256,) and layer._codebook.dtype == torch.bfloat16
    layer4 = torch.nn.Module()
    m4 = LUTFusedMoEMethod(LUTConfig(code_bits=4, codebook_scope="block"))
    m4.create_weights(layer4, 4, 256, 128, torch.bfloat16, device="cpu")
    assert layer4.w13_weight.shape == (4, 256, 128)
    assert layer4.w13_codebooks.shape == (4, 256, 4, 16)
    assert layer4.w2_codebooks.dtype == torch.float16


def test_stacks_reject_host_tensors():
    from block_lut_amd.formats import BL4Stack, RefStack
    with pytest.raises(ValueError):
        BL4Stack(torch.zeros(1, 8, 32, dtype=torch.uint8),
                 torch.zeros(1, 8, 1, 16, dtype=torch.bfloat16))
    with pytest.raises(ValueError):
        RefStack(torch.zeros(1, 8, 64, dtype=torch.uint8), torch.zeros(1, 4, dtype=torch.bfloat16),
                 torch.zeros(256, dtype=torch.bfloat16))


def test_decompress_has_no_cpu_path():
    from block_lut_amd.decompress import decompress_blocklut
    with pytest.raises(ValueError):
        decompress_blocklut(torch.zeros(128, dtype=torch.uint8), torch.ones(1, dtype=torch.bfloat16),
                            torch.zeros(256, dtype=torch.bfloat16))


def test_missing_library_fails_loudly(monkeypatch):
    from block_lut_amd import _native as N
    monkeypatch.setattr(N, "LIB_PATH", "/nonexistent/liblutmoe.so")
    monkeypatch.setattr(N, "_lib", None)
    with pytest.raises(N.LutMoeNotBuilt):
        N.lib()


def test_product_never_imports_the_oracle():
    pkg = os.path.join(ROOT, "block_lut_amd")
    for dirpath, _, files in os.walk(pkg):
        for f in files:
            if not f.endswith(".py"):
                continue
            tree = ast.parse(open(os.path.join(dirpath, f)).read())
            for node in ast.walk(tree):
                if isinstance(node, ast.Import):
                    assert all(not a.name.startswith("oracle") for a in node.names), f
                elif isinstance(node, ast.ImportFrom):
                    assert not (node.module or "").startswith("oracle"), f


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True)
    assert r.returncode == 2 and "one GPU" in r.stderr


def test_gguf_reader_roundtrip_and_expert_names(tmp_path):
    """read_gguf parses what a GGUF v3 writer produces (typed metadata, arrays, tensor
    infos, 32-byte aligned data) and sizes an unknown-type tensor by the next offset."""
    from block_lut_amd import checkpoint as C
    from lutmoe_testutil import GGUF_BLOCKLUT8_TEST_ID, write_gguf
    rng = np.random.default_rng(0)
    a = rng.integers(0, 256, 1000, dtype=np.uint8)
    b = rng.integers(0, 256, 333, dtype=np.uint8)
    lut = rng.integers(0, 65536, 256, dtype=np.uint16)
    p = str(tmp_path / "t.gguf")
    write_gguf(p, [("lut-moe.enabled", True), ("lut-moe.block_size", 128), ("general.name", "x"),
                   ("lut-moe.lut_table", lut.tolist()), ("hparams.eps", 1e-6)],
               [("model.layers.0.mlp.experts.0.gate_proj.weight", (1000,), GGUF_BLOCKLUT8_TEST_ID, a.tobytes()),
                ("model.norm.weight", (333,), 0, b.tobytes())])
    g = C.read_gguf(p)
    assert g.kv["lut-moe.enabled"] is True and g.kv["lut-moe.block_size"] == 128
    assert g.kv["general.name"] == "x" and np.array_equal(g.kv["lut-moe.lut_table"], lut)
    dims, tid, raw = g.tensors["model.layers.0.mlp.experts.0.gate_proj.weight"]
    assert dims == (1000,) and tid == GGUF_BLOCKLUT8_TEST_ID
    assert np.array_equal(raw[:1000], a)
    assert np.array_equal(g.tensors["model.norm.weight"][2][:333], b)
    assert C.is_expert_tensor("model.layers.3.mlp.experts.7.down_proj.weight")
    assert C.is_expert_tensor("blk.3.ffn_up_exps.weight")
    assert not C.is_expert_tensor("model.layers.3.mlp.shared_expert.down_proj.weight")
    assert not C.is_expert_tensor("model.layers.3.mlp.gate.weight")


def test_fused_lut_moe_op_fake_shapes():
    """lutmoe::fused_lut_moe is a torch.library op whose fake kernel gives the layer's
    output shape and dtype (what torch.compile traces), without a GPU."""
    import torch
    from torch._subclasses.fake_tensor import FakeTensorMode
    import block_lut_amd.fast_moe  # noqa: F401  (registers the op)
    E, H, I, T, k = 4, 256, 128, 5, 2
    with FakeTensorMode():
        x = torch.empty(T, H, dtype=torch.bfloat16)
        ids = torch.empty(T, k, dtype=torch.int32)
        w = torch.empty(T, k, dtype=torch.float32)
        w13 = torch.empty(E, 2 * I, H, dtype=torch.uint8)
        w2 = torch.empty(E, H, I, dtype=torch.uint8)
        a13 = torch.empty(E, 2 * I * H // 128, dtype=torch.bfloat16)
        a2 = torch.empty(E, H * I // 128, dtype=torch.bfloat16)
        cb = torch.empty(256, dtype=torch.bfloat16)
        out = torch.ops.lutmoe.fused_lut_moe(x, ids, w, w13, a13, w2, a2, cb)
        assert tuple(out.shape) == (T, H) and out.dtype == torch.bfloat16
        out1 = torch.ops.lutmoe.fused_lut_moe(x[0], ids[:1], w[:1], w13, a13, w2, a2, cb)
        assert tuple(out1.shape) == (1, H)
