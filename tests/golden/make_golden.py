"""Writes the golden fixtures under tests/golden/ (run where the reference
checkout exists at /root/reference; the tests only read the fixtures).

codebooks.npz   derived data from the reference's shipped codebook files
                (models/{qwen,deepseek}/*.npy), loaded with numpy
                allow_pickle=False:
                  qwen_blocklut_256_bf16   bf16 bits of blocklut_256 as
                                           LUTQuantizer.load casts it
                                           (vllm_lut/quantizer.py:372-378)
                  qwen_blocklut_256_f32, qwen_blocklut_16_f32,
                  {qwen,deepseek}_nested_lut_{16,64}_f32,
                  {qwen,deepseek}_nested_map_256to{16,64}_u8,
                  {qwen,deepseek}_nested_lut_mapped{16,64}_u16  (as shipped)
quantizer.npz   input/output vectors of the reference's LUTQuantizer
                (vllm_lut/quantizer.py), imported by file path in this
                container for the functions nothing else pins:
                  quantize()  fp32 and bf16 inputs (tie rule, bf16 division),
                              padded length;
                  _train_kmeans() for fixed torch seeds (randperm stream);
                  _greedy_merge().
"""
from __future__ import annotations

import importlib.util
import os
import sys

import numpy as np

REF = "/root/reference"
HERE = os.path.dirname(os.path.abspath(__file__))


def f32_to_bf16_bits(x):
    import torch
    return torch.from_numpy(np.asarray(x, np.float32)).to(torch.bfloat16).view(torch.int16) \
        .numpy().view(np.uint16)


def codebooks():
    out = {}
    q = os.path.join(REF, "models", "qwen")
    d = os.path.join(REF, "models", "deepseek")
    lut = np.load(os.path.join(q, "blocklut_256.npy"), allow_pickle=False).astype(np.float32)
    out["qwen_blocklut_256_f32"] = lut
    out["qwen_blocklut_256_bf16"] = f32_to_bf16_bits(lut)
    out["qwen_blocklut_16_f32"] = np.load(os.path.join(q, "blocklut_16.npy"),
                                          allow_pickle=False).astype(np.float32)
    for tag, base in (("qwen", q), ("deepseek", d)):
        for k in (16, 64):
            out[f"{tag}_nested_lut_{k}_f32"] = np.load(
                os.path.join(base, f"nested_lut_{k}.npy"), allow_pickle=False).astype(np.float32)
            out[f"{tag}_nested_map_256to{k}_u8"] = np.load(
                os.path.join(base, f"nested_map_256to{k}.npy"), allow_pickle=False).astype(np.uint8)
            out[f"{tag}_nested_lut_mapped{k}_u16"] = np.load(
                os.path.join(base, f"nested_lut_mapped{k}.npy"), allow_pickle=False).astype(np.uint16)
        out[f"{tag}_blocklut_256_f32"] = np.load(os.path.join(base, "blocklut_256.npy"),
                                                 allow_pickle=False).astype(np.float32)
    np.savez_compressed(os.path.join(HERE, "codebooks.npz"), **out)


def km_big_data():
    """230,000 samples (more than _train_kmeans' 200,000 max_samples), regenerated
    from this seed by the tests instead of being stored."""
    return (np.random.default_rng(123).standard_normal(230000) * 0.3).astype(np.float32)


def quantizer_vectors():
    import torch
    spec = importlib.util.spec_from_file_location(
        "reference_quantizer", os.path.join(REF, "vllm_lut", "quantizer.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    out = {}
    cb = torch.from_numpy(np.load(os.path.join(REF, "models", "qwen", "blocklut_256.npy"),
                                  allow_pickle=False)).to(torch.bfloat16)
    qz = mod.LUTQuantizer(code_type="BLOCKLUT", block_size=128, device="cpu")
    rng = np.random.default_rng(7)
    # fp32 input, whole blocks
    w = (rng.standard_normal((48, 256)) * 0.02).astype(np.float32)
    r = qz.quantize(torch.from_numpy(w), cb)
    out["q_f32_w"] = w
    out["q_f32_idx"] = r["indices"].numpy()
    out["q_f32_absmax"] = r["absmax"].view(torch.int16).numpy().view(np.uint16)
    # fp32 input, padded tail (N % 128 != 0), with exact zeros and ties
    w2 = (rng.standard_normal(1000) * 0.05).astype(np.float32)
    w2[:17] = 0.0
    w2[200:328] = 0.0                      # an all-zero block (absmax clamp)
    r = qz.quantize(torch.from_numpy(w2), cb)
    out["q_pad_w"] = w2
    out["q_pad_idx"] = r["indices"].numpy()
    out["q_pad_absmax"] = r["absmax"].view(torch.int16).numpy().view(np.uint16)
    # bf16 input (normalisation divides in bf16)
    w3 = torch.from_numpy((rng.standard_normal((32, 384)) * 0.02).astype(np.float32)).to(torch.bfloat16)
    r = qz.quantize(w3, cb)
    out["q_bf16_w"] = w3.view(torch.int16).numpy().view(np.uint16)
    out["q_bf16_idx"] = r["indices"].numpy()
    out["q_bf16_absmax"] = r["absmax"].view(torch.int16).numpy().view(np.uint16)
    # _train_kmeans on CPU with fixed seeds
    data = (rng.standard_normal(5000)).astype(np.float32)
    for seed, k, it in ((0, 16, 5), (3, 64, 8)):
        torch.manual_seed(seed)
        c = qz._train_kmeans(torch.from_numpy(data), k, it)
        out[f"km_s{seed}_k{k}_it{it}"] = c.view(torch.int16).numpy().view(np.uint16)
    out["km_data"] = data
    big = km_big_data()                    # > max_samples: subset path
    torch.manual_seed(11)
    c = qz._train_kmeans(torch.from_numpy(big), 16, 3)
    out["km_big_s11_k16_it3"] = c.view(torch.int16).numpy().view(np.uint16)
    # _greedy_merge 64 -> 16 on float32 centroids
    c64 = np.sort(rng.standard_normal(64).astype(np.float32))
    out["gm_in"] = c64
    out["gm_out"] = qz._greedy_merge(torch.from_numpy(c64), 16).numpy()
    np.savez_compressed(os.path.join(HERE, "quantizer.npz"), **out)


if __name__ == "__main__":
    codebooks()
    quantizer_vectors()
    print("wrote", os.listdir(HERE))
    sys.exit(0)
