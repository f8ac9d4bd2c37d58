#!/usr/bin/env python3
"""Benchmark of the LUT-MoE hot path on one MI355X.

Default workload (one step = one MoE layer decode step):
  Qwen1.5-MoE-A2.7B-shaped layer, hidden 2048, moe_intermediate 1408, 60
  routed experts, top-4 softmax routing of N(0,1) logits, SwiGLU gate/up/down
  all BL4 4-bit (64-weight blocks, 16-entry codebooks), T = 1 token of bf16
  N(0,1) activations.  Each step is one call of the MoE block forward from
  router logits: two kernels, the first computing the softmax/top-k routing
  and the token permutation in every CTA (its first CTA stores them for the
  second) and running the grouped LUT-GEMV gate/up + SwiGLU, the second the
  down projection + weighted combine.  Steps rotate over 16 distinct layer weight copies (8.3 GB,
  each step with its own routing) so the touched bytes per rotation exceed
  the 256 MB Infinity Cache: the figure is cold-HBM, not MALL.

value      = algorithmic HBM bytes of the timed steps / timed seconds (TB/s);
             algorithmic bytes per step = sum over the step's distinct routed
             experts of 8,650,752 B (codes 0.5 B/weight + bf16 tables
             32 B per 64 weights) + 2*T*H*2 B of activations.
roofline   = the gate/up + SwiGLU kernel (the dominant kernel) timed alone with
             HIP events over a captured graph of its launches.
cpu_baseline = the reference's CPU dequant + matmul path restated with torch
             on the host (oracle/cpu_baseline.py), on a bounded sample of the
             same steps.
extra      = the other configurations (decode T=8/32, DeepSeek-V2-Lite prefill
             grouped GEMM TFLOP/s, switch-base-8 single linear, hot-cache decode,
             and the NestedLUT tier workload: Qwen shape, 20 experts each at 2, 3
             and 4 bits, Zipf(1.1) expert popularity with Gumbel-top-4 routing,
             decode T=16 and prefill T=1024; the Mixtral-8x7B-shaped stack of
             32 resident layers: decode B=1/64 and prefill 4096 tokens).

Weights are synthetic BL4 data of the configured shapes (uniform random 4-bit
codes, sorted N(0, 0.02) codebook entries): throughput does not depend on the
values.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "LUT-MoE layer µs/token + achieved HBM TB/s (bs=1); prefill grouped-GEMM TFLOP/s"
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
QWEN = dict(H=2048, I=1408, E=60, k=4, S=0)
DSV2 = dict(H=2048, I=1408, E=64, k=6, S=2)
BYTES_PER_WEIGHT = 1.0   # BL4: 0.5 B codes + 32 B table per 64 weights


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def measured_traffic(name):
    """HBM bytes per launch of the dominant kernel from a committed counter summary
    (FETCH_SIZE and WRITE_SIZE passes, each scaled by what it reads for a copy of known
    size), with the summary's name and the commit it records; (None, None) when the
    summary is absent."""
    path = os.path.join(ROOT, "profiles", name)
    traffic, commit = None, None
    try:
        for line in open(path):
            if line.startswith("traffic_bytes_per_launch:"):
                traffic = int(float(line.split(":", 1)[1]))
            if line.startswith("measured_at_commit:"):
                commit = line.split(":", 1)[1].strip()
    except OSError:
        return None, None
    return traffic, f"profiles/{name} (measured at commit {commit})" if traffic is not None else None


def decode_kernel_label(T, P, E_tot):
    """The gate/up kernel the library launches for this batch (the tokens-per-pass rule of
    decode.hip's tb_for for BL4: one token its own kernel, two-token passes up to 16
    tokens, and up to 32 while the experts hold at most 3 positions on average)."""
    if T <= 1:
        return "bl4_decode_gate_up_t1"
    tb = 2 if T <= 16 or (T <= 32 and P <= 3 * min(P, E_tot)) else 4
    return f"bl4_decode_gate_up<{tb}>"


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=480)
    p.add_argument("--warmup", type=int, default=32)
    p.add_argument("--tokens", type=int, default=1)
    p.add_argument("--layers", type=int, default=16, help="rotating layer weight copies")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    p.add_argument("--no-extra", action="store_true", help="skip the other configurations")
    p.add_argument("--cpu-seconds", type=float, default=12.0)
    p.add_argument("--pmc-sample", action="store_true",
                   help="run only a 256 MiB device copy and the decode gate/up kernel of the "
                        "default workload (for rocprofv3 --pmc passes), then exit")
    p.add_argument("--nested-sample", action="store_true",
                   help="run only the NestedLUT tier workload (decode T=16 and prefill T=1024, "
                        "graph-captured, for rocprofv3 kernel traces), then exit")
    p.add_argument("--prefill-sample", action="store_true",
                   help="run only the DeepSeek-V2-Lite T=2048 prefill (graph-captured, 10 replays, "
                        "for rocprofv3 kernel traces), then exit")
    return p.parse_args()


def main():
    a = parse()
    if a.gpus != 1:
        print(f"bench.py measures one GPU only (every box here has one GPU); --gpus {a.gpus} "
              "is not supported", file=sys.stderr)
        sys.exit(2)
    import torch
    from block_lut_amd import ops
    from block_lut_amd import _native as N
    from block_lut_amd.formats import BL4Stack, MoEWeights, NestedExpert, NestedStack

    dev = torch.device("cuda:0")
    torch.manual_seed(0)
    gen = torch.Generator(device="cpu").manual_seed(1234)

    def rand_stack(E, M, K):
        codes = torch.randint(0, 256, (E, M, K // 2), dtype=torch.uint8, device=dev)
        tabs = torch.randn((E, M, K // 64, 16), device=dev) * 0.02
        tabs = torch.sort(tabs, dim=-1).values.to(torch.bfloat16)
        return BL4Stack(codes, tabs)

    def rand_layer(c):
        E = c["E"] + c["S"]
        return MoEWeights(rand_stack(E, 2 * c["I"], c["H"]), rand_stack(E, c["H"], c["I"]),
                          c["H"], c["I"], c["E"], c["S"])

    def expert_bytes(c):
        return 3 * c["H"] * c["I"] * BYTES_PER_WEIGHT

    class Step:
        """Preallocated inputs/outputs of one layer step (graph-capturable)."""

        def __init__(self, layer, c, T):
            self.layer, self.c, self.T = layer, c, T
            self.logits = torch.randn((T, c["E"]), generator=gen).to(dev)
            self.x = torch.randn((T, c["H"]), generator=gen).to(torch.bfloat16).to(dev)
            self.w = torch.empty((T, c["k"]), dtype=torch.float32, device=dev)
            self.ids = torch.empty((T, c["k"]), dtype=torch.int32, device=dev)
            self.sink = None
            self.out = torch.empty((T, c["H"]), dtype=torch.bfloat16, device=dev)
            self.ws = ops.new_workspace(layer, T, c["k"], dev)
            ops.route_topk(self.logits, c["k"], out_w=self.w, out_ids=self.ids)
            torch.cuda.synchronize()
            ids = self.ids.cpu()
            self.U = int(torch.unique(ids).numel()) + c["S"]
            self.bytes = self.U * expert_bytes(c) + 2 * T * c["H"] * 2
            self.bytes_gate_up = self.U * 2 * c["H"] * c["I"] * BYTES_PER_WEIGHT + T * c["H"] * 2

        def run(self, path=ops.PATH_AUTO, stages=N.STAGE_ALL):
            ops.moe_forward_logits(self.layer, self.x, self.logits, self.c["k"], out=self.out,
                                   workspace=self.ws, path=path, stages=stages)

    def graph_of(fns):
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            for f in fns:
                f()
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for f in fns:
                f()
        torch.cuda.synchronize()
        return g

    def time_graph(g, reps):
        st, en = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        st.record()
        for _ in range(reps):
            g.replay()
        en.record()
        torch.cuda.synchronize()
        return st.elapsed_time(en) / 1e3   # seconds

    # ------------------------------------------------------------ main leg
    c = QWEN
    T = a.tokens
    if a.pmc_sample:
        # calibration: a plain copy of known size (256 MiB read + 256 MiB written)
        src = torch.empty(1 << 28, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
        layers = [rand_layer(c) for _ in range(a.layers)]
        steps = [Step(L, c, T) for L in layers]
        for s in steps:
            s.run(stages=N.STAGE_GATE_UP)
        for s in steps:
            s.run(stages=N.STAGE_GATE_UP)
        torch.cuda.synchronize()
        log(f"[bench] pmc sample: gate/up algorithmic bytes per launch "
            f"{sum(s.bytes_gate_up for s in steps) / len(steps):.0f}")
        return
    if a.nested_sample:
        res = nested_tiers(a, ops, N, torch, dev, NestedExpert, NestedStack, MoEWeights, graph_of, time_graph)
        log(f"[bench] nested sample: {json.dumps(res)}")
        return
    if a.prefill_sample:
        d = DSV2
        sp = Step(rand_layer(d), d, 2048)
        g = graph_of([lambda: sp.run(path=ops.PATH_MFMA)])
        time_graph(g, 2)
        sec = time_graph(g, 10) / 10
        flops = 6 * d["H"] * d["I"] * 2048 * (d["k"] + d["S"])
        log(f"[bench] prefill sample: DeepSeek T=2048 {sec * 1e6:.1f} us, {flops / sec / 1e12:.1f} TFLOP/s "
            f"({flops} flops per layer)")
        return
    log(f"[bench] building {a.layers} Qwen-shaped BL4 layers ({a.layers * c['E'] * expert_bytes(c) / 1e9:.1f} GB)")
    layers = [rand_layer(c) for _ in range(a.layers)]
    steps = [Step(L, c, T) for L in layers]
    R = len(steps)
    g_step = graph_of([s.run for s in steps])
    partial = {}

    def run_steps(n):
        """Exactly n layer steps in rotation order: whole rotations (one graph of all
        layers) and a graph of the first n % R layers."""
        full, rem = divmod(n, R)
        for _ in range(full):
            g_step.replay()
        if rem:
            if rem not in partial:
                partial[rem] = graph_of([s.run for s in steps[:rem]])
            partial[rem].replay()

    K, W = max(1, a.steps), max(0, a.warmup)
    if K % R and K % R not in partial:
        partial[K % R] = graph_of([s.run for s in steps[:K % R]])
    run_steps(W)
    torch.cuda.synchronize()
    log(f"[bench] warmup {W} steps done; timing {K} steps")
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    ev0.record()
    run_steps(K)
    ev1.record()
    torch.cuda.synchronize()
    secs = ev0.elapsed_time(ev1) / 1e3
    full, rem = divmod(K, R)
    bytes_total = full * sum(s.bytes for s in steps) + sum(s.bytes for s in steps[:rem])
    value_tbs = bytes_total / secs / 1e12
    ms_per_step = secs / K * 1e3
    us_per_token = ms_per_step * 1e3 / T
    log(f"[bench] {ms_per_step * 1e3:.2f} us/layer-step, {value_tbs:.3f} TB/s")

    # dominant kernel alone (gate/up + SwiGLU grouped LUT-GEMV), timed with HIP events
    # around a graph of its launches on the stream they run on
    g_gu = graph_of([lambda s=s: s.run(stages=N.STAGE_GATE_UP) for s in steps])
    time_graph(g_gu, 4)
    r_gu = max(8, min(32, K // R))
    secs_gu = time_graph(g_gu, r_gu)
    dur_gu = secs_gu / (r_gu * len(steps))
    bytes_gu = sum(s.bytes_gate_up for s in steps) / len(steps)
    ach_gu = bytes_gu / dur_gu / 1e9
    g_dn = graph_of([lambda s=s: s.run(stages=N.STAGE_DOWN) for s in steps])
    secs_dn = time_graph(g_dn, r_gu)
    dur_dn = secs_dn / (r_gu * len(steps))
    bytes_dn = sum(s.U * c["H"] * c["I"] * BYTES_PER_WEIGHT for s in steps) / len(steps)
    log(f"[bench] gate_up kernel {dur_gu * 1e6:.2f} us ({ach_gu:.0f} GB/s); "
        f"down+combine {dur_dn * 1e6:.2f} us ({bytes_dn / dur_dn / 1e9:.0f} GB/s)")
    traffic, traffic_src = measured_traffic("decode_gate_up_traffic.md")

    result = {
        "metric": METRIC,
        "value": round(value_tbs, 4),
        "unit": "TB/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (random BL4 codes and sorted N(0,0.02) codebooks of the configured "
                "shapes; N(0,1) bf16 activations and router logits)",
        "config": {"workload": f"Qwen1.5-MoE-A2.7B-shaped MoE layer decode, T={T} token(s): "
                               "H2048 I1408 E60 top-4 softmax, SwiGLU BL4 4-bit (64-weight "
                               f"blocks, 16-entry codebooks); {a.layers} rotating layer copies "
                               "(cold HBM)",
                   "tokens": T, "rotating_layers": a.layers,
                   "avg_distinct_experts": round(sum(s.U for s in steps) / len(steps), 3)},
        "us_per_token": round(us_per_token, 3),
        "tokens_per_s": round(T / (ms_per_step / 1e3), 1),
        "roofline": {"bound": "hbm",
                     "kernel": decode_kernel_label(T, T * (c["k"] + c["S"]), c["E"] + c["S"]),
                     "achieved": round(ach_gu, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(ach_gu / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "traffic_source": traffic_src,
                     "avg_launch_us": round(dur_gu * 1e6, 3),
                     "algorithmic_bytes_per_launch": int(bytes_gu)},
        "kernels": {"decode_down_combine_us": round(dur_dn * 1e6, 3),
                    "decode_down_combine_GBs": round(bytes_dn / dur_dn / 1e9, 1)},
    }
    floor = stream_floor(N, torch, dev, steps, c, graph_of, time_graph) if T == 1 else {}
    if floor:
        floor["decode_T1_floor_over_layer"] = round(floor["decode_T1_stream_floor_all_us"] / (ms_per_step * 1e3), 4)

    # ---------------------------------------------------------- extra configs
    result["extra"] = dict(floor)
    if not a.no_extra:
        extra = dict(floor)
        # hot cache: one layer, same routing every step
        g_hot = graph_of([steps[0].run] * 16)
        time_graph(g_hot, 4)
        sh = time_graph(g_hot, 16) / (16 * 16)
        extra["decode_T1_hot_cache_us"] = round(sh * 1e6, 3)
        extra["decode_T1_hot_cache_TBs"] = round(steps[0].bytes / sh / 1e12, 3)
        for Tn in (8, 32):
            ss = [Step(L, c, Tn) for L in layers]
            g = graph_of([s.run for s in ss])
            time_graph(g, 2)
            sec = time_graph(g, 8) / (8 * len(ss))
            b = sum(s.bytes for s in ss) / len(ss)
            extra[f"decode_T{Tn}_us_per_layer"] = round(sec * 1e6, 2)
            extra[f"decode_T{Tn}_TBs"] = round(b / sec / 1e12, 3)
            extra[f"decode_T{Tn}_avg_distinct_experts"] = round(sum(s.U for s in ss) / len(ss), 2)
            log(f"[bench] decode T={Tn}: {sec * 1e6:.1f} us/layer, {b / sec / 1e12:.3f} TB/s")
            del ss, g
        del layers, steps, g_step, g_gu, g_dn, g_hot, partial
        torch.cuda.empty_cache()
        # DeepSeek-V2-Lite prefill, 2048 tokens, grouped MFMA GEMM
        d = DSV2
        lay = rand_layer(d)
        sp = Step(lay, d, 2048)
        g = graph_of([lambda: sp.run(path=ops.PATH_MFMA)])
        time_graph(g, 2)
        sec = time_graph(g, 10) / 10
        sec_pf = sec
        flops = 6 * d["H"] * d["I"] * 2048 * (d["k"] + d["S"])
        extra["prefill_dsv2_T2048_us"] = round(sec * 1e6, 1)
        extra["prefill_dsv2_T2048_TFLOPs"] = round(flops / sec / 1e12, 1)
        extra["prefill_dsv2_T2048_frac_bf16_peak"] = round(flops / sec / 1e12 / BF16_PEAK_TFLOPS, 4)
        log(f"[bench] prefill DeepSeek T=2048: {sec * 1e6:.0f} us, {flops / sec / 1e12:.1f} TFLOP/s")
        del lay, sp, g
        torch.cuda.empty_cache()
        # the same prefill on the reference's own REF format (uint8 codes into
        # one bf16[256] codebook, bf16 absmax per 128 weights)
        from block_lut_amd.formats import RefStack
        cbk = torch.sort(torch.randn(256, device=dev)).values.to(torch.bfloat16)

        def ref_stack(E, M, K):
            codes = torch.randint(0, 256, (E, M, K), dtype=torch.uint8, device=dev)
            am = (torch.rand((E, M * K // 128), device=dev) * 0.05 + 0.01).to(torch.bfloat16)
            return RefStack(codes, am, cbk, 128)

        E2 = d["E"] + d["S"]
        lay = MoEWeights(ref_stack(E2, 2 * d["I"], d["H"]), ref_stack(E2, d["H"], d["I"]),
                         d["H"], d["I"], d["E"], d["S"])
        sp = Step(lay, d, 2048)
        g = graph_of([lambda: sp.run(path=ops.PATH_MFMA)])
        time_graph(g, 2)
        sec = time_graph(g, 10) / 10
        extra["prefill_ref_dsv2_T2048_us"] = round(sec * 1e6, 1)
        extra["prefill_ref_dsv2_T2048_TFLOPs"] = round(flops / sec / 1e12, 1)
        log(f"[bench] prefill DeepSeek T=2048, REF format: {sec * 1e6:.0f} us, {flops / sec / 1e12:.1f} TFLOP/s")
        del lay, sp, g
        torch.cuda.empty_cache()
        # the main decode workload (T tokens, rotating layer copies) on the REF format
        Eq = c["E"] + c["S"]
        rl = [MoEWeights(ref_stack(Eq, 2 * c["I"], c["H"]), ref_stack(Eq, c["H"], c["I"]),
                         c["H"], c["I"], c["E"], c["S"]) for _ in range(a.layers)]
        rs = [Step(L, c, T) for L in rl]
        g = graph_of([s.run for s in rs])
        time_graph(g, 2)
        sec_r = time_graph(g, 8) / (8 * len(rs))
        b_r = sum(s.U * 3 * c["H"] * c["I"] * (1 + 2 / 128) + 2 * T * c["H"] * 2 for s in rs) / len(rs)
        extra[f"decode_ref_T{T}_us_per_layer"] = round(sec_r * 1e6, 2)
        extra[f"decode_ref_T{T}_TBs"] = round(b_r / sec_r / 1e12, 3)
        log(f"[bench] decode T={T}, REF format: {sec_r * 1e6:.1f} us/layer, {b_r / sec_r / 1e12:.3f} TB/s")
        del rl, rs, g
        torch.cuda.empty_cache()
        ceil = measured_ceilings(torch, dev, d)
        extra.update(ceil)
        extra["prefill_dsv2_T2048_frac_hipblaslt_ceiling"] = round(
            flops / sec_pf / 1e12 / ceil["ceiling_hipblaslt_bf16_TFLOPs"], 4)
        extra["decode_T1_frac_device_copy_ceiling"] = round(
            result["value"] * 1e3 / ceil["ceiling_device_copy_GBs"], 4)
        extra.update(nested_tiers(a, ops, N, torch, dev, NestedExpert, NestedStack, MoEWeights,
                                  graph_of, time_graph))
        torch.cuda.empty_cache()
        extra.update(mixtral_stack(ops, torch, dev, rand_stack, MoEWeights, graph_of, time_graph))
        torch.cuda.empty_cache()
        # switch-base-8 single BL4 linear 768 -> 3072, one token of fp32 activations (the
        # configured precision, fp32 output); the same with the row rounded to bf16 beside it
        st1 = rand_stack(1, 3072, 768)
        for name, xdt in (("switch_linear_768x3072_us", torch.float32),
                          ("switch_linear_768x3072_bf16x_us", torch.bfloat16)):
            x1 = torch.randn((1, 768), device=dev).to(xdt)
            y1 = torch.empty((1, 3072), dtype=torch.float32, device=dev)

            def c1(x1=x1, y1=y1):
                ops.gemv(st1, x1, out=y1)
            g = graph_of([c1] * 32)
            time_graph(g, 2)
            sec = time_graph(g, 10) / (10 * 32)
            extra[name] = round(sec * 1e6, 3)
        extra["switch_linear_768x3072_GBs"] = round(3072 * 768 * BYTES_PER_WEIGHT / (extra["switch_linear_768x3072_us"] * 1e-6) / 1e9, 1)
        result["extra"] = extra

    # ------------------------------------------------------------ CPU leg
    if not a.no_cpu:
        result["cpu_baseline"] = cpu_baseline(a, c, T)
        if not a.no_extra:
            result["extra"].update(cpu_other_workloads(result["extra"].pop("_nested_touched", None)))
    result.get("extra", {}).pop("_nested_touched", None)

    print(json.dumps(result), flush=True)


def stream_floor(N, torch, dev, steps, c, graph_of, time_graph):
    """HBM floor of the one-token layer: lutmoe_decode_stream_probe launches, whose CTAs
    issue exactly the weight loads of the one-token gate/up and down kernels for each
    step's own experts (the same rotating layers) and nothing else, graph-timed like the
    layer.  "all": both kernels' loads in one launch (the step's bytes); "w13": the gate/up
    kernel's alone (the gate/up bytes)."""
    import ctypes
    lib = N.lib()
    for s in steps:
        s.slot_ids = s.ids.reshape(-1).contiguous()

    out = {}
    for which, name, nb in ((3, "all", lambda s: s.bytes - 2 * c["H"] * 2),
                            (1, "w13", lambda s: s.bytes_gate_up - c["H"] * 2)):
        sinks = []
        for s in steps:
            d = s.layer.desc()
            n = int(lib.lutmoe_decode_stream_probe_sink_words(ctypes.byref(d), c["k"], which))
            sinks.append(torch.empty(max(1, n), dtype=torch.int32, device=dev))

        def probe(s, sink, which=which):
            d = s.layer.desc()
            N.check("lutmoe_decode_stream_probe",
                    lib.lutmoe_decode_stream_probe(ctypes.byref(d), s.slot_ids.data_ptr(), c["k"], which,
                                                   sink.data_ptr(), torch.cuda.current_stream().cuda_stream))
        g = graph_of([lambda s=s, k=k: probe(s, k) for s, k in zip(steps, sinks)])
        time_graph(g, 4)
        sec = time_graph(g, 16) / (16 * len(steps))
        by = sum(nb(s) for s in steps) / len(steps)
        out[f"decode_T1_stream_floor_{name}_us"] = round(sec * 1e6, 3)
        out[f"decode_T1_stream_floor_{name}_TBs"] = round(by / sec / 1e12, 3)
        log(f"[bench] stream floor ({name}): {sec * 1e6:.2f} us, {by / sec / 1e12:.3f} TB/s")
        del g
    return out


def measured_ceilings(torch, dev, d, T=2048):
    """Measured ceilings beside the published peaks: a 1 GiB device-to-device copy (read +
    write bytes per second), and torch's bf16 GEMM (hipBLASLt) on the dense-equivalent shapes
    of the DeepSeek T=2048 prefill: [T*(k+S), H] x [H, 2I] and [T*(k+S), I] x [I, H]."""
    def timed(fn, reps):
        fn()
        torch.cuda.synchronize()
        t0 = torch.cuda.Event(enable_timing=True)
        t1 = torch.cuda.Event(enable_timing=True)
        t0.record()
        for _ in range(reps):
            fn()
        t1.record()
        torch.cuda.synchronize()
        return t0.elapsed_time(t1) / reps * 1e-3

    out = {}
    src = torch.empty(1 << 29, dtype=torch.bfloat16, device=dev).normal_()
    dst = torch.empty_like(src)
    sec = timed(lambda: dst.copy_(src), 10)
    out["ceiling_device_copy_GBs"] = round(2 * src.numel() * 2 / sec / 1e9, 1)
    del src, dst
    torch.cuda.empty_cache()
    P = T * (d["k"] + d["S"])
    fl = tsum = 0.0
    for K, Nn in ((d["H"], 2 * d["I"]), (d["I"], d["H"])):
        a_ = torch.randn(P, K, device=dev).to(torch.bfloat16)
        b_ = torch.randn(K, Nn, device=dev).to(torch.bfloat16)
        o_ = torch.empty(P, Nn, dtype=torch.bfloat16, device=dev)
        tsum += timed(lambda: torch.mm(a_, b_, out=o_), 20)
        fl += 2.0 * P * K * Nn
        del a_, b_, o_
    out["ceiling_hipblaslt_bf16_TFLOPs"] = round(fl / tsum / 1e12, 1)
    out["ceiling_blas_library"] = str(torch.backends.cuda.preferred_blas_library())
    log(f"[bench] ceilings: device copy {out['ceiling_device_copy_GBs']:.0f} GB/s, "
        f"bf16 GEMM {out['ceiling_hipblaslt_bf16_TFLOPs']:.0f} TFLOP/s")
    return out


def mixtral_stack(ops, torch, dev, rand_stack, MoEWeights, graph_of, time_graph):
    """Mixtral-8x7B-shaped stack of 32 MoE layers resident in HBM (H4096,
    I14336, 8 experts, top-2 softmax with renormalisation, SwiGLU BL4: 1.41 GB
    per layer, 45 GB in all).  Decode B=1 and B=64: one step = the batch
    through all 32 layers (each layer its own router logits); bytes = the
    distinct routed experts of every layer at 1.0 B/weight + activations.
    Prefill: 4096 tokens through all 32 layers on the grouped MFMA path;
    flops = 32 * 6*H*I*T*k."""
    H, I, E, k, L = 4096, 14336, 8, 2, 32
    log(f"[bench] Mixtral stack: building {L} layers ({L * 3 * H * I * E / 1e9:.1f} GB)")
    layers = [MoEWeights(rand_stack(E, 2 * I, H), rand_stack(E, H, I), H, I, E, 0) for _ in range(L)]
    gen = torch.Generator(device="cpu").manual_seed(8)
    res = {}
    for B in (1, 64):
        xs = [torch.randn((B, H), generator=gen).to(torch.bfloat16).to(dev) for _ in range(L)]
        lgs = [torch.randn((B, E), generator=gen).to(dev) for _ in range(L)]
        outs = [torch.empty((B, H), dtype=torch.bfloat16, device=dev) for _ in range(L)]
        ws = ops.new_workspace(layers[0], B, k, dev)
        U = sum(int(torch.unique(torch.topk(lg, k, dim=1).indices).numel()) for lg in lgs)
        calls = [lambda l=l, x=x, lg=lg, o=o: ops.moe_forward_logits(l, x, lg, k, renormalize=True, out=o,
                                                                     workspace=ws)
                 for l, x, lg, o in zip(layers, xs, lgs, outs)]
        g = graph_of(calls)
        time_graph(g, 2)
        sec = time_graph(g, 6) / 6
        by = U * 3 * H * I * BYTES_PER_WEIGHT + L * 2 * B * H * 2
        res[f"mixtral_decode_B{B}_ms_per_step"] = round(sec * 1e3, 4)
        res[f"mixtral_decode_B{B}_us_per_layer"] = round(sec * 1e6 / L, 2)
        res[f"mixtral_decode_B{B}_TBs"] = round(by / sec / 1e12, 3)
        log(f"[bench] Mixtral decode B={B}: {sec * 1e3:.3f} ms per step of {L} layers "
            f"({sec * 1e6 / L:.1f} us/layer), {by / sec / 1e12:.3f} TB/s")
        del xs, lgs, outs, ws, calls, g
    T = 4096
    x = torch.randn((T, H), generator=gen).to(torch.bfloat16).to(dev)
    lgs = [torch.randn((T, E), generator=gen).to(dev) for _ in range(L)]
    out = torch.empty((T, H), dtype=torch.bfloat16, device=dev)
    ws = ops.new_workspace(layers[0], T, k, dev)
    calls = [lambda l=l, lg=lg: ops.moe_forward_logits(l, x, lg, k, renormalize=True, out=out, workspace=ws,
                                                       path=ops.PATH_MFMA)
             for l, lg in zip(layers, lgs)]
    g = graph_of(calls)
    time_graph(g, 1)
    sec = time_graph(g, 3) / 3
    flops = L * 6 * H * I * T * k
    res["mixtral_prefill_T4096_ms_per_stack"] = round(sec * 1e3, 3)
    res["mixtral_prefill_T4096_TFLOPs"] = round(flops / sec / 1e12, 1)
    log(f"[bench] Mixtral prefill T=4096: {sec * 1e3:.2f} ms per {L} layers, {flops / sec / 1e12:.1f} TFLOP/s")
    del layers, x, lgs, out, ws, calls, g
    torch.cuda.empty_cache()
    # the dense bf16 ceiling on Mixtral's own shapes: [T*k, H] x [H, 2I] and [T*k, I] x [I, H]
    P = T * k
    fl = tsum = 0.0
    for Kd, Nd in ((H, 2 * I), (I, H)):
        a_ = torch.randn(P, Kd, device=dev).to(torch.bfloat16)
        b_ = torch.randn(Kd, Nd, device=dev).to(torch.bfloat16)
        o_ = torch.empty(P, Nd, dtype=torch.bfloat16, device=dev)
        torch.mm(a_, b_, out=o_)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(10):
            torch.mm(a_, b_, out=o_)
        e1.record()
        torch.cuda.synchronize()
        tsum += e0.elapsed_time(e1) / 10 * 1e-3
        fl += 2.0 * P * Kd * Nd
        del a_, b_, o_
    ceil = fl / tsum / 1e12
    res["mixtral_ceiling_hipblaslt_bf16_TFLOPs"] = round(ceil, 1)
    res["mixtral_prefill_T4096_frac_hipblaslt_ceiling"] = round(flops / sec / 1e12 / ceil, 4)
    log(f"[bench] Mixtral-shape bf16 GEMM ceiling {ceil:.0f} TFLOP/s")
    return res


def nested_tiers(a, ops, N, torch, dev, NestedExpert, NestedStack, MoEWeights, graph_of,
                 time_graph):
    """NestedLUT tier workload: Qwen1.5-MoE shape (H2048, I1408, E60, top-4),
    experts at 2/3/4 bits (20 each, seeded permutation), expert popularity
    p_e ~ rank^-1.1 (seeded rank permutation) and Gumbel-top-4 routing: the
    router logits are log p_e + Gumbel noise, so the kernels' own softmax /
    top-k performs the Gumbel-top-k selection.  Decode T=16 (HBM bytes of the
    touched experts at their tiers) and prefill T=1024 (MFMA flops)."""
    import numpy as np
    H, I, E, k = 2048, 1408, 60, 4
    rng = np.random.default_rng(2024)
    bits = np.array([2] * 20 + [3] * 20 + [4] * 20)[rng.permutation(E)]
    rank = rng.permutation(E) + 1
    logp = np.log(rank.astype(np.float64) ** -1.1 / np.sum(rank.astype(np.float64) ** -1.1))

    def stack(M, K):
        ex = []
        n = M * K
        for b in bits:
            b = int(b)
            size = n // 4 + (n // 8 if b >= 3 else 0) + (n // 8 if b >= 4 else 0)
            planes = torch.randint(0, 256, (size,), dtype=torch.uint8, device=dev)
            tab = torch.sort(torch.randn((M, K // 64, 1 << b), device=dev) * 0.02, dim=-1).values
            ex.append(NestedExpert(b, planes, tab.to(torch.bfloat16)))
        return NestedStack(ex, M, K)

    def exp_bytes(b):
        w = 3 * H * I
        return w * b / 8 + (w / 64) * (1 << b) * 2

    nl = 4   # 4 layer copies: about 1.4 GB, past the Infinity Cache
    layers = [MoEWeights(stack(2 * I, H), stack(H, I), H, I, E, 0) for _ in range(nl)]
    out = {"_nested_touched": {}}
    for T, path, label in ((16, ops.PATH_GEMV, "decode"), (1024, ops.PATH_MFMA, "prefill")):
        steps = []
        touched = {2: 0, 3: 0, 4: 0}
        for L in layers:
            g = rng.gumbel(size=(T, E))
            lg = torch.from_numpy((logp[None, :] + g).astype(np.float32)).to(dev)
            ids = np.argsort(-(logp[None, :] + g), axis=1, kind="stable")[:, :k]
            uniq = np.unique(ids)
            for e in uniq:
                touched[int(bits[e])] += 1 / nl
            x = torch.randn((T, H), device=dev).to(torch.bfloat16)
            o = torch.empty((T, H), dtype=torch.bfloat16, device=dev)
            ws = ops.new_workspace(L, T, k, dev)
            steps.append((L, lg, x, o, ws, sum(exp_bytes(int(bits[e])) for e in uniq)))
        out["_nested_touched"][T] = touched
        fns = [(lambda s=s: ops.moe_forward_logits(s[0], s[2], s[1], k, out=s[3], workspace=s[4],
                                                   path=path)) for s in steps]
        g = graph_of(fns)
        time_graph(g, 2)
        sec = time_graph(g, 8) / (8 * len(steps))
        if label == "decode":
            b = sum(s[5] for s in steps) / len(steps) + 2 * T * H * 2
            out["nested_tiers_decode_T16_us_per_layer"] = round(sec * 1e6, 2)
            out["nested_tiers_decode_T16_TBs"] = round(b / sec / 1e12, 3)
            log(f"[bench] nested tiers decode T=16: {sec * 1e6:.1f} us/layer, {b / sec / 1e12:.3f} TB/s")
        else:
            fl = 6 * H * I * T * k
            out["nested_tiers_prefill_T1024_us"] = round(sec * 1e6, 1)
            out["nested_tiers_prefill_T1024_TFLOPs"] = round(fl / sec / 1e12, 1)
            log(f"[bench] nested tiers prefill T=1024: {sec * 1e6:.0f} us, {fl / sec / 1e12:.1f} TFLOP/s")
        del g
    del layers
    torch.cuda.empty_cache()
    return out


def cpu_model() -> str:
    """The host CPU as /proc/cpuinfo names it, with its family / model / stepping numbers
    (a virtualised host may report only a short model name)."""
    info = {}
    try:
        for line in open("/proc/cpuinfo"):
            if ":" in line:
                key, val = (t.strip() for t in line.split(":", 1))
                if key in ("model name", "vendor_id", "cpu family", "model", "stepping") and key not in info:
                    info[key] = val
    except OSError:
        return "unknown"
    return (f"{info.get('model name', 'unknown')} ({info.get('vendor_id', '?')} family "
            f"{info.get('cpu family', '?')} model {info.get('model', '?')} stepping {info.get('stepping', '?')})")


def cpu_other_workloads(nested_touched):
    """The reference's CPU dequant + matmul path (oracle/cpu_baseline.py) beside the other
    workloads, on the host cores, each on a bounded sample (about 5 s in all):
      switch-base-8 single linear: fp32 F.linear of one fp32 row over the dequantised
        [3072, 768] BL4 weights, median of >= 20 calls;
      DeepSeek-V2-Lite prefill T=2048: the reference's multi-token branch per expert
        (dequantise W13 and W2, both projections over all 2048 tokens), median over 6
        experts, times the step's 66 experts;
      NestedLUT tiers: the same per expert at 2, 3 and 4 bits (2 experts each) for T=16
        and T=1024, times the step's touched experts per tier (the bench's own routing).
    Figures: ms per layer step, and the GPU metrics' units (TB/s of algorithmic bytes,
    TFLOP/s of routed flops)."""
    import statistics
    import torch
    from oracle.cpu_baseline import (bl4_dequant_torch, expert_all_tokens, linear_fp32,
                                     table_dequant_torch)
    ncores = len(os.sched_getaffinity(0))
    torch.set_num_threads(ncores)
    g = torch.Generator().manual_seed(77)
    out = {"cpu_other_cores": ncores}

    def timed(fn, n, warm=2):
        for _ in range(warm):
            fn()
        ts = []
        for _ in range(n):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
        return statistics.median(ts)

    def bl4(M, K):
        return (torch.randint(0, 256, (M, K // 2), dtype=torch.uint8, generator=g),
                torch.sort(torch.randn((M, K // 64, 16), generator=g) * 0.02, dim=-1).values.to(torch.bfloat16))

    c1 = bl4(3072, 768)
    x1 = torch.randn((1, 768), generator=g)
    sec = timed(lambda: linear_fp32(x1, *c1), 40, warm=3)
    out["cpu_switch_linear_768x3072_us"] = round(sec * 1e6, 1)
    out["cpu_switch_linear_768x3072_GBs"] = round(3072 * 768 * BYTES_PER_WEIGHT / sec / 1e9, 3)

    H, I = 2048, 1408

    def expert_time(T, make13, make2, n):
        """Median over n fresh experts of dequantise + both projections over all T tokens;
        make13 / make2 build an expert's stored weights (untimed) and return its dequantiser."""
        x = torch.randn((T, H), generator=g).to(torch.bfloat16)
        ts = []
        for _ in range(n):
            deq13, deq2 = make13(), make2()
            t0 = time.perf_counter()
            expert_all_tokens(x, deq13(), deq2())
            ts.append(time.perf_counter() - t0)
        return statistics.median(ts)

    def bl4_expert(M, K):
        st = bl4(M, K)
        return lambda: bl4_dequant_torch(*st)

    d = DSV2
    per = expert_time(2048, lambda: bl4_expert(2 * I, H), lambda: bl4_expert(H, I), 6)
    n_exp = d["E"] + d["S"]
    step = per * n_exp
    flops = 6 * d["H"] * d["I"] * 2048 * (d["k"] + d["S"])
    out["cpu_prefill_dsv2_T2048_ms"] = round(step * 1e3, 1)
    out["cpu_prefill_dsv2_T2048_TFLOPs"] = round(flops / step / 1e12, 4)
    out["cpu_prefill_dsv2_T2048_sample"] = (f"median of 6 experts ({per * 1e3:.0f} ms each: dequantise W13 + W2, "
                                            f"F.linear over all 2048 tokens) x {n_exp} experts")
    if nested_touched:
        for T, key in ((16, "decode_T16"), (1024, "prefill_T1024")):
            tot = 0.0
            for b in (2, 3, 4):
                def nested_expert(M, K, b=b):
                    codes = torch.randint(0, 1 << b, (M, K), dtype=torch.uint8, generator=g)
                    tab = torch.sort(torch.randn((M, K // 64, 1 << b), generator=g) * 0.02,
                                     dim=-1).values.to(torch.bfloat16)
                    return lambda: table_dequant_torch(codes, tab)
                tb = expert_time(T, lambda: nested_expert(2 * I, H), lambda: nested_expert(H, I), 2)
                tot += tb * nested_touched[T][b]
            out[f"cpu_nested_tiers_{key}_ms"] = round(tot * 1e3, 1)
            if T == 1024:
                out[f"cpu_nested_tiers_{key}_TFLOPs"] = round(6 * H * I * T * 4 / tot / 1e12, 4)
        out["cpu_nested_tiers_sample"] = ("per tier the median of 2 experts (dequantise through the tier's "
                                          "table, F.linear over all tokens) x the step's touched experts "
                                          "of that tier (average over the bench's 4 layers)")
    torch.set_num_threads(ncores)
    return out


def cpu_baseline(a, c, T):
    """The reference's CPU dequant + matmul path on a bounded sample of the same
    workload (Qwen layer decode, T tokens, top-4 of 60 experts): 3 warm-up steps, then
    the median of the timed steps, on all host cores (40 % of --cpu-seconds) and on one
    thread (60 %), at least 20 steps each."""
    import statistics
    import torch
    from oracle.cpu_baseline import moe_layer_step
    ncores = len(os.sched_getaffinity(0))
    g = torch.Generator().manual_seed(99)
    H, I, E, k = c["H"], c["I"], c["E"], c["k"]
    t_gen = time.perf_counter()
    experts13, experts2 = {}, {}
    for e in range(E):   # every expert once: the sample's steps route over all of them
        experts13[e] = (torch.randint(0, 256, (2 * I, H // 2), dtype=torch.uint8, generator=g),
                        torch.sort(torch.randn((2 * I, H // 64, 16), generator=g) * 0.02,
                                   dim=-1).values.to(torch.bfloat16))
        experts2[e] = (torch.randint(0, 256, (H, I // 2), dtype=torch.uint8, generator=g),
                       torch.sort(torch.randn((H, I // 64, 16), generator=g) * 0.02,
                                  dim=-1).values.to(torch.bfloat16))
    t_gen = time.perf_counter() - t_gen
    inputs = []
    for _ in range(64):
        logits = torch.randn((T, E), generator=g)
        w, ids = torch.topk(torch.softmax(logits, -1), k, dim=-1)
        x = torch.randn((T, H), generator=g).to(torch.bfloat16)
        nbytes = int(torch.unique(ids).numel()) * 3 * H * I * BYTES_PER_WEIGHT + 2 * T * H * 2
        inputs.append((x, ids, w, nbytes))

    def measure(threads, seconds, min_reps=20, warm=3):
        torch.set_num_threads(threads)
        for i in range(warm):
            x, ids, w, _ = inputs[i]
            moe_layer_step(x, ids, w, experts13, experts2)
        times, by = [], []
        while len(times) < min_reps or sum(times) < seconds:
            x, ids, w, nb = inputs[(warm + len(times)) % len(inputs)]
            t0 = time.perf_counter()
            moe_layer_step(x, ids, w, experts13, experts2)
            times.append(time.perf_counter() - t0)
            by.append(nb)
        med = statistics.median(times)
        return med, statistics.median(by), sum(times), len(times)

    med_all, by_all, tot_all, n_all = measure(ncores, 0.4 * a.cpu_seconds)
    med_one, by_one, tot_one, n_one = measure(1, 0.6 * a.cpu_seconds)
    torch.set_num_threads(ncores)
    return {"value": round(by_all / med_all / 1e12, 6), "unit": "TB/s", "cores": ncores, "kind": "port",
            "ms_per_step": round(med_all * 1e3, 3),
            "us_per_token": round(med_all / T * 1e6, 1),
            "one_thread": {"value": round(by_one / med_one / 1e12, 6), "unit": "TB/s",
                           "ms_per_step": round(med_one * 1e3, 3)},
            "cpu_model": cpu_model(),
            "sample": f"Qwen-shaped layer decode steps (T={T}, top-4 of 60 BL4 experts), torch CPU "
                      f"dequant gather + bf16 F.linear: median of {n_all} steps on {ncores} threads "
                      f"({tot_all:.1f} s) and of {n_one} steps on 1 thread ({tot_one:.1f} s), each after "
                      f"3 warm-up steps; weights generated beforehand ({t_gen:.1f} s, untimed)"}


if __name__ == "__main__":
    main()
