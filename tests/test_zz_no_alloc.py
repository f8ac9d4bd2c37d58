"""lutmoe_moe_forward_noalloc (the library's own device scratch, no allocation)
against lutmoe_moe_forward with a caller workspace, both through the C ABI:
bit-identical outputs on two calls in a row, the second with a smaller input,
and a layer too large for the scratch rejected with the sizes in the error text."""
import ctypes

import numpy as np
import pytest

import oracle as O
from lutmoe_testutil import BL4Expertset, rel_maxabs, to_dev_bf16

pytestmark = pytest.mark.gpu


def _call_both(N, moe, x, w, ids, out_a, out_b, ws, k, path):
    import torch
    T = x.shape[0]
    d = moe.desc()
    stream = torch.cuda.current_stream().cuda_stream
    rc = N.lib().lutmoe_moe_forward(ctypes.byref(d), x.data_ptr(), w.data_ptr(), ids.data_ptr(), T, k,
                                    out_a.data_ptr(), N.DTYPE_F32, ws.data_ptr(), ws.numel(), path, stream)
    N.check("lutmoe_moe_forward", rc)
    rc = N.lib().lutmoe_moe_forward_noalloc(ctypes.byref(d), x.data_ptr(), w.data_ptr(), ids.data_ptr(), T, k,
                                            out_b.data_ptr(), N.DTYPE_F32, path, stream)
    N.check("lutmoe_moe_forward_noalloc", rc)
    torch.cuda.synchronize()


@pytest.mark.parametrize("Ts,path", [((9, 3), 0), ((1, 1), 0), ((40, 5), 0), ((24, 2), 2)])
def test_noalloc_matches_workspace_entry_point(gpu, Ts, path):
    import torch
    from block_lut_amd import _native as N
    from block_lut_amd import ops
    from block_lut_amd.formats import MoEWeights
    E, S, k, H, I = 8, 1, 2, 512, 320
    w13 = BL4Expertset(E + S, 2 * I, H, seed=81, n_iter=8)
    w2 = BL4Expertset(E + S, H, I, seed=82, n_iter=8)
    moe = MoEWeights(w13.stack(gpu), w2.stack(gpu), H, I, E, S)
    rng = np.random.default_rng(sum(Ts) + path)
    for T in Ts:
        xb = O.f32_to_bf16(rng.standard_normal((T, H)).astype(np.float32))
        rw, rids = O.route(rng.standard_normal((T, E)).astype(np.float32), k)
        x = to_dev_bf16(xb, gpu)
        w = torch.from_numpy(rw).to(gpu)
        ids = torch.from_numpy(rids.astype(np.int32)).to(gpu)
        out_a = torch.full((T, H), float("nan"), dtype=torch.float32, device=gpu)
        out_b = torch.full((T, H), float("nan"), dtype=torch.float32, device=gpu)
        ws = ops.new_workspace(moe, T, k, gpu)
        _call_both(N, moe, x, w, ids, out_a, out_b, ws, k, path)
        assert torch.equal(out_a, out_b), T
        ref = O.moe_layer(xb, rids, rw, w13.deq_f32, w2.deq_f32,
                          shared=[(w13.deq_f32(E + s), w2.deq_f32(E + s)) for s in range(S)])
        assert rel_maxabs(out_b.cpu().numpy(), ref) <= 1e-3, T


def test_noalloc_rejects_layers_beyond_its_scratch(gpu):
    import torch
    from block_lut_amd import _native as N
    from block_lut_amd.formats import BL4Stack, MoEWeights
    H, I, E, k, T = 2048, 1408, 4, 2, 4096
    codes13 = torch.zeros((E, 2 * I, H // 2), dtype=torch.uint8, device=gpu)
    tabs13 = torch.zeros((E, 2 * I, H // 64, 16), dtype=torch.bfloat16, device=gpu)
    codes2 = torch.zeros((E, H, I // 2), dtype=torch.uint8, device=gpu)
    tabs2 = torch.zeros((E, H, I // 64, 16), dtype=torch.bfloat16, device=gpu)
    moe = MoEWeights(BL4Stack(codes13, tabs13), BL4Stack(codes2, tabs2), H, I, E, 0)
    d = moe.desc()
    need = N.lib().lutmoe_moe_workspace_size(ctypes.byref(d), T, k)
    assert need > (32 << 20)
    x = torch.zeros((T, H), dtype=torch.bfloat16, device=gpu)
    w = torch.zeros((T, k), dtype=torch.float32, device=gpu)
    ids = torch.zeros((T, k), dtype=torch.int32, device=gpu)
    out = torch.zeros((T, H), dtype=torch.float32, device=gpu)
    rc = N.lib().lutmoe_moe_forward_noalloc(ctypes.byref(d), x.data_ptr(), w.data_ptr(), ids.data_ptr(), T, k,
                                            out.data_ptr(), N.DTYPE_F32, 0,
                                            torch.cuda.current_stream().cuda_stream)
    assert rc == N.LUTMOE_EWORKSPACE
    msg = N.lib().lutmoe_last_error().decode()
    assert str(need) in msg and str(32 << 20) in msg
    torch.cuda.synchronize()
    assert torch.count_nonzero(out) == 0


@pytest.mark.parametrize("T,path", [(1, 0), (9, 0), (40, 0)])
def test_noalloc_graph_capture(gpu, T, path):
    """lutmoe_noalloc_prepare, then lutmoe_moe_forward_noalloc captured into a HIP graph
    (torch.cuda.CUDAGraph) and replayed three times with new activations and routing
    copied into its input buffers between replays, with eager work and synchronisations in
    between: every replay equals lutmoe_moe_forward with a caller workspace, bit for bit."""
    import torch
    from block_lut_amd import _native as N
    from block_lut_amd import ops
    from block_lut_amd.formats import MoEWeights
    E, S, k, H, I = 8, 1, 2, 512, 320
    w13 = BL4Expertset(E + S, 2 * I, H, seed=83, n_iter=8)
    w2 = BL4Expertset(E + S, H, I, seed=84, n_iter=8)
    moe = MoEWeights(w13.stack(gpu), w2.stack(gpu), H, I, E, S)
    d = moe.desc()
    assert N.lib().lutmoe_noalloc_prepare() == 0
    x = torch.zeros((T, H), dtype=torch.bfloat16, device=gpu)
    w = torch.zeros((T, k), dtype=torch.float32, device=gpu)
    ids = torch.zeros((T, k), dtype=torch.int32, device=gpu)
    out = torch.zeros((T, H), dtype=torch.float32, device=gpu)

    def call():
        N.check("lutmoe_moe_forward_noalloc",
                N.lib().lutmoe_moe_forward_noalloc(ctypes.byref(d), x.data_ptr(), w.data_ptr(), ids.data_ptr(), T,
                                                   k, out.data_ptr(), N.DTYPE_F32, path,
                                                   torch.cuda.current_stream().cuda_stream))
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        call()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        call()
    torch.cuda.synchronize()
    rng = np.random.default_rng(500 + T)
    ws = ops.new_workspace(moe, T, k, gpu)
    for rep in range(3):
        xb = O.f32_to_bf16(rng.standard_normal((T, H)).astype(np.float32))
        rw, rids = O.route(rng.standard_normal((T, E)).astype(np.float32), k)
        x.copy_(to_dev_bf16(xb, gpu))
        w.copy_(torch.from_numpy(rw).to(gpu))
        ids.copy_(torch.from_numpy(rids.astype(np.int32)).to(gpu))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got = out.clone()
        ref_out = torch.full((T, H), float("nan"), dtype=torch.float32, device=gpu)
        N.check("lutmoe_moe_forward",
                N.lib().lutmoe_moe_forward(ctypes.byref(d), x.data_ptr(), w.data_ptr(), ids.data_ptr(), T, k,
                                           ref_out.data_ptr(), N.DTYPE_F32, ws.data_ptr(), ws.numel(), path,
                                           torch.cuda.current_stream().cuda_stream))
        torch.cuda.synchronize()
        assert torch.equal(got, ref_out), (T, rep)
        ref = O.moe_layer(xb, rids, rw, w13.deq_f32, w2.deq_f32,
                          shared=[(w13.deq_f32(E + s), w2.deq_f32(E + s)) for s in range(S)])
        assert rel_maxabs(got.cpu().numpy(), ref) <= 1e-3, (T, rep)
