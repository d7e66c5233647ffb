"""HIP graph capture of the library's calls (torch.cuda.graph over the caller's
stream): the allocation-free routed decode layer
(k3_hip_moe_route_layer_device_noalloc) and a one-position K3-style MoE block
(k3_hip_moe_block_device, whose shared expert then runs on the caller's
stream instead of the library's side stream).  Each graph is replayed three
times, with eager calls of the same entry point on other inputs, and host
synchronisations, between the replays; every replay must write exactly the
eager result, bit for bit (the outputs are poisoned with NaN before each
replay, so a replay that wrote nothing fails).  The captured calls launch
kernels only: zero fills are kernels, not memset nodes.
"""
import ctypes as C

import numpy as np
import pytest

from deltafin_amd import synth

pytestmark = pytest.mark.gpu

REPLAYS = 3


def say(msg):
    print(f"[gpu-case] {msg}", flush=True)


def _bits(t):
    import torch
    return t.view(torch.int16 if t.dtype == torch.bfloat16 else torch.int32).cpu().numpy()


def test_noalloc_route_layer_graph_replays(gpu):
    import torch
    from deltafin_amd import _lib, moe
    g = moe.preset(2)
    n_bank, k = 40, 16
    stride = g.expert_span
    say("graph: no-alloc routed decode layer, preset 2, top-16 of 40, bf16 x/out")
    bank = torch.empty(n_bank * stride, dtype=torch.uint8, device="cuda")
    moe.synth_bank(g, bank, stride, n_bank, 0, 909)
    rng = np.random.default_rng(909)
    logits = torch.from_numpy(rng.standard_normal((2, n_bank)).astype(np.float32)).cuda()
    x32 = synth.bf16_bits_to_f32(synth.to_bf16_bits(
        rng.standard_normal((2, g.hidden)).astype(np.float32)))
    x = torch.from_numpy(x32).cuda().to(torch.bfloat16)
    outs = torch.empty((2, g.hidden), dtype=torch.bfloat16, device="cuda")
    ids = torch.empty((2, k), dtype=torch.int32, device="cuda")
    wts = torch.empty((2, k), dtype=torch.float32, device="cuda")
    lib = _lib.load()

    def call(i):
        rc = lib.k3_hip_moe_route_layer_device_noalloc(
            C.byref(g), bank.data_ptr(), stride, n_bank, logits[i].data_ptr(), k,
            x[i].data_ptr(), _lib.K3_DTYPE_BF16, outs[i].data_ptr(), _lib.K3_DTYPE_BF16,
            ids[i].data_ptr(), wts[i].data_ptr(), moe.stream_handle())
        assert rc == 0, _lib.last_error()

    call(0)
    call(1)
    torch.cuda.synchronize()
    want = [(_bits(outs[i]), ids[i].cpu().numpy(), _bits(wts[i])) for i in range(2)]
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        call(0)
    for r in range(REPLAYS):
        outs[0].fill_(float("nan"))
        ids[0].fill_(-1)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert np.array_equal(_bits(outs[0]), want[0][0]), f"replay {r}: output"
        assert np.array_equal(ids[0].cpu().numpy(), want[0][1]), f"replay {r}: route ids"
        assert np.array_equal(_bits(wts[0]), want[0][2]), f"replay {r}: route weights"
        call(1)  # eager work on the same scratch between replays
        torch.cuda.synchronize()
        assert np.array_equal(_bits(outs[1]), want[1][0]), f"eager call after replay {r}"


def test_block_one_position_graph_replays(gpu):
    import torch
    from deltafin_amd import _lib, moe, spine
    H, R, Sh, E, I, K = 576, 256, 320, 40, 128, 8
    say("graph: one-position MoE block, small BF16 spine (576/256/320, 40 experts, top-8)")
    g = _lib.geometry(R, I, _lib.K3_ACT_SITU)
    stride = g.expert_span
    bank = torch.empty(E * stride, dtype=torch.uint8, device="cuda")
    moe.synth_bank(g, bank, stride, E, 0, 313)
    rng = np.random.default_rng(313)

    def mat(rows, cols):
        v = rng.standard_normal((rows, cols), dtype=np.float32) * np.float32(0.05)
        return torch.from_numpy((v.view(np.uint32) >> 16).astype(np.uint16).view(np.int16)).cuda()

    sp = spine.MoeSpine("bf16", mat(E, H),
                        torch.from_numpy((rng.standard_normal(E) * 0.01).astype(np.float32)).cuda(),
                        mat(R, H),
                        torch.from_numpy((1.0 + 0.1 * rng.standard_normal(R)).astype(np.float32)).cuda(),
                        mat(H, R), mat(Sh, H), mat(Sh, H), mat(H, Sh), top_k=K)
    hidden = torch.from_numpy(rng.standard_normal((2, H), dtype=np.float32)).cuda()
    ws = spine.moe_block_workspace(sp, g, 1)
    ws_eager = spine.moe_block_workspace(sp, g, 1)
    out = torch.empty((1, H), dtype=torch.float32, device="cuda")
    o0, i0, w0 = spine.moe_block(sp, g, bank, stride, hidden[0:1], workspace=ws)
    o1, i1, w1 = spine.moe_block(sp, g, bank, stride, hidden[1:2], workspace=ws_eager)
    torch.cuda.synchronize()
    want0, want1 = _bits(o0), _bits(o1)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        gi = spine.moe_block(sp, g, bank, stride, hidden[0:1], workspace=ws, out=out)
    for r in range(REPLAYS):
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert np.array_equal(_bits(out), want0), f"replay {r}: block output"
        assert np.array_equal(gi[1].cpu().numpy(), i0.cpu().numpy()), f"replay {r}: route ids"
        e1, _, _ = spine.moe_block(sp, g, bank, stride, hidden[1:2], workspace=ws_eager)
        torch.cuda.synchronize()
        assert np.array_equal(_bits(e1), want1), f"eager block after replay {r}"
