"""GPU tests of the fused single-launch decode path (k_decode_fused), selected
with k3_hip_set_fused_decode (the two-launch path is the default).

The fused kernel runs the router, gate/up, down and the ordered combine of one
token in one launch, handing h between workgroups through device memory and a
per-workspace ticket counter.  Its arithmetic is that of the two-launch path
(k_glu_decode + k_down_g64), so every output here must be bit-identical to the
two-launch output on the same inputs, and both must match the fp64 oracle
(oracle.moe_layer_f64, the restatement of provider_cuda_moe.cpp:1203-1258)
within the parity tolerance.

Geometries cover each column split of the gate/up sweep (S = 1, 2, 4 waves)
and several down batch counts (NB = 2, 4, 7, 8), SiLU and SiTU.  Back-to-back
launches on one workspace check that each launch returns its ticket counters to
zero; launches on two streams check two fused kernels in flight at once.
"""
import numpy as np
import pytest

import oracle
from deltafin_amd import synth

pytestmark = pytest.mark.gpu

TOL = 1e-3
N_BANK = 24

GEOMETRIES = [  # hidden, intermediate, activation name
    (7168, 2048, "silu"),   # config 2: S = 4, NB = 7
    (4096, 2048, "silu"),   # S = 2, NB = 4
    (2048, 2048, "situ"),   # S = 1, NB = 2
    (8192, 2048, "silu"),   # S = 4, NB = 8
]


def say(msg):
    print(f"[gpu-case] {msg}", flush=True)


def _geo(hidden, inter, act):
    from deltafin_amd import _lib
    return _lib.geometry(hidden, inter, _lib.K3_ACT_SILU if act == "silu" else _lib.K3_ACT_SITU)


def _bank(g, seed):
    import torch
    from deltafin_amd import moe
    stride = g.expert_span
    bank = torch.empty(N_BANK * stride, dtype=torch.uint8, device="cuda")
    moe.synth_bank(g, bank, stride, N_BANK, 0, seed)
    return bank, stride


def _bf16_dev(x32):
    import torch
    return torch.from_numpy(synth.to_bf16_bits(x32).view(np.int16)).view(torch.bfloat16).cuda()


def _routed(g, bank, stride, logits, k, x, ws, odt, fused, out=None):
    """One router-mode layer call on the selected path; returns the outputs and
    the kernel classes that ran."""
    from deltafin_amd import _lib, moe
    prev = _lib.set_fused_decode(fused)
    try:
        _lib.timing_begin(64)
        res = moe.moe_route_layer(g, bank, stride, N_BANK, logits, k, x, ws, out_dtype=odt,
                                  out=out)
        kern, dropped = _lib.timing_end()
    finally:
        _lib.set_fused_decode(prev)
    assert dropped == 0
    return res, kern


def _same(a, b):
    import torch
    return torch.equal(a.view(torch.int16) if a.dtype == torch.bfloat16 else a.view(torch.int32),
                       b.view(torch.int16) if b.dtype == torch.bfloat16 else b.view(torch.int32))


@pytest.mark.parametrize("hidden,inter,act", GEOMETRIES)
def test_fused_matches_two_launch_and_oracle(gpu, hidden, inter, act):
    import torch
    from deltafin_amd import moe
    g = _geo(hidden, inter, act)
    say(f"fused vs two-launch vs oracle: hidden {hidden} inter {inter} {act}")
    bank, stride = _bank(g, 4321 + hidden)
    ws = moe.workspace(g, 16)
    rng = np.random.default_rng(hidden)
    for k, odt in [(16, torch.float32), (16, torch.bfloat16), (7, torch.float32),
                   (1, torch.bfloat16)]:
        logits = torch.from_numpy(rng.standard_normal(N_BANK).astype(np.float32)).cuda()
        x32 = synth.bf16_bits_to_f32(synth.to_bf16_bits(
            rng.standard_normal(g.hidden).astype(np.float32)))
        x = _bf16_dev(x32)
        (of, idf, wf), kf = _routed(g, bank, stride, logits, k, x, ws, odt, True)
        (os_, ids_, ws_), ks = _routed(g, bank, stride, logits, k, x, ws, odt, False)
        torch.cuda.synchronize()
        assert kf.get("decode_fused", {}).get("launches") == 1, kf
        assert "glu_decode" not in kf and "down_decode" not in kf, kf
        assert ks["glu_decode"]["launches"] == 1 and ks["down_decode"]["launches"] == 1, ks
        assert _same(of, os_), f"k={k} {odt}: fused and two-launch outputs differ"
        assert torch.equal(idf, ids_) and torch.equal(wf, ws_)
        if k == 16 and odt == torch.float32:
            rid, rw = oracle.topk_softmax(logits.cpu().numpy(), k)
            assert idf.cpu().numpy().tolist() == rid.tolist()
            spans = [oracle.synth_expert(4321 + hidden, int(e), g.hidden, g.intermediate)
                     for e in rid]
            ref, mag = oracle.moe_layer_f64(spans, rw, g.hidden, g.intermediate, g.activation,
                                            x32)
            err = oracle.cond_rel_err(of.cpu().numpy(), ref, mag, g.intermediate)
            assert err <= TOL, f"cond rel err {err:.3e}"


def test_fused_pointer_mode_matches_two_launch(gpu):
    """Caller-routed layer (explicit span pointers and weights)."""
    import torch
    from deltafin_amd import _lib, moe
    g = moe.preset(2)
    say("fused pointer mode vs two-launch")
    bank, stride = _bank(g, 99)
    ws = moe.workspace(g, 16)
    rng = np.random.default_rng(5)
    for n in (16, 12, 2):
        ids = rng.choice(N_BANK, size=n, replace=False)
        w = rng.random(n).astype(np.float32)
        spans = [bank.data_ptr() + int(e) * stride for e in ids]
        x = _bf16_dev(rng.standard_normal(g.hidden).astype(np.float32))
        outs = []
        for fused in (True, False):
            prev = _lib.set_fused_decode(fused)
            try:
                outs.append(moe.moe_layer(g, spans, w.tolist(), x, ws, out_dtype=torch.float32))
            finally:
                _lib.set_fused_decode(prev)
        torch.cuda.synchronize()
        assert _same(outs[0], outs[1]), f"n={n}"


def test_fused_back_to_back_resets(gpu):
    """40 launches queued on one workspace without a host sync: a counter left
    non-zero by one launch would make the next one skip work or read h early."""
    import torch
    from deltafin_amd import _lib, moe
    g = moe.preset(2)
    T = 40
    say(f"fused back to back: {T} tokens on one workspace")
    bank, stride = _bank(g, 7)
    ws = moe.workspace(g, 16)
    rng = np.random.default_rng(11)
    logits = torch.from_numpy(rng.standard_normal((T, N_BANK)).astype(np.float32)).cuda()
    x = _bf16_dev(rng.standard_normal((T, g.hidden)).astype(np.float32)).view(T, g.hidden)
    outs = {}
    for fused in (True, False):
        o = torch.full((T, g.hidden), float("nan"), dtype=torch.bfloat16, device="cuda")
        prev = _lib.set_fused_decode(fused)
        try:
            _lib.timing_begin(4 * T)
            for t in range(T):
                moe.moe_route_layer(g, bank, stride, N_BANK, logits[t], 16, x[t], ws,
                                    out=o[t], want_route=False)
            kern, _ = _lib.timing_end()
        finally:
            _lib.set_fused_decode(prev)
        if fused:
            assert kern["decode_fused"]["launches"] == T, kern
        outs[fused] = o
    torch.cuda.synchronize()
    assert not torch.isnan(outs[True].float()).any()
    for t in range(T):
        assert _same(outs[True][t], outs[False][t]), f"token {t}"


def test_fused_two_streams(gpu):
    """Two workspaces on two streams, 16 tokens each, queued together so fused
    kernels of both streams can be resident at once."""
    import torch
    from deltafin_amd import _lib, moe
    g = moe.preset(2)
    T = 16
    say(f"fused on two streams: 2 x {T} tokens")
    bank, stride = _bank(g, 3)
    rng = np.random.default_rng(13)
    logits = torch.from_numpy(rng.standard_normal((2, T, N_BANK)).astype(np.float32)).cuda()
    x = _bf16_dev(rng.standard_normal((2, T, g.hidden)).astype(np.float32)).view(2, T, g.hidden)
    wss = [moe.workspace(g, 16) for _ in range(2)]
    outs = torch.full((2, T, g.hidden), float("nan"), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream() for _ in range(2)]
    prev = _lib.set_fused_decode(True)
    try:
        for t in range(T):
            for s in range(2):
                with torch.cuda.stream(streams[s]):
                    moe.moe_route_layer(g, bank, stride, N_BANK, logits[s, t], 16, x[s, t],
                                        wss[s], out=outs[s, t], want_route=False)
        torch.cuda.synchronize()
    finally:
        _lib.set_fused_decode(prev)
    ws1 = moe.workspace(g, 16)
    for s in range(2):
        for t in range(T):
            ref, _, _ = moe.moe_route_layer(g, bank, stride, N_BANK, logits[s, t], 16, x[s, t],
                                            ws1, want_route=False)
            torch.cuda.synchronize()
            assert _same(outs[s, t], ref), f"stream {s} token {t}"


def test_fp32_activations_take_two_launch_path(gpu):
    import torch
    from deltafin_amd import moe
    g = moe.preset(2)
    say("fp32 x runs the two-launch path")
    bank, stride = _bank(g, 17)
    ws = moe.workspace(g, 16)
    rng = np.random.default_rng(17)
    logits = torch.from_numpy(rng.standard_normal(N_BANK).astype(np.float32)).cuda()
    x = torch.from_numpy(rng.standard_normal(g.hidden).astype(np.float32)).cuda()
    _, kern = _routed(g, bank, stride, logits, 16, x, ws, torch.float32, True)
    assert "decode_fused" not in kern and kern["glu_decode"]["launches"] == 1, kern
