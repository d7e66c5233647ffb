"""GPU tests of the one-launch path for one-expert layers (k_expert_chain),
on by default (k3_hip_set_decode_chain).

A single-token layer call with one routed expert given as a span pointer
(bf16 x, raw-v1, intermediate 2048) runs the gate/up sweep and the down rows
in one launch: workgroups hand h over through device memory as tagged 64-bit
entries instead of a second launch.  Its arithmetic is that of the two
launches (k_glu_decode's 2-row units + k_down_few), so every output here must
be bit-identical to the two-launch output on the same inputs, and both must
match the fp64 oracle (oracle.expert_f64, the restatement of
tools/fused_gemv_batch.c:465-518) within the parity tolerance.

Geometries cover each column split the path takes (S = 2, 3, 4 waves; one
and two units per pipeline).  The fallback mode makes every workgroup compute
the gate/up shares it finds missing at once (the path a workgroup takes when
not every workgroup is resident); back-to-back calls check that the per
workgroup call counts advance the tag; two streams queue two launches at once
(not every workgroup of both can be resident); a captured graph replays the
launch with the same arguments.
"""
import numpy as np
import pytest

import oracle
from deltafin_amd import synth

pytestmark = pytest.mark.gpu

TOL = 1e-3
N_EXPERTS = 6

GEOMETRIES = [  # hidden, activation
    (7168, "silu"),   # config 1: S = 4, two units per pipeline
    (8192, "silu"),   # S = 4
    (6144, "situ"),   # S = 3, 384 threads
    (4096, "silu"),   # S = 2, one unit per pipeline
]


def say(msg):
    print(f"[gpu-case] {msg}", flush=True)


def _geo(hidden, act):
    from deltafin_amd import _lib
    return _lib.geometry(hidden, 2048, _lib.K3_ACT_SILU if act == "silu" else _lib.K3_ACT_SITU)


def _chain_expected(hidden, cus):
    """Whether the host takes the one-launch path for this hidden size
    (mirrors chain_decode's shape checks for one expert)."""
    G = hidden // 32
    S = (G + 63) // 64
    groups = max(1, min(512 // (64 * S), 16 // S))
    if (512 + groups - 1) // groups > cus:
        return False
    grid = min(cus, (1024 + groups - 1) // groups)
    threads = 64 * S * groups
    iters = (1024 + grid * groups - 1) // (grid * groups)
    return grid == cus and threads >= 384 and grid * threads // 64 >= (hidden + 3) // 4 \
        and iters in (1, 2)


def _bank(g, seed):
    import torch
    from deltafin_amd import moe
    stride = g.expert_span
    bank = torch.empty(N_EXPERTS * stride, dtype=torch.uint8, device="cuda")
    moe.synth_bank(g, bank, stride, N_EXPERTS, 0, seed)
    return bank, stride


def _bf16_dev(x32):
    import torch
    return torch.from_numpy(synth.to_bf16_bits(x32).view(np.int16)).view(torch.bfloat16).cuda()


def _call(g, span, x, ws, odt, mode, out=None):
    """One one-expert layer call in chain mode `mode`; returns the output and
    the kernel classes that ran."""
    from deltafin_amd import _lib, moe
    prev = _lib.set_decode_chain(mode)
    try:
        _lib.timing_begin(16)
        y = moe.moe_layer(g, [span], [1.0], x, ws, out_dtype=odt, out=out)
        kern, dropped = _lib.timing_end()
    finally:
        _lib.set_decode_chain(prev)
    assert dropped == 0
    return y, kern


def _same(a, b):
    import torch
    return torch.equal(a.view(torch.int16) if a.dtype == torch.bfloat16 else a.view(torch.int32),
                       b.view(torch.int16) if b.dtype == torch.bfloat16 else b.view(torch.int32))


@pytest.mark.parametrize("hidden,act", GEOMETRIES)
def test_chain_matches_two_launch_and_oracle(gpu, hidden, act):
    import torch
    from deltafin_amd import _lib, moe
    g = _geo(hidden, act)
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    expect = _chain_expected(hidden, cus)
    say(f"chain vs two-launch vs oracle: hidden {hidden} {act} (chain expected: {expect})")
    bank, stride = _bank(g, 900 + hidden)
    ws = moe.workspace(g, 1)
    rng = np.random.default_rng(hidden)
    for e, odt in [(0, torch.float32), (3, torch.bfloat16), (5, torch.float32)]:
        span = bank.data_ptr() + e * stride
        x32 = synth.bf16_bits_to_f32(synth.to_bf16_bits(
            rng.standard_normal(g.hidden).astype(np.float32)))
        x = _bf16_dev(x32)
        y2, k2 = _call(g, span, x, ws, odt, _lib.DECODE_CHAIN_OFF)
        y1, k1 = _call(g, span, x, ws, odt, _lib.DECODE_CHAIN_ON)
        yf, kf = _call(g, span, x, ws, odt, _lib.DECODE_CHAIN_FALLBACK)
        torch.cuda.synchronize()
        assert k2["glu_decode"]["launches"] == 1 and k2["down_decode"]["launches"] == 1, k2
        if expect:
            assert k1.get("decode_chain", {}).get("launches") == 1, k1
            assert "glu_decode" not in k1 and "down_decode" not in k1, k1
            assert kf.get("decode_chain", {}).get("launches") == 1, kf
        assert _same(y1, y2), f"expert {e} {odt}: one launch and two launches differ"
        assert _same(yf, y2), f"expert {e} {odt}: fallback and two launches differ"
        if odt == torch.float32:
            sp = bank[e * stride: e * stride + g.expert_span].cpu().numpy()
            ref, _, mag = oracle.expert_f64(sp, g.hidden, g.intermediate, g.activation, x32)
            err = oracle.cond_rel_err(y1.cpu().numpy(), ref, mag, g.intermediate)
            assert err <= TOL, f"cond rel err {err:.3e}"


def test_chain_special_scales(gpu):
    """Scale bytes the reference treats specially, in both phases: a gate
    row with scale byte 255 (NaN: its h, and so every output, is NaN), a group
    of an up row with scale byte 0 (the group contributes +0.0), a down row
    with 255 (that output NaN) and a group of another with 0.  One launch and
    two launches agree bit for bit, NaN payloads included."""
    import torch
    from deltafin_amd import _lib, moe
    g = _geo(7168, "silu")
    say("chain special scale bytes")
    bank, stride = _bank(g, 91)
    off = moe.span_offsets(g)
    G, GI = g.hidden // 32, g.intermediate // 32
    ws = moe.workspace(g, 1)
    rng = np.random.default_rng(91)
    x = _bf16_dev(rng.standard_normal(g.hidden).astype(np.float32))
    cases = [
        ("up row 5 scale 0, down rows 17 / 4000 scales 255 / 0",
         [(off["w3s"] + 5 * G + 3, 0), (off["w2s"] + 17 * GI + 9, 255), (off["w2s"] + 4000 * GI, 0)]),
        ("gate row 1000 scale 255", [(off["w1s"] + 1000 * G + 100, 255)]),
    ]
    for name, edits in cases:
        span = bank[:stride].clone()
        for o, v in edits:
            span[o] = v
        y2, k2 = _call(g, span.data_ptr(), x, ws, torch.float32, _lib.DECODE_CHAIN_OFF)
        y1, k1 = _call(g, span.data_ptr(), x, ws, torch.float32, _lib.DECODE_CHAIN_ON)
        torch.cuda.synchronize()
        assert "decode_chain" in k1 and "glu_decode" in k2, (k1, k2)
        assert _same(y1, y2), name
        yh = y1.cpu().numpy()
        if "gate row" in name:
            assert np.isnan(yh).all(), name
        else:
            assert np.isnan(yh[17]) and np.isfinite(np.delete(yh, 17)).all(), name


def test_chain_back_to_back(gpu):
    """40 calls queued on one workspace without a host sync, experts and
    activations changing: each call's tag must differ from the last, or a
    reader would take the previous call's h."""
    import torch
    from deltafin_amd import _lib, moe
    g = _geo(7168, "silu")
    T = 40
    say(f"chain back to back: {T} calls on one workspace")
    bank, stride = _bank(g, 77)
    ws = moe.workspace(g, 1)
    rng = np.random.default_rng(77)
    x = _bf16_dev(rng.standard_normal((T, g.hidden)).astype(np.float32)).view(T, g.hidden)
    outs = {}
    for mode in (_lib.DECODE_CHAIN_ON, _lib.DECODE_CHAIN_OFF):
        o = torch.full((T, g.hidden), float("nan"), dtype=torch.float32, device="cuda")
        prev = _lib.set_decode_chain(mode)
        try:
            for t in range(T):
                moe.moe_layer(g, [bank.data_ptr() + (t % N_EXPERTS) * stride], [1.0], x[t], ws,
                              out=o[t])
        finally:
            _lib.set_decode_chain(prev)
        outs[mode] = o
    torch.cuda.synchronize()
    assert not torch.isnan(outs[_lib.DECODE_CHAIN_ON]).any()
    for t in range(T):
        assert _same(outs[_lib.DECODE_CHAIN_ON][t], outs[_lib.DECODE_CHAIN_OFF][t]), f"call {t}"


def test_chain_two_streams(gpu):
    """Two workspaces on two streams, 16 calls each, queued together: the two
    launches cannot both have every workgroup resident, so a workgroup may
    have to compute missing gate/up shares itself."""
    import torch
    from deltafin_amd import _lib, moe
    g = _geo(7168, "silu")
    T = 16
    say(f"chain on two streams: 2 x {T} calls")
    bank, stride = _bank(g, 55)
    rng = np.random.default_rng(55)
    x = _bf16_dev(rng.standard_normal((2, T, g.hidden)).astype(np.float32)).view(2, T, g.hidden)
    wss = [moe.workspace(g, 1) for _ in range(2)]
    outs = torch.full((2, T, g.hidden), float("nan"), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream() for _ in range(2)]
    prev = _lib.set_decode_chain(_lib.DECODE_CHAIN_ON)
    try:
        for t in range(T):
            for s in range(2):
                with torch.cuda.stream(streams[s]):
                    moe.moe_layer(g, [bank.data_ptr() + ((t + s) % N_EXPERTS) * stride], [1.0],
                                  x[s, t], wss[s], out=outs[s, t])
        torch.cuda.synchronize()
    finally:
        _lib.set_decode_chain(prev)
    ws1 = moe.workspace(g, 1)
    prev = _lib.set_decode_chain(_lib.DECODE_CHAIN_OFF)
    try:
        for s in range(2):
            for t in range(T):
                ref = moe.moe_layer(g, [bank.data_ptr() + ((t + s) % N_EXPERTS) * stride], [1.0],
                                    x[s, t], ws1)
                torch.cuda.synchronize()
                assert _same(outs[s, t], ref), f"stream {s} call {t}"
    finally:
        _lib.set_decode_chain(prev)


def test_chain_graph_replay(gpu):
    """The launch captured once and replayed with new activations copied into
    its input between replays: the tag comes from device-side call counts, so
    each replay waits for its own h.  Every replay is checked against an
    eager two-launch call."""
    import torch
    from deltafin_amd import _lib, moe
    g = _geo(7168, "silu")
    say("chain graph replay")
    bank, stride = _bank(g, 33)
    span = bank.data_ptr() + 2 * stride
    ws = moe.workspace(g, 1)
    rng = np.random.default_rng(33)
    xs = _bf16_dev(rng.standard_normal((6, g.hidden)).astype(np.float32)).view(6, g.hidden)
    x_in = xs[0].clone()
    y_out = torch.empty(g.hidden, dtype=torch.float32, device="cuda")
    prev = _lib.set_decode_chain(_lib.DECODE_CHAIN_ON)
    try:
        moe.moe_layer(g, [span], [1.0], x_in, ws, out=y_out)  # warm the path outside capture
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            moe.moe_layer(g, [span], [1.0], x_in, ws, out=y_out)
        torch.cuda.synchronize()
        ws2 = moe.workspace(g, 1)
        for r in range(6):
            x_in.copy_(xs[r])
            y_out.fill_(float("nan"))
            graph.replay()
            torch.cuda.synchronize()
            _lib.set_decode_chain(_lib.DECODE_CHAIN_OFF)
            ref = moe.moe_layer(g, [span], [1.0], xs[r], ws2)
            torch.cuda.synchronize()
            _lib.set_decode_chain(_lib.DECODE_CHAIN_ON)
            assert _same(y_out, ref), f"replay {r}"
    finally:
        _lib.set_decode_chain(prev)


def test_chain_mode_values(gpu):
    from deltafin_amd import _lib
    say("chain mode values")
    prev = _lib.set_decode_chain(_lib.DECODE_CHAIN_OFF)
    try:
        assert prev == _lib.DECODE_CHAIN_ON
        assert _lib.set_decode_chain(_lib.DECODE_CHAIN_FALLBACK) == _lib.DECODE_CHAIN_OFF
        with pytest.raises(_lib.K3HipError):
            _lib.set_decode_chain(3)
    finally:
        _lib.set_decode_chain(prev)
