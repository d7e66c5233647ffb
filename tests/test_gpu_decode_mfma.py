"""The matrix-core gate/up kernel of the single-token layer (k_glu_mfma,
selected by k3_hip_set_decode_mfma) against the fp64 oracle and against the
vector-ALU kernel on the same inputs.

The kernel folds each chunk's E8M0 scale into the fp4 -> bf16 convert and
multiplies bf16 activation terms on the matrix cores (fp32 x as three terms
that sum to it exactly), so its outputs equal the vector kernel's up to the
summation order: both must meet the oracle bar (TOL), and they must agree
with each other within SAME (a few fp32 roundings of the terms' size).
Cases: K3 and the benchmark geometry, caller routes with 16 and 10 experts
(6, 8 and 4 units per unit pipeline), fp32 and bf16 activations, the device
router (ids and weights bit-identical between the two kernels), and the scale
bytes the reference treats specially: 0 is +0.0 (a whole bank of zero scale
bytes gives an exactly zero output), 255 poisons the row with NaN, and bytes
far from 127 scale exactly (tools/fused_gemv.c:247-249,
tools/cuda_moe_kernels.cu:128-131).
"""
import numpy as np
import pytest

import oracle
from deltafin_amd import synth

pytestmark = pytest.mark.gpu

TOL = 1e-3
SAME = 1e-5


def say(msg):
    print(f"[gpu-case] {msg}", flush=True)


def _layer(g, spans, w, x32, xdt, mode):
    import torch
    from deltafin_amd import _lib, moe
    dx = (torch.from_numpy(synth.to_bf16_bits(x32).view(np.int16)).view(torch.bfloat16).cuda()
          if xdt == "bf16" else torch.from_numpy(x32).cuda())
    ds = [torch.from_numpy(sp).cuda() for sp in spans]
    ws = moe.workspace(g, len(spans))
    prev = _lib.set_decode_mfma(mode)
    try:
        out = moe.moe_layer(g, ds, w, dx, ws)
        torch.cuda.synchronize()
    finally:
        _lib.set_decode_mfma(prev)
    return out.cpu().numpy()


@pytest.mark.parametrize("preset_id,n,xdt", [(1, 16, "f32"), (1, 10, "f32"), (2, 16, "f32"),
                                             (2, 16, "bf16"), (1, 16, "bf16")],
                         ids=["k3_16_f32", "k3_10_f32", "bench_16_f32", "bench_16_bf16",
                              "k3_16_bf16"])
def test_mfma_gate_up_caller_routes(gpu, preset_id, n, xdt):
    from deltafin_amd import _lib, moe
    g = moe.preset(preset_id)
    say(f"decode mfma: preset {preset_id}, {n} experts, x {xdt}")
    spans = [oracle.synth_expert(515, e, g.hidden, g.intermediate) for e in range(n)]
    rng = np.random.default_rng(516)
    w = rng.random(n).astype(np.float32)
    w /= w.sum()
    x = rng.standard_normal(g.hidden).astype(np.float32)
    if xdt == "bf16":
        x = synth.bf16_bits_to_f32(synth.to_bf16_bits(x))
    mode = _lib.DECODE_DOTS_MFMA_F32 if xdt == "f32" else _lib.DECODE_DOTS_MFMA_ALL
    got = _layer(g, spans, w, x, xdt, mode)
    valu = _layer(g, spans, w, x, xdt, _lib.DECODE_DOTS_VALU)
    again = _layer(g, spans, w, x, xdt, mode)
    assert np.array_equal(got.view(np.uint32), again.view(np.uint32)), "reruns differ"
    ref, mag = oracle.moe_layer_f64(spans, w.astype(np.float64), g.hidden, g.intermediate,
                                    g.activation, x)
    err = oracle.cond_rel_err(got, ref, mag, g.intermediate)
    assert err <= TOL, f"matrix-core path vs oracle: {err:.3e}"
    assert oracle.cond_rel_err(valu, ref, mag, g.intermediate) <= TOL
    d = oracle.cond_rel_err(got, valu.astype(np.float64), mag, g.intermediate)
    say(f"decode mfma: oracle {err:.2e}, vs vector kernel {d:.2e}")
    assert d <= SAME, f"matrix-core vs vector kernel: {d:.3e}"


def test_mfma_gate_up_router_mode(gpu):
    """Device router + layer (bf16 x, benchmark geometry, 48-expert bank):
    both kernels publish the same ids and bit-identical weights."""
    import torch
    from deltafin_amd import _lib, moe
    g = moe.preset(2)
    n_bank, k = 48, 16
    say("decode mfma: router mode, 48-expert bank, top 16")
    stride = g.expert_span
    bank = torch.empty(n_bank * stride, dtype=torch.uint8, device="cuda")
    moe.synth_bank(g, bank, stride, n_bank, 0, 77)
    ws = moe.workspace(g, k)
    rng = np.random.default_rng(78)
    logits = rng.standard_normal(n_bank).astype(np.float32)
    x = synth.bf16_bits_to_f32(synth.to_bf16_bits(rng.standard_normal(g.hidden).astype(np.float32)))
    dx = torch.from_numpy(synth.to_bf16_bits(x).view(np.int16)).view(torch.bfloat16).cuda()
    res = {}
    for mode in (_lib.DECODE_DOTS_MFMA_ALL, _lib.DECODE_DOTS_VALU):
        prev = _lib.set_decode_mfma(mode)
        try:
            out, ids, wts = moe.moe_route_layer(g, bank, stride, n_bank,
                                                torch.from_numpy(logits).cuda(), k, dx, ws)
            torch.cuda.synchronize()
        finally:
            _lib.set_decode_mfma(prev)
        res[mode] = (out.cpu().numpy(), ids.cpu().numpy(), wts.cpu().numpy())
    mo, mi, mw = res[_lib.DECODE_DOTS_MFMA_ALL]
    vo, vi, vw = res[_lib.DECODE_DOTS_VALU]
    assert np.array_equal(mi, vi) and np.array_equal(mw.view(np.uint32), vw.view(np.uint32))
    rid, rw = oracle.topk_softmax(logits, k)
    assert mi.tolist() == rid.tolist()
    spans = [oracle.synth_expert(77, int(e), g.hidden, g.intermediate) for e in rid]
    ref, mag = oracle.moe_layer_f64(spans, rw, g.hidden, g.intermediate, g.activation, x)
    assert oracle.cond_rel_err(mo, ref, mag, g.intermediate) <= TOL
    assert oracle.cond_rel_err(mo, vo.astype(np.float64), mag, g.intermediate) <= SAME


def _scales_view(span, g, which):
    """The gate (w1) or up (w3) scale plane of a raw-v1 span as [rows, groups]."""
    off = oracle.expert_offsets(g.hidden, g.intermediate)
    base = off[1] if which == "gate" else off[5]
    G = g.hidden // 32
    return span[base:base + g.intermediate * G].reshape(g.intermediate, G)


def test_mfma_scale_bytes(gpu):
    """Scale bytes 0, 255 and far from 127 through the matrix-core kernel (K3,
    16 experts, fp32 x)."""
    from deltafin_amd import _lib, moe
    g = moe.preset(1)
    n = 16
    say("decode mfma: scale bytes 0 / 255 / extreme")
    rng = np.random.default_rng(919)
    w = rng.random(n).astype(np.float32)
    w /= w.sum()
    x = rng.standard_normal(g.hidden).astype(np.float32)
    mode = _lib.DECODE_DOTS_MFMA_F32
    # Far from 127 (exact powers of two in both kernels): some chunks of every
    # expert at 2^-27 and 2^23.
    spans = [oracle.synth_expert(920, e, g.hidden, g.intermediate).copy() for e in range(n)]
    for e, sp in enumerate(spans):
        for which in ("gate", "up"):
            sv = _scales_view(sp, g, which)
            sv[(e * 37) % g.intermediate, ::7] = 100
            sv[(e * 53 + 11) % g.intermediate, 3::9] = 150
            sv[(e * 29 + 5) % g.intermediate, :] = 0   # a whole row reads +0.0
    got = _layer(g, spans, w, x, "f32", mode)
    ref, mag = oracle.moe_layer_f64(spans, w.astype(np.float64), g.hidden, g.intermediate,
                                    g.activation, x)
    assert np.all(np.isfinite(got))
    assert oracle.cond_rel_err(got, ref, mag, g.intermediate) <= TOL
    # Every scale byte 0: every gate and up row is +0.0, so is the output.
    zero = [sp.copy() for sp in spans]
    for sp in zero:
        _scales_view(sp, g, "gate")[:] = 0
        _scales_view(sp, g, "up")[:] = 0
    z = _layer(g, zero, w, x, "f32", mode)
    assert np.all(z == 0.0), "scale byte 0 must contribute exactly +0.0"
    # One 255 byte in one gate row of one expert: NaN reaches every output (the
    # down projection sums over that h element), as in the oracle.
    poison = [sp.copy() for sp in spans]
    _scales_view(poison[3], g, "gate")[17, 5] = 255
    p = _layer(g, poison, w, x, "f32", mode)
    pref, _ = oracle.moe_layer_f64(poison, w.astype(np.float64), g.hidden, g.intermediate,
                                   g.activation, x)
    assert np.all(np.isnan(pref)) and np.all(np.isnan(p))


def test_decode_mfma_mode_switch(gpu):
    """The setting is process-wide, returns the previous value and rejects
    unknown modes."""
    from deltafin_amd import _lib
    lib = _lib.load()
    prev = lib.k3_hip_set_decode_mfma(_lib.DECODE_DOTS_VALU)
    assert prev in (0, 1, 2)
    assert lib.k3_hip_set_decode_mfma(_lib.DECODE_DOTS_MFMA_ALL) == _lib.DECODE_DOTS_VALU
    assert lib.k3_hip_set_decode_mfma(7) == _lib.K3_HIP_E_INVALID
    assert lib.k3_hip_set_decode_mfma(prev) == _lib.DECODE_DOTS_MFMA_ALL
