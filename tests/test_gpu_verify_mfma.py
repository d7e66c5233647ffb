"""GPU parity of the matrix-core verify path (block-scaled FP4 MFMA).

Every routed expert is read once per verify batch and multiplied for all of
its positions on v_mfma_scale_f32_16x16x128_f8f6f4: weights as stored (E2M1 +
E8M0), activations as fp8 terms with per-32 scales.  Each case checks the
outputs against the fp64 oracle (max relative error <= 1e-3 per output,
oracle.cond_rel_err) and the routes against the oracle's top-k (IDs
identical), for the verify paths the library can run (K3_VERIFY_* modes).
"""
import numpy as np
import pytest

import oracle
from deltafin_amd import _lib, synth

pytestmark = pytest.mark.gpu

TOL = 1e-3
MODES = {"mfma": _lib.VERIFY_UNION_MFMA, "positions": _lib.VERIFY_POSITIONS,
         "valu": _lib.VERIFY_UNION_VALU}


def say(msg):
    print(f"[gpu-case] {msg}", flush=True)


def _t(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _bf16(x32):
    import torch
    return torch.from_numpy(synth.to_bf16_bits(x32).view(np.int16)).view(torch.bfloat16).cuda()


def _bf16_round(x32):
    return synth.bf16_bits_to_f32(synth.to_bf16_bits(x32)).reshape(x32.shape)


@pytest.fixture
def verify_mode(gpu):
    """Set the process-wide verify path for one test and restore AUTO after."""
    modes = []

    def set_mode(mode):
        modes.append(_lib.set_verify_mode(mode))

    yield set_mode
    _lib.set_verify_mode(_lib.VERIFY_AUTO)


_ROUTE_REFS = {}
_BANK_EXPERTS = {}


def _bank_expert(e, g):
    if e not in _BANK_EXPERTS:
        _BANK_EXPERTS[e] = oracle.synth_expert(901, e, g.hidden, g.intermediate)
    return _BANK_EXPERTS[e]


@pytest.mark.parametrize("m", [1, 2, 4, 16])
@pytest.mark.parametrize("mode", ["mfma", "positions", "valu"])
def test_verify_route_modes(gpu, verify_mode, m, mode):
    """Device-routed verify over a 48-expert bank: with M = 16 positions each
    routing 16 of 48 experts, most experts carry many positions (the small-M
    contraction the matrix cores serve)."""
    import torch
    from deltafin_amd import moe
    g = moe.preset(2)
    n_bank, k = 48, 16
    say(f"verify route mode={mode} M={m} bank={n_bank}")
    verify_mode(MODES[mode])
    stride = g.expert_span
    bank = torch.empty(n_bank * stride, dtype=torch.uint8, device="cuda")
    moe.synth_bank(g, bank, stride, n_bank, 0, 901)
    rng = np.random.default_rng(300 + m)
    logits = rng.standard_normal((m, n_bank)).astype(np.float32)
    x = _bf16_round(rng.standard_normal((m, g.hidden)).astype(np.float32))
    ws = moe.workspace(g, m * k, m)
    out, ids, wts = moe.moe_verify_route(g, bank, stride, n_bank, _t(logits), k,
                                         _bf16(x).reshape(m, g.hidden), ws)
    torch.cuda.synchronize()
    out, ids, wts = out.cpu().numpy(), ids.cpu().numpy(), wts.cpu().numpy()
    for p in range(m):
        rid, rw = oracle.topk_softmax(logits[p], k)
        assert ids[p].tolist() == rid.tolist(), f"position {p} route"
        assert np.allclose(wts[p], rw, rtol=1e-6, atol=1e-7)
        key = (m, p)
        if key not in _ROUTE_REFS:  # the three paths share positions: one oracle run each
            spans = [_bank_expert(int(e), g) for e in rid]
            _ROUTE_REFS[key] = oracle.moe_layer_f64(spans, rw, g.hidden, g.intermediate,
                                                    g.activation, x[p])
        ref, mag = _ROUTE_REFS[key]
        err = oracle.cond_rel_err(out[p], ref, mag, g.intermediate)
        assert err <= TOL, f"position {p}: {err:.3e}"


def _shared_table(n_experts, n_positions, per_position, seed):
    """Routes where positions draw their experts from a small shared set."""
    rng = np.random.default_rng(seed)
    routes = [rng.permutation(n_experts)[:per_position].tolist() for _ in range(n_positions)]
    weights = [rng.random(len(r)).astype(np.float32) for r in routes]
    weights = [w / w.sum() for w in weights]
    return routes, weights


@pytest.mark.parametrize("preset_id,xdt", [(2, "bf16"), (2, "f32"), (1, "f32"), (1, "bf16")])
def test_verify_mfma_shared_table(gpu, verify_mode, preset_id, xdt):
    """Caller-routed verify where 16 positions share 16 experts (every expert
    carries up to 16 token columns): preset 2 (SiLU) and preset 1 (K3 SiTU),
    bf16 x (two fp8 terms) and fp32 x (three)."""
    import torch
    from deltafin_amd import moe
    g = moe.preset(preset_id)
    say(f"verify mfma shared table preset={preset_id} x={xdt}")
    verify_mode(_lib.VERIFY_UNION_MFMA)
    n_exp, m = 16, 16
    spans = [oracle.synth_expert(31, e, g.hidden, g.intermediate) for e in range(n_exp)]
    d = [_t(sp) for sp in spans]
    routes, weights = _shared_table(n_exp, m, 12, 7 + preset_id)
    rng = np.random.default_rng(11)
    x = rng.standard_normal((m, g.hidden)).astype(np.float32)
    if xdt == "bf16":
        x = _bf16_round(x)
        xd = _bf16(x).reshape(m, g.hidden)
    else:
        xd = _t(x)
    edges, wts, offs = [], [], [0]
    for r, w in zip(routes, weights):
        edges += [d[e] for e in r]
        wts += w.tolist()
        offs.append(len(edges))
    ws = moe.workspace(g, len(edges), m)
    out = moe.moe_verify(g, edges, wts, offs, xd, ws)
    torch.cuda.synchronize()
    out = out.cpu().numpy()
    for p, (r, w) in enumerate(zip(routes, weights)):
        ref, mag = oracle.moe_layer_f64([spans[e] for e in r], w.astype(np.float64), g.hidden,
                                        g.intermediate, g.activation, x[p])
        err = oracle.cond_rel_err(out[p], ref, mag, g.intermediate)
        assert err <= TOL, f"position {p}: {err:.3e}"


@pytest.mark.parametrize("n_bank,m", [(48, 16), (384, 16), (48, 3)])
@pytest.mark.parametrize("mode", ["mfma", "valu"])
def test_verify_bank_plan_matches_table(gpu, verify_mode, n_bank, m, mode):
    """The device-routed verify groups its edges by expert id (counts and
    position masks over the bank's experts); the caller-table verify groups
    the same edges by comparing span pointers.  On the same routes the two
    calls give the same outputs, bit for bit, on both union paths; with 16
    positions over 48 experts most experts carry several positions."""
    import torch
    from deltafin_amd import moe
    g = moe.preset(2)
    k = 16
    say(f"verify bank plan vs table mode={mode} M={m} bank={n_bank}")
    verify_mode(MODES[mode])
    stride = g.expert_span
    bank = torch.empty(n_bank * stride, dtype=torch.uint8, device="cuda")
    moe.synth_bank(g, bank, stride, n_bank, 0, 905)
    rng = np.random.default_rng(40 + m + n_bank)
    logits = rng.standard_normal((m, n_bank)).astype(np.float32)
    x = _bf16(rng.standard_normal((m, g.hidden)).astype(np.float32)).reshape(m, g.hidden)
    ws = moe.workspace(g, m * k, m)
    out_r, ids, wts = moe.moe_verify_route(g, bank, stride, n_bank, _t(logits), k, x, ws)
    torch.cuda.synchronize()
    ids_h, wts_h = ids.cpu().numpy().reshape(-1), wts.cpu().numpy().reshape(-1)
    assert len(set(ids_h.tolist())) < m * k or m < 16
    edges = [bank.data_ptr() + int(e) * stride for e in ids_h]
    out_t = moe.moe_verify(g, edges, wts_h.tolist(), [p * k for p in range(m + 1)], x, ws)
    torch.cuda.synchronize()
    a, b = out_r.cpu().numpy(), out_t.cpu().numpy()
    assert np.all(np.isfinite(a))
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_verify_mfma_bf16_out_empty_position(gpu, verify_mode):
    """bf16 outputs within one bf16 ulp of the oracle plus the fp32 band; an
    empty position gives a zero row; one expert repeated inside a position."""
    import math
    import torch
    from deltafin_amd import moe
    g = moe.preset(2)
    say("verify mfma bf16 out, empty position, repeated expert")
    verify_mode(_lib.VERIFY_UNION_MFMA)
    spans = [oracle.synth_expert(41, e, g.hidden, g.intermediate) for e in range(5)]
    d = [_t(sp) for sp in spans]
    routes = [[0, 1, 2], [], [2, 3, 0, 4], [4, 4]]
    rng = np.random.default_rng(5)
    x = _bf16_round(rng.standard_normal((4, g.hidden)).astype(np.float32))
    edges, wts, offs = [], [], [0]
    for r in routes:
        w = rng.random(len(r)).astype(np.float32)
        edges += [d[e] for e in r]
        wts += w.tolist()
        offs.append(len(edges))
    ws = moe.workspace(g, len(edges), 4)
    out = moe.moe_verify(g, edges, wts, offs, _bf16(x).reshape(4, g.hidden), ws,
                         out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    bits = out.view(torch.int16).cpu().numpy().view(np.uint16)
    for p, r in enumerate(routes):
        if not r:
            assert np.all(bits[p] == 0)
            continue
        ref, mag = oracle.moe_layer_f64([spans[e] for e in r],
                                        np.asarray(wts[offs[p]:offs[p + 1]], np.float64),
                                        g.hidden, g.intermediate, g.activation, x[p])
        got = synth.bf16_bits_to_f32(bits[p]).astype(np.float64)
        scale = np.maximum(np.abs(ref), mag / math.sqrt(g.intermediate))
        ulp = np.maximum(np.abs(ref), 1e-30) * 2.0 ** -7
        assert np.all(np.abs(got - ref) <= ulp + TOL * scale), f"position {p}"


def test_verify_mfma_capability(gpu, verify_mode):
    """The matrix-core path takes at most 16 edges per expert: forcing it on a
    route with 17 returns K3_HIP_E_CAPABILITY; AUTO runs the call elsewhere."""
    import torch
    from deltafin_amd import moe
    g = moe.preset(2)
    say("verify mfma capability miss")
    span = _t(oracle.synth_expert(51, 0, g.hidden, g.intermediate))
    other = _t(oracle.synth_expert(51, 1, g.hidden, g.intermediate))
    m = 16
    # position 0 holds the expert twice, positions 1-15 once each: 17 edges
    edges = [span, span] + [span, other] * 15
    offs = [0, 2] + [2 + 2 * (i + 1) for i in range(15)]
    assert offs[-1] == len(edges) and len(offs) == m + 1
    wts = [0.5] * len(edges)
    x = _bf16(_bf16_round(np.random.default_rng(0).standard_normal((m, g.hidden))
                          .astype(np.float32))).reshape(m, g.hidden)
    ws = moe.workspace(g, len(edges), m)
    verify_mode(_lib.VERIFY_UNION_MFMA)
    with pytest.raises(_lib.K3HipError) as ei:
        moe.moe_verify(g, edges, wts, offs, x, ws)
    assert ei.value.status == _lib.K3_HIP_E_CAPABILITY
    verify_mode(_lib.VERIFY_AUTO)
    out = moe.moe_verify(g, edges, wts, offs, x, ws)
    torch.cuda.synchronize()
    assert np.all(np.isfinite(out.cpu().numpy()))


def test_verify_mfma_scale_255(gpu, verify_mode):
    """A 255 scale byte in a gate row makes that h element NaN
    (tools/cuda_moe_kernels.cu:128-131), so every output of a position that
    routes the expert is NaN; other positions stay finite and in tolerance."""
    import torch
    from deltafin_amd import moe
    g = moe.preset(2)
    say("verify mfma scale 255")
    verify_mode(_lib.VERIFY_UNION_MFMA)
    spans = [oracle.synth_expert(61, e, g.hidden, g.intermediate) for e in range(4)]
    bad = spans[1].copy()
    w1s = oracle.expert_offsets(g.hidden, g.intermediate)[1]
    bad[w1s + 5 * (g.hidden // 32) + 3] = 255  # gate row 5, group 3
    spans[1] = bad
    d = [_t(sp) for sp in spans]
    routes = [[0, 1], [2, 3], [3, 1, 0], [0, 2]]
    rng = np.random.default_rng(9)
    x = _bf16_round(rng.standard_normal((4, g.hidden)).astype(np.float32))
    edges, wts, offs = [], [], [0]
    for r in routes:
        edges += [d[e] for e in r]
        wts += [1.0 / len(r)] * len(r)
        offs.append(len(edges))
    ws = moe.workspace(g, len(edges), 4)
    out = moe.moe_verify(g, edges, wts, offs, _bf16(x).reshape(4, g.hidden), ws)
    torch.cuda.synchronize()
    out = out.cpu().numpy()
    for p, r in enumerate(routes):
        if 1 in r:
            assert np.all(np.isnan(out[p])), f"position {p} should be NaN"
            continue
        ref, mag = oracle.moe_layer_f64([spans[e] for e in r], np.full(len(r), 1.0 / len(r)),
                                        g.hidden, g.intermediate, g.activation, x[p])
        assert oracle.cond_rel_err(out[p], ref, mag, g.intermediate) <= TOL


def test_verify_mfma_spans_above_2g_low_word(gpu, verify_mode):
    """Expert spans whose addresses have bit 31 of the low word set, and clear.
    The kernels rebuild each span pointer in scalar registers from two 32-bit
    halves; widening a half that went through a signed int would set the high
    word to all ones for the first kind and fault (this case pins that)."""
    import torch
    from deltafin_amd import moe
    g = moe.preset(2)
    span = g.expert_span
    say("verify mfma spans at low words above and below 2^31")
    verify_mode(_lib.VERIFY_UNION_MFMA)
    per_site = 3
    buf = torch.empty((1 << 31) + per_site * span + 4096, dtype=torch.uint8, device="cuda")
    base = buf.data_ptr()
    ptrs, spans = [], []
    for site in (0, 1 << 31):  # low-word bit 31 differs between the two sites
        off = site + ((-(base + site)) & 255)
        for j in range(per_site):
            sp = oracle.synth_expert(71, len(spans), g.hidden, g.intermediate)
            o = off + j * span
            buf[o:o + span].copy_(torch.from_numpy(sp))
            ptrs.append(base + o)
            spans.append(sp)
    lows = {(p & 0xffffffff) >= 0x80000000 for p in ptrs}
    assert lows == {True, False}
    routes = [[0, 3, 1], [4, 5, 2, 0], [3, 4], [1, 2, 5, 3]]
    rng = np.random.default_rng(13)
    x = _bf16_round(rng.standard_normal((4, g.hidden)).astype(np.float32))
    edges, wts, offs = [], [], [0]
    for r in routes:
        w = rng.random(len(r)).astype(np.float32)
        edges += [ptrs[e] for e in r]
        wts += w.tolist()
        offs.append(len(edges))
    ws = moe.workspace(g, len(edges), 4)
    out = moe.moe_verify(g, edges, wts, offs, _bf16(x).reshape(4, g.hidden), ws)
    torch.cuda.synchronize()
    out = out.cpu().numpy()
    for p, r in enumerate(routes):
        ref, mag = oracle.moe_layer_f64([spans[e] for e in r],
                                        np.asarray(wts[offs[p]:offs[p + 1]], np.float64),
                                        g.hidden, g.intermediate, g.activation, x[p])
        assert oracle.cond_rel_err(out[p], ref, mag, g.intermediate) <= TOL, f"position {p}"
    del buf
