"""GPU parity: the gfx950 library through its C ABI against the CPU oracle.

Bar: max relative error <= 1e-3 against the
fp64-accumulated oracle, measured per output against max(|ref|, mag/sqrt(n))
where mag is the sum of |terms| of that output (oracle.cond_rel_err), with
router top-k IDs identical.  bf16 outputs are compared with the oracle rounded
to bf16 within one bf16 ulp.  Known-answer tests reproduce the reference's
in-code KATs (provider_cpu_isa_test.c:60-76, provider_cuda_moe.cpp:297-422).
"""
import ctypes as C
import math

import numpy as np
import pytest

import oracle
from deltafin_amd import synth

pytestmark = pytest.mark.gpu

TOL = 1e-3


def say(msg):
    print(f"[gpu-case] {msg}", flush=True)


def _t(a, dtype=None):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(a))
    if dtype is not None:
        t = t.to(dtype)
    return t.cuda()


def _bf16(x32):
    import torch
    return torch.from_numpy(synth.to_bf16_bits(x32).view(np.int16)).view(torch.bfloat16).cuda()


def _bf16_ulp_ok(out_bits: np.ndarray, ref64: np.ndarray, mag, n_terms) -> bool:
    got = synth.bf16_bits_to_f32(out_bits).astype(np.float64)
    scale = np.maximum(np.abs(ref64), np.asarray(mag) / math.sqrt(n_terms))
    # one bf16 ulp of the reference value plus the fp32 tolerance band
    ulp = np.maximum(np.abs(ref64), 1e-30) * 2.0 ** -7
    return bool(np.all(np.abs(got - ref64) <= ulp + TOL * scale))


def _mxfp4(rows, cols, seed, lo=119, hi=127):
    p, s = oracle.synth_mxfp4(seed, 0, rows * cols // 2, rows * cols // 32, lo, hi)
    return p, s


# ------------------------------------------------------------------ known answers
def test_available(gpu):
    say("k3_hip_moe_available")
    assert gpu.k3_hip_moe_available(0) == 1


def test_kat_all_0x22(gpu):
    """provider_cpu_isa_test.c:60-76: every code +1.0, scale 2^0, x = 1 -> 32.0 exactly."""
    import torch
    from deltafin_amd import moe
    say("kat all 0x22")
    p = _t(np.full(32, 0x22, np.uint8))
    s = _t(np.full(2, 127, np.uint8))
    for xt in (torch.float32, torch.bfloat16):
        x = torch.ones(32, dtype=xt, device="cuda")
        y = moe.mxfp4_gemv(p, s, x, 2, 32)
        torch.cuda.synchronize()
        assert y.cpu().tolist() == [32.0, 32.0]


def test_kat_all_codes_two_batches(gpu):
    """provider_cuda_moe.cpp:297-360: every E2M1 code, scales {127,126}, two x rows."""
    import torch
    from deltafin_amd import moe
    say("kat all codes")
    packed = np.zeros(32, np.uint8)
    for i in range(16):
        ph = (2 * i) % 16
        packed[i] = ph | (((ph + 1) % 16) << 4)
        packed[16 + i] = (15 - ph) | ((14 - ph) << 4)
    scales = np.array([127, 126], np.uint8)
    x = np.zeros(64, np.float32)
    x[:32] = np.arange(32) / 32.0
    x[32:] = (np.arange(32) - 15.0) / 17.0
    expected = np.zeros((2, 2), np.float32)
    for b in range(2):
        for r in range(2):
            tot = np.float32(0)
            for c in range(32):
                byte = packed[r * 16 + c // 2]
                code = byte & 15 if c % 2 == 0 else byte >> 4
                w = np.float32(math.ldexp(oracle.e2m1(int(code)), int(scales[r]) - 127))
                tot = np.float32(math.fma(w, x[b * 32 + c], tot)) if hasattr(math, "fma") \
                    else np.float32(w * x[b * 32 + c] + tot)
            expected[b, r] = tot
    xd = _t(x.reshape(2, 32))
    y1 = moe.mxfp4_gemv(_t(packed), _t(scales), xd, 2, 32)
    y2 = moe.mxfp4_gemv(_t(packed), _t(scales), xd, 2, 32)
    torch.cuda.synchronize()
    a, b = y1.cpu().numpy(), y2.cpu().numpy()
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    assert np.max(np.abs(a - expected)) <= 2e-4
    # element order: each code appears, so a swapped nibble order would fail here
    single = moe.mxfp4_gemv(_t(packed), _t(scales), xd[0].contiguous(), 2, 32)
    torch.cuda.synchronize()
    assert np.max(np.abs(single.cpu().numpy() - expected[0])) <= 2e-4


def test_kat_one_hot_expert_situ(gpu):
    """provider_cuda_moe.cpp:362-422: one nonzero element per matrix at K3 shape."""
    import torch
    from deltafin_amd import moe
    say("kat one-hot expert (K3 SiTU)")
    g = moe.preset(1)
    off = moe.span_offsets(g)
    span = np.zeros(off["span"], np.uint8)
    span[off["w1p"]] = 0x02
    span[off["w1s"]] = 127
    span[off["w2p"]] = 0x02
    span[off["w2s"]] = 127
    span[off["w3p"]] = 0x04
    span[off["w3s"]] = 127
    x = np.zeros((2, g.hidden), np.float32)
    x[0, 0] = 1.0
    x[1, 0] = -0.5
    dspan, dx = _t(span), _t(x)
    h1, o1 = moe.moe_launch(g, dspan, dx)
    h2, o2 = moe.moe_launch(g, dspan, dx)
    torch.cuda.synchronize()
    o1, o2 = o1.cpu().numpy(), o2.cpu().numpy()
    assert np.array_equal(o1.view(np.uint32), o2.view(np.uint32))
    exp = np.zeros_like(o1)
    for r, v in enumerate((1.0, -0.5)):
        exp[r, 0] = oracle.act(oracle.ACT_SITU, v, 2 * v)
    assert np.max(np.abs(o1 - exp)) <= 2e-5


def test_scale_255_poisons_row(gpu):
    """tools/cuda_moe_kernels.cu:128-131: a 255 scale byte makes the row NaN."""
    import torch
    from deltafin_amd import moe
    say("scale 255 NaN row")
    rows, cols = 8, 256
    p, s = _mxfp4(rows, cols, 3)
    s = s.copy()
    s[3 * (cols // 32) + 5] = 255
    x = np.random.default_rng(0).standard_normal(cols).astype(np.float32)
    y = moe.mxfp4_gemv(_t(p), _t(s), _t(x), rows, cols)
    torch.cuda.synchronize()
    y = y.cpu().numpy()
    ref = oracle.gemv_f64(p, s, x, rows, cols)
    assert np.isnan(y[3]) and np.isnan(ref[3])
    assert np.all(np.isfinite(np.delete(y, 3)))


# ------------------------------------------------------------------ GEMV parity
@pytest.mark.parametrize("rows,cols", [(2048, 7168), (7168, 2048), (3072, 3584), (3584, 3072),
                                       (100, 96), (1, 32)])
@pytest.mark.parametrize("xdt", ["f32", "bf16"])
@pytest.mark.parametrize("batches", [1, 3])
def test_gemv_parity(gpu, rows, cols, xdt, batches):
    import torch
    from deltafin_amd import moe
    say(f"gemv {rows}x{cols} x={xdt} batches={batches}")
    p, s = _mxfp4(rows, cols, rows * 7 + cols)
    rng = np.random.default_rng(rows + cols)
    x = rng.standard_normal((batches, cols)).astype(np.float32)
    if xdt == "bf16":
        x = synth.bf16_bits_to_f32(synth.to_bf16_bits(x)).reshape(batches, cols)
        dx = _bf16(x).reshape(batches, cols)
    else:
        dx = _t(x)
    y = moe.mxfp4_gemv(_t(p), _t(s), dx if batches > 1 else dx[0].contiguous(), rows, cols)
    torch.cuda.synchronize()
    y = y.cpu().numpy().reshape(batches, rows)
    for b in range(batches):
        ref, mag = oracle.gemv_f64(p, s, x[b], rows, cols, with_mag=True)
        err = oracle.cond_rel_err(y[b], ref, mag, cols)
        assert err <= TOL, f"batch {b}: cond rel err {err:.3e}"


def test_gemv_bf16_output(gpu):
    import torch
    from deltafin_amd import moe
    say("gemv bf16 output")
    rows, cols = 2048, 7168
    p, s = _mxfp4(rows, cols, 11)
    x = np.random.default_rng(5).standard_normal(cols).astype(np.float32)
    y = moe.mxfp4_gemv(_t(p), _t(s), _t(x), rows, cols, out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    bits = y.cpu().view(torch.int16).numpy().view(np.uint16)
    ref, mag = oracle.gemv_f64(p, s, x, rows, cols, with_mag=True)
    assert _bf16_ulp_ok(bits, ref, mag, cols)


# ------------------------------------------------------------------ expert / layer parity
def _experts(n, hidden, inter, seed, first=0):
    return [oracle.synth_expert(seed, first + e, hidden, inter) for e in range(n)]


@pytest.mark.parametrize("preset_id", [1, 2])
def test_moe_launch_parity(gpu, preset_id):
    import torch
    from deltafin_amd import moe
    g = moe.preset(preset_id)
    say(f"moe_launch preset {preset_id}")
    span = _experts(1, g.hidden, g.intermediate, 21)[0]
    x = np.random.default_rng(preset_id).standard_normal((2, g.hidden)).astype(np.float32)
    h, out = moe.moe_launch(g, _t(span), _t(x))
    torch.cuda.synchronize()
    out = out.cpu().numpy()
    for b in range(2):
        ref, hr, mag = oracle.expert_f64(span, g.hidden, g.intermediate, g.activation, x[b])
        err = oracle.cond_rel_err(out[b], ref, mag, g.intermediate)
        assert err <= TOL, f"row {b}: {err:.3e}"


@pytest.mark.parametrize("preset_id,xdt,odt", [(2, "bf16", "f32"), (2, "bf16", "bf16"),
                                               (2, "f32", "f32"), (1, "f32", "f32")])
def test_moe_layer_device_parity(gpu, preset_id, xdt, odt):
    import torch
    from deltafin_amd import moe
    g = moe.preset(preset_id)
    say(f"moe_layer_device preset {preset_id} x={xdt} out={odt}")
    n = 16
    spans = _experts(n, g.hidden, g.intermediate, 99)
    rng = np.random.default_rng(42)
    lg = rng.standard_normal(n).astype(np.float64)
    w = np.exp(lg - lg.max())
    w = (w / w.sum()).astype(np.float32)
    x = rng.standard_normal(g.hidden).astype(np.float32)
    if xdt == "bf16":
        x = synth.bf16_bits_to_f32(synth.to_bf16_bits(x))
        dx = _bf16(x)
    else:
        dx = _t(x)
    dspans = [_t(sp) for sp in spans]
    ws = moe.workspace(g, n)
    out = moe.moe_layer(g, dspans, w, dx, ws,
                        out_dtype=torch.bfloat16 if odt == "bf16" else torch.float32)
    out2 = moe.moe_layer(g, dspans, w, dx, ws,
                         out_dtype=torch.bfloat16 if odt == "bf16" else torch.float32)
    torch.cuda.synchronize()
    ref, mag = oracle.moe_layer_f64(spans, w.astype(np.float64), g.hidden, g.intermediate,
                                    g.activation, x)
    if odt == "bf16":
        bits = out.cpu().view(torch.int16).numpy().view(np.uint16)
        assert np.array_equal(bits, out2.cpu().view(torch.int16).numpy().view(np.uint16))
        assert _bf16_ulp_ok(bits, ref, mag, g.intermediate)
    else:
        o = out.cpu().numpy()
        assert np.array_equal(o.view(np.uint32), out2.cpu().numpy().view(np.uint32))
        err = oracle.cond_rel_err(o, ref, mag, g.intermediate)
        assert err <= TOL, f"cond rel err {err:.3e}"


def test_route_layer_parity(gpu):
    """Device router + layer over a resident bank: IDs identical to the oracle top-k."""
    import torch
    from deltafin_amd import moe
    g = moe.preset(2)
    n_bank, k = 40, 16
    say(f"route layer bank={n_bank}")
    stride = g.expert_span
    bank = torch.empty(n_bank * stride, dtype=torch.uint8, device="cuda")
    moe.synth_bank(g, bank, stride, n_bank, 0, 1234)
    ws = moe.workspace(g, k)
    rng = np.random.default_rng(7)
    for tok in range(3):
        logits = rng.standard_normal(n_bank).astype(np.float32)
        x = synth.bf16_bits_to_f32(synth.to_bf16_bits(rng.standard_normal(g.hidden).astype(np.float32)))
        out, ids, wts = moe.moe_route_layer(g, bank, stride, n_bank, _t(logits), k, _bf16(x), ws)
        torch.cuda.synchronize()
        rid, rw = oracle.topk_softmax(logits, k)
        assert ids.cpu().numpy().tolist() == rid.tolist()
        assert np.max(np.abs(wts.cpu().numpy() - rw)) <= 1e-6
        spans = [oracle.synth_expert(1234, int(e), g.hidden, g.intermediate) for e in rid]
        ref, mag = oracle.moe_layer_f64(spans, rw, g.hidden, g.intermediate, g.activation, x)
        err = oracle.cond_rel_err(out.cpu().numpy(), ref, mag, g.intermediate)
        assert err <= TOL, f"token {tok}: {err:.3e}"


def test_synth_bank_matches_oracle(gpu):
    import torch
    from deltafin_amd import moe
    g = moe.preset(1)
    say("synth bank vs oracle")
    stride = g.expert_span + 4096
    bank = torch.empty(3 * stride, dtype=torch.uint8, device="cuda")
    moe.synth_bank(g, bank, stride, 3, 5, 77)
    torch.cuda.synchronize()
    host = bank.cpu().numpy()
    for e in range(3):
        ref = oracle.synth_expert(77, 5 + e, g.hidden, g.intermediate)
        assert np.array_equal(host[e * stride: e * stride + g.expert_span], ref)


@pytest.mark.parametrize("m", [1, 4, 8, 16])
def test_verify_route_parity(gpu, m):
    import torch
    from deltafin_amd import moe
    g = moe.preset(2)
    n_bank, k = 48, 16
    say(f"verify route M={m} bank={n_bank}")
    stride = g.expert_span
    bank = torch.empty(n_bank * stride, dtype=torch.uint8, device="cuda")
    moe.synth_bank(g, bank, stride, n_bank, 0, 555)
    rng = np.random.default_rng(100 + m)
    logits = rng.standard_normal((m, n_bank)).astype(np.float32)
    x = synth.bf16_bits_to_f32(synth.to_bf16_bits(rng.standard_normal((m, g.hidden)).astype(np.float32))).reshape(m, g.hidden)
    ws = moe.workspace(g, m * k, m)
    out, ids, wts = moe.moe_verify_route(g, bank, stride, n_bank, _t(logits), k,
                                         _bf16(x).reshape(m, g.hidden), ws)
    torch.cuda.synchronize()
    out = out.cpu().numpy()
    ids = ids.cpu().numpy()
    cache = {}
    for p in range(m):
        rid, rw = oracle.topk_softmax(logits[p], k)
        assert ids[p].tolist() == rid.tolist()
        spans = []
        for e in rid:
            if int(e) not in cache:
                cache[int(e)] = oracle.synth_expert(555, int(e), g.hidden, g.intermediate)
            spans.append(cache[int(e)])
        ref, mag = oracle.moe_layer_f64(spans, rw, g.hidden, g.intermediate, g.activation, x[p])
        err = oracle.cond_rel_err(out[p], ref, mag, g.intermediate)
        assert err <= TOL, f"position {p}: {err:.3e}"


def test_verify_table_matches_layer(gpu):
    """Caller-routed verify with repeated experts and an empty position equals
    per-position layer calls."""
    import torch
    from deltafin_amd import moe
    g = moe.preset(1)
    say("verify table vs per-position layer")
    spans = _experts(5, g.hidden, g.intermediate, 8)
    d = [_t(sp) for sp in spans]
    routes = [[0, 1, 2], [], [2, 3, 0, 4], [4]]
    rng = np.random.default_rng(3)
    x = rng.standard_normal((4, g.hidden)).astype(np.float32)
    edges, wts, offs = [], [], [0]
    for r in routes:
        w = rng.random(len(r)).astype(np.float32)
        edges += [d[e] for e in r]
        wts += w.tolist()
        offs.append(len(edges))
    ws = moe.workspace(g, len(edges), 4)
    out = moe.moe_verify(g, edges, wts, offs, _t(x), ws)
    torch.cuda.synchronize()
    out = out.cpu().numpy()
    for p, r in enumerate(routes):
        if not r:
            assert np.all(out[p] == 0)
            continue
        ref, mag = oracle.moe_layer_f64([spans[e] for e in r], wts[offs[p]:offs[p + 1]], g.hidden,
                                        g.intermediate, g.activation, x[p])
        assert oracle.cond_rel_err(out[p], ref, mag, g.intermediate) <= TOL


@pytest.mark.parametrize("m", [4, 8, 16])
def test_verify_route_bank384(gpu, m):
    """Device-routed verify over a config-3-sized bank (384 experts, 8.98 GB:
    span addresses on both sides of every 2^31 boundary of the low word)."""
    import torch
    from deltafin_amd import moe
    g = moe.preset(2)
    n_bank, k = 384, 16
    say(f"verify route M={m} bank={n_bank}")
    stride = g.expert_span
    bank = torch.empty(n_bank * stride, dtype=torch.uint8, device="cuda")
    moe.synth_bank(g, bank, stride, n_bank, 0, 777)
    rng = np.random.default_rng(200 + m)
    logits = rng.standard_normal((m, n_bank)).astype(np.float32)
    x = synth.bf16_bits_to_f32(synth.to_bf16_bits(
        rng.standard_normal((m, g.hidden)).astype(np.float32))).reshape(m, g.hidden)
    ws = moe.workspace(g, m * k, m)
    out, ids, _ = moe.moe_verify_route(g, bank, stride, n_bank, _t(logits), k,
                                       _bf16(x).reshape(m, g.hidden), ws)
    torch.cuda.synchronize()
    out = out.cpu().numpy()
    for p in range(m):
        rid, rw = oracle.topk_softmax(logits[p], k)
        assert ids[p].cpu().numpy().tolist() == rid.tolist()
        spans = [oracle.synth_expert(777, int(e), g.hidden, g.intermediate) for e in rid]
        ref, mag = oracle.moe_layer_f64(spans, rw, g.hidden, g.intermediate, g.activation, x[p])
        assert oracle.cond_rel_err(out[p], ref, mag, g.intermediate) <= TOL


@pytest.mark.skipif(not oracle.ref_available(), reason="reference CPU library not built")
def test_k3_layer_vs_reference_expert_set(gpu):
    """K3 at full shape (hidden 3584, intermediate 3072, SiTU, 16 experts)
    against the reference's own whole-set call mxfp4_moe_expert_set
    (tools/fused_gemv_batch.c:465-518, built from the reference sources into
    oracle/_ref), within 2e-4 of the output's condition scale, the bound the
    reference's full-layer parity test uses (provider_moe_test.cpp:268-296).
    Checked through the device surface and through the descriptor surface with
    raw-v1 and scale4-v2 spans."""
    import torch
    from deltafin_amd import _lib, moe
    g = moe.preset(1)
    assert gpu.k3_hip_configure_v1(C.byref(g)) == 0
    n = 16
    say(f"K3 layer vs reference mxfp4_moe_expert_set, {n} experts")
    spans = _experts(n, g.hidden, g.intermediate, 808)
    rng = np.random.default_rng(909)
    w = rng.random(n).astype(np.float32)
    w /= w.sum()
    x = rng.standard_normal(g.hidden).astype(np.float32)
    want = oracle.ref_expert_set(spans, w, x, g.hidden, g.intermediate, threads=8)
    _, mag = oracle.moe_layer_f64(spans, w.astype(np.float64), g.hidden, g.intermediate,
                                  g.activation, x)
    outs = {}
    dspans = [_t(sp) for sp in spans]
    outs["device"] = moe.moe_layer(g, dspans, w, _t(x), moe.workspace(g, n)).cpu().numpy()
    outs["descriptor raw-v1"] = moe.moe_layer_desc(spans, w, x)
    s4 = [oracle.scale4_span(sp) for sp in spans]
    outs["descriptor scale4-v2"] = moe.moe_layer_desc(s4, w, x, layout=_lib.K3_LAYOUT_SCALE4_V2)
    torch.cuda.synchronize()
    for name, got in outs.items():
        err = oracle.cond_rel_err(got, want, mag, g.intermediate)
        assert err <= 2e-4, f"{name}: {err:.3e}"


@pytest.mark.parametrize("n", [1, 3, 8, 13])
def test_k3_layer_route_counts(gpu, n):
    """The K3 down kernel at every workgroup shape it takes (1, 2, 4 and 7 row
    pairs per workgroup for 1, 3, 8 and 13 routed experts), raw-v1 against the
    oracle, and scale4-v2 spans bit-equal to raw-v1 (same arithmetic)."""
    import torch
    from deltafin_amd import _lib, moe
    g = moe.preset(1)
    assert gpu.k3_hip_configure_v1(C.byref(g)) == 0
    say(f"K3 layer, {n} experts")
    spans = _experts(n, g.hidden, g.intermediate, 515 + n)
    rng = np.random.default_rng(n)
    w = rng.random(n).astype(np.float32) + 0.05
    w /= w.sum()
    x = rng.standard_normal(g.hidden).astype(np.float32)
    dspans = [_t(sp) for sp in spans]
    ws = moe.workspace(g, n)
    out = moe.moe_layer(g, dspans, w, _t(x), ws)
    out_bf = moe.moe_layer(g, dspans, w, _t(x), ws, out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    o = out.cpu().numpy()
    ref, mag = oracle.moe_layer_f64(spans, w.astype(np.float64), g.hidden, g.intermediate,
                                    g.activation, x)
    err = oracle.cond_rel_err(o, ref, mag, g.intermediate)
    assert err <= TOL, f"cond rel err {err:.3e}"
    bits = out_bf.cpu().view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(bits, synth.to_bf16_bits(o))
    s4 = [oracle.scale4_span(sp) for sp in spans]
    got = moe.moe_layer_desc(s4, w, x, layout=_lib.K3_LAYOUT_SCALE4_V2)
    assert np.array_equal(got.view(np.uint32), moe.moe_layer_desc(spans, w, x).view(np.uint32))


@pytest.mark.parametrize("n,xdt", [(1, "bf16"), (1, "f32"), (2, "bf16"), (3, "f32")])
def test_moe_layer_few_experts(gpu, n, xdt):
    """Preset 2 with 1-3 routed experts: the gate/up kernel's 2-row units (a
    pipeline would otherwise hold one unit) and the down kernel's 16 / n
    workgroups per CU, against the oracle; two calls bit-equal."""
    import torch
    from deltafin_amd import moe
    g = moe.preset(2)
    say(f"layer preset 2, {n} experts, x={xdt}")
    spans = _experts(n, g.hidden, g.intermediate, 700 + n)
    rng = np.random.default_rng(70 + n)
    w = rng.random(n).astype(np.float32) + 0.1
    w /= w.sum()
    x = rng.standard_normal(g.hidden).astype(np.float32)
    if xdt == "bf16":
        x = synth.bf16_bits_to_f32(synth.to_bf16_bits(x))
        dx = _bf16(x)
    else:
        dx = _t(x)
    dspans = [_t(sp) for sp in spans]
    ws = moe.workspace(g, n)
    out = moe.moe_layer(g, dspans, w, dx, ws).cpu().numpy()
    out2 = moe.moe_layer(g, dspans, w, dx, ws).cpu().numpy()
    assert np.array_equal(out.view(np.uint32), out2.view(np.uint32))
    ref, mag = oracle.moe_layer_f64(spans, w.astype(np.float64), g.hidden, g.intermediate,
                                    g.activation, x)
    err = oracle.cond_rel_err(out, ref, mag, g.intermediate)
    assert err <= TOL, f"cond rel err {err:.3e}"


@pytest.mark.parametrize("preset_id,n", [(2, 20), (2, 32), (1, 24)])
def test_moe_layer_many_experts(gpu, preset_id, n):
    """More than 16 routed experts (up to K3_HIP_MAX_TOKEN_EXPERTS = 32): the
    down kernel for more experts than a workgroup has waves (k_down_blocks,
    waves walking several experts), against the oracle."""
    import torch
    from deltafin_amd import moe
    g = moe.preset(preset_id)
    say(f"layer preset {preset_id}, {n} experts")
    spans = _experts(n, g.hidden, g.intermediate, 900 + n)
    rng = np.random.default_rng(90 + n)
    w = rng.random(n).astype(np.float32) + 0.05
    w /= w.sum()
    x = rng.standard_normal(g.hidden).astype(np.float32)
    dspans = [_t(sp) for sp in spans]
    ws = moe.workspace(g, n)
    out = moe.moe_layer(g, dspans, w, _t(x), ws).cpu().numpy()
    ref, mag = oracle.moe_layer_f64(spans, w.astype(np.float64), g.hidden, g.intermediate,
                                    g.activation, x)
    err = oracle.cond_rel_err(out, ref, mag, g.intermediate)
    assert err <= TOL, f"cond rel err {err:.3e}"


def test_route_layer_top24(gpu):
    """Device router with top_k 24 over a 40-expert bank: ids identical to the
    oracle's top-k, output within the bar."""
    import torch
    from deltafin_amd import moe
    g = moe.preset(2)
    n_bank, k = 40, 24
    say(f"route layer bank={n_bank} top_k={k}")
    stride = g.expert_span
    bank = torch.empty(n_bank * stride, dtype=torch.uint8, device="cuda")
    moe.synth_bank(g, bank, stride, n_bank, 0, 4321)
    ws = moe.workspace(g, k)
    rng = np.random.default_rng(24)
    logits = rng.standard_normal(n_bank).astype(np.float32)
    x = synth.bf16_bits_to_f32(synth.to_bf16_bits(rng.standard_normal(g.hidden).astype(np.float32)))
    out, ids, wts = moe.moe_route_layer(g, bank, stride, n_bank, _t(logits), k, _bf16(x), ws)
    torch.cuda.synchronize()
    rid, rw = oracle.topk_softmax(logits, k)
    assert ids.cpu().numpy().tolist() == rid.tolist()
    assert np.max(np.abs(wts.cpu().numpy() - rw)) <= 1e-6
    spans = [oracle.synth_expert(4321, int(e), g.hidden, g.intermediate) for e in rid]
    ref, mag = oracle.moe_layer_f64(spans, rw, g.hidden, g.intermediate, g.activation, x)
    err = oracle.cond_rel_err(out.cpu().numpy(), ref, mag, g.intermediate)
    assert err <= TOL, f"cond rel err {err:.3e}"
