"""GPU tests of the scale4-v2 expert layout through the descriptor surface
(k3_hip_moe_layer_desc_v1 / k3_hip_moe_positions_desc_v1), the consumer the
reference has in its Metal bridge (tools/metal_moe.mm:127-155, :353-450;
tools/metal/moe_mxfp4.metal:194-300).

scale4-v2 keeps the E2M1 planes of raw-v1 byte for byte and stores each
matrix's E8M0 scales as 4-bit indices over a per-matrix base, so a layer over
scale4-v2 spans must equal, bit for bit, the same layer over the raw-v1 spans
they were made from (both run the same kernels and arithmetic; only where the
scale byte comes from differs), and both must match the fp64 oracle.
"""
import ctypes as C

import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu

TOL = 1e-3
H, I = 3584, 3072


def say(msg):
    print(f"[gpu-case] {msg}", flush=True)


def _k3(lib):
    from deltafin_amd import _lib, moe
    g = moe.preset(1)
    assert lib.k3_hip_configure_v1(C.byref(g)) == 0, _lib.last_error()
    return g


def _experts(n, seed, lo=119, hi=127):
    raw = [oracle.synth_expert(seed, e, H, I, lo, hi) for e in range(n)]
    return raw, [oracle.scale4_span(r, bytes([e] * 32)) for e, r in enumerate(raw)]


def _weights(n, seed):
    lg = np.random.default_rng(seed).standard_normal(n)
    w = np.exp(lg - lg.max())
    return (w / w.sum()).astype(np.float32)


def test_capability_reported(gpu):
    from deltafin_amd import _lib
    _k3(gpu)
    assert gpu.k3_hip_layout_capabilities() & _lib.K3_CAP_SCALE4_V2


def test_layer_scale4_equals_raw_and_oracle(gpu):
    from deltafin_amd import _lib, moe
    g = _k3(gpu)
    n = 16
    say(f"scale4-v2 layer, {n} K3 experts")
    # one expert spans the whole 4-bit range of its base
    raw, s4 = _experts(n - 1, 31)
    wide = oracle.synth_expert(32, 0, H, I, 100, 115)
    raw.append(wide)
    s4.append(oracle.scale4_span(wide))
    assert s4[-1][64:67].tolist() == [100, 100, 100]
    w = _weights(n, 1)
    x = np.random.default_rng(2).standard_normal(H).astype(np.float32)
    out_raw = moe.moe_layer_desc(raw, w, x)
    out_s4 = moe.moe_layer_desc(s4, w, x, layout=_lib.K3_LAYOUT_SCALE4_V2)
    assert np.array_equal(out_s4.view(np.uint32), out_raw.view(np.uint32))
    ref, mag = oracle.moe_layer_f64(raw, w.astype(np.float64), H, I, g.activation, x)
    err = oracle.cond_rel_err(out_s4, ref, mag, I)
    assert err <= TOL, f"cond rel err {err:.3e}"


def test_positions_scale4(gpu):
    """Verify positions over scale4-v2 spans run one decode layer per position
    (an empty position gives a zero row)."""
    from deltafin_amd import _lib, moe
    g = _k3(gpu)
    say("scale4-v2 positions")
    raw, s4 = _experts(6, 41)
    edges = [0, 1, 2, 3, 4, 2, 5, 0, 4, 1, 3, 5]
    offs = [0, 5, 5, 12]
    w = np.concatenate([_weights(5, 3), _weights(7, 4)])
    x = np.random.default_rng(5).standard_normal((3, H)).astype(np.float32)
    S4 = _lib.K3_LAYOUT_SCALE4_V2
    out = moe.moe_positions_desc([s4[e] for e in edges], offs, w, x, layout=S4)
    assert np.all(out[1] == 0)
    for p in (0, 2):
        sl = slice(offs[p], offs[p + 1])
        one = moe.moe_layer_desc([s4[e] for e in edges[sl]], w[sl], x[p], layout=S4)
        assert np.array_equal(out[p].view(np.uint32), one.view(np.uint32)), f"position {p}"
        ref, mag = oracle.moe_layer_f64([raw[e] for e in edges[sl]], w[sl].astype(np.float64),
                                        H, I, g.activation, x[p])
        assert oracle.cond_rel_err(out[p], ref, mag, I) <= TOL


def test_scale4_device_blobs(gpu):
    """Device-resident scale4-v2 spans: the header is read back for the checks."""
    import torch
    from deltafin_amd import _lib, moe
    _k3(gpu)
    say("scale4-v2 device blobs")
    raw, s4 = _experts(4, 51)
    dev = [torch.from_numpy(s).cuda() for s in s4]
    torch.cuda.synchronize()
    w = _weights(4, 6)
    x = np.random.default_rng(7).standard_normal(H).astype(np.float32)
    S4 = _lib.K3_LAYOUT_SCALE4_V2
    a = moe.moe_layer_desc(s4, w, x, layout=S4)
    b = moe.moe_layer_desc(dev, w, x, layout=S4)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_scale4_rejections(gpu):
    from deltafin_amd import _lib, moe
    _k3(gpu)
    say("scale4-v2 descriptor rejections")
    raw, s4 = _experts(2, 61)
    w = _weights(2, 8)
    x = np.zeros(H, np.float32)
    lib = gpu
    d = moe._descs([s4[0], raw[1]], _lib.K3_SCALE4_V2_EXPERT_SPAN, _lib.K3_LAYOUT_SCALE4_V2)
    d[1].layout_id = _lib.K3_LAYOUT_RAW_V1
    d[1].blob_bytes = _lib.K3_RAW_V1_EXPERT_SPAN
    out = np.empty(H, np.float32)
    rc = lib.k3_hip_moe_layer_desc_v1(d, 2, w.ctypes.data, x.ctypes.data, out.ctypes.data)
    assert rc == _lib.K3_HIP_E_DESCRIPTOR and "mixed" in _lib.last_error()
    bad = s4[1].copy()
    bad[70] = 1  # reserved padding
    d = moe._descs([s4[0], bad], _lib.K3_SCALE4_V2_EXPERT_SPAN, _lib.K3_LAYOUT_SCALE4_V2)
    rc = lib.k3_hip_moe_layer_desc_v1(d, 2, w.ctypes.data, x.ctypes.data, out.ctypes.data)
    assert rc == _lib.K3_HIP_E_DESCRIPTOR and "reserved" in _lib.last_error()
    d = moe._descs([raw[0]], _lib.K3_RAW_V1_EXPERT_SPAN, _lib.K3_LAYOUT_SCALE4_V2)
    rc = lib.k3_hip_moe_layer_desc_v1(d, 1, w.ctypes.data, x.ctypes.data, out.ctypes.data)
    assert rc == _lib.K3_HIP_E_DESCRIPTOR


def test_scale4_index_15_over_base_240_is_nan(gpu):
    """Base 240 plus index 15 is E8M0 255: the row it scales is NaN, as with a
    raw 255 byte (tools/cuda_moe_kernels.cu:128-131)."""
    from deltafin_amd import _lib, moe
    _k3(gpu)
    say("scale4-v2 NaN through base 240 + 15")
    raw = oracle.synth_expert(71, 0, H, I)  # scale bytes in [119, 127]
    off = oracle.expert_offsets(H, I)
    raw[off[3]:off[4]] += 121  # w2 scales in [240, 248]: base 240
    raw[off[3] + 5 * (I // 32) + 7] = 255  # w2 row 5, group 7: index 15
    span4 = oracle.scale4_span(raw)
    assert span4[65] == 240
    # x this small leaves h at zero, so every output row is 0 except the
    # NaN-scaled one (0 * NaN)
    x = np.random.default_rng(9).standard_normal(H).astype(np.float32) * 1e-30
    a = moe.moe_layer_desc([raw], [1.0], x)
    b = moe.moe_layer_desc([span4], [1.0], x, layout=_lib.K3_LAYOUT_SCALE4_V2)
    assert np.isnan(a[5]) and np.isnan(b[5])
    assert np.array_equal(np.isnan(a), np.isnan(b))
    fin = ~np.isnan(a)
    assert np.array_equal(a[fin].view(np.uint32), b[fin].view(np.uint32))
