"""CPU pins of the spine oracle (oracle/spine.py) and host-side checks of the
spine C ABI (include/k3_hip_spine_abi.h) that need no GPU.

Each oracle function is checked against something other than its own formula:
closed-form BF16 values, pure-Python loops, linearity, one-hot inputs, the
dense row-int8 materialisation and closed-form RMS norms.
"""
import math
import struct

import numpy as np
import pytest

from oracle import spine as S


def _py_bf16(bits: int) -> float:
    return struct.unpack("<f", struct.pack("<I", (bits & 0xFFFF) << 16))[0]


def test_bf16_fixture_patterns_closed_form():
    # IEEE binary32 with the low 16 bits zero: sign, 8-bit exponent, 7-bit fraction.
    want = {
        0x0000: 0.0, 0x0001: 2.0 ** -133, 0x007F: 127 * 2.0 ** -133, 0x0080: 2.0 ** -126,
        0x3D00: 0.03125, 0x3E80: 0.25, 0x3F00: 0.5, 0x3F80: 1.0, 0x4000: 2.0, 0x4040: 3.0,
        0x4080: 4.0, 0x8000: -0.0, 0xBD00: -0.03125, 0xBE80: -0.25, 0xBF00: -0.5, 0xBF80: -1.0,
    }
    got = S.bf16_to_f32(S.FIXTURE_PATTERNS)
    for bits, value in zip(S.FIXTURE_PATTERNS.tolist(), got.tolist()):
        assert value == want[bits], hex(bits)
        assert math.copysign(1.0, value) == math.copysign(1.0, want[bits])


def test_bf16_special_encodings():
    bits = np.array([0x7F80, 0xFF80, 0x7FC0, 0x7F81, 0x7F7F, 0x3F81], dtype=np.uint16)
    v = S.bf16_to_f32(bits)
    assert v[0] == np.inf and v[1] == -np.inf
    assert np.isnan(v[2]) and np.isnan(v[3])
    assert v[4] == np.float32((2 - 2.0 ** -7) * 2.0 ** 127)  # largest finite BF16
    assert v[5] == np.float32(1 + 2.0 ** -7)
    every = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    assert np.array_equal(S.bf16_to_f32_bits(every), np.arange(65536, dtype=np.uint32) << 16)


def test_spine_bf16_against_python_loops():
    rng = np.random.default_rng(7)
    w = rng.integers(0, 65536, size=(5, 37), dtype=np.uint32).astype(np.uint16)
    w[(S.bf16_to_f32_bits(w) & 0x7F800000) == 0x7F800000] = 0x3F80  # finite only
    x = rng.standard_normal((3, 37)).astype(np.float32)
    got = S.spine_bf16_f64(w, x)
    for p in range(3):
        for r in range(5):
            want = sum(_py_bf16(int(w[r, c])) * float(x[p, c]) for c in range(37))
            assert got[p, r] == pytest.approx(want, rel=1e-12, abs=1e-300)


def test_spine_bf16_linearity_and_one_hot():
    rng = np.random.default_rng(8)
    w = (rng.standard_normal((9, 64)).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
    a = rng.standard_normal((1, 64)).astype(np.float32)
    b = rng.standard_normal((1, 64)).astype(np.float32)
    lin = S.spine_bf16_f64(w, a) * 2.0 - S.spine_bf16_f64(w, b) * 0.5
    both = S.spine_bf16_f64(w, (2 * a.astype(np.float64) - 0.5 * b).astype(np.float32))
    assert np.allclose(lin, both, rtol=1e-6, atol=1e-6)
    for c in (0, 17, 63):
        e = np.zeros((1, 64), np.float32)
        e[0, c] = 1.0
        assert np.array_equal(S.spine_bf16_f64(w, e)[0], S.bf16_to_f32(w[:, c]).astype(np.float64))


def test_spine_int8_against_dense_and_loops():
    rng = np.random.default_rng(9)
    q = rng.integers(-128, 128, size=(6, 48), dtype=np.int8)
    s = rng.uniform(0.001, 0.1, size=6).astype(np.float32)
    x = rng.standard_normal((2, 48)).astype(np.float32)
    dense = q.astype(np.float64) * s.astype(np.float64)[:, None]  # materialize_row_int8
    got = S.spine_int8_f64(q, s, x)
    assert np.allclose(got, x.astype(np.float64) @ dense.T, rtol=1e-12, atol=1e-12)
    want = [[float(s[r]) * sum(int(q[r, c]) * float(x[p, c]) for c in range(48)) for r in range(6)]
            for p in range(2)]
    assert np.allclose(got, want, rtol=1e-12, atol=1e-12)
    ones = np.ones((6, 48), np.int8)
    assert np.allclose(S.spine_int8_f64(ones, s, x)[1], s * x[1].astype(np.float64).sum())


def test_rms_norm_closed_forms():
    eps = 1e-5
    for c in (0.0, 1.0, -3.0, 1e-3):
        x = np.full((1, 16), c, np.float32)
        w = np.arange(1, 17, dtype=np.float32)
        got = S.rms_norm_f64(x, w, eps)[0]
        c = float(np.float32(c))
        want = w.astype(np.float64) * (c / math.sqrt(c * c + float(np.float32(eps))))
        assert np.allclose(got, want, rtol=1e-12, atol=0)
    x = np.array([[3.0, 4.0]], np.float32)  # mean square 12.5
    got = S.rms_norm_f64(x, np.array([1.0, 2.0], np.float32), 0.0)[0]
    assert np.allclose(got, [3 / math.sqrt(12.5), 8 / math.sqrt(12.5)], rtol=1e-15)
    rng = np.random.default_rng(10)
    x = rng.standard_normal((3, 100)).astype(np.float32)
    w = rng.standard_normal(100).astype(np.float32)
    assert np.allclose(S.rms_norm_f64(x, w, 0.0), S.rms_norm_f64(8 * x, w, 0.0), rtol=1e-12)


def test_reference_fixture_shapes_and_bound():
    w, act, exp = S.spine_fixture(19, 521, 5)
    assert w.shape == (19, 521) and act.shape == (521,) and exp.shape == (19,)
    assert w[0, 0] == S.FIXTURE_PATTERNS[5] and w[0, 1] == S.FIXTURE_PATTERNS[(13 + 5) % 16]
    assert act[0] == np.float32((5 % 29 - 14) / 31.0)
    assert S.spine_close(exp, exp)
    assert not S.spine_close(exp + 1e-3, exp)
    bad = exp.copy()
    bad[3] = np.nan
    assert not S.spine_close(bad, exp)


# ----------------------------------------------------------- host-side ABI checks


def test_spine_abi_host_checks():
    from deltafin_amd import _lib
    lib = _lib.load()
    assert lib.k3_hip_spine_bf16_abi_version() == 1
    buf = np.zeros(64, np.float32)
    p = buf.ctypes.data
    # argument checks fail before anything is enqueued (-1, as the reference's)
    assert lib.k3_hip_spine_bf16_launch_v1(None, p, p, 1, 8, 1, None) == _lib.K3_SPINE_E_INVALID
    assert "null" in lib.k3_hip_spine_last_error().decode()
    assert lib.k3_hip_spine_bf16_launch_v1(p, p, p, 1, 8, 65, None) == _lib.K3_SPINE_E_INVALID
    assert lib.k3_hip_spine_bf16_launch_v1(p, p, p, 1, 8, 0, None) == _lib.K3_SPINE_E_INVALID
    assert lib.k3_hip_spine_bf16_launch_v1(p, p, p, 0, 8, 1, None) == _lib.K3_SPINE_E_INVALID
    assert lib.k3_hip_spine_int8_launch_v1(p, None, p, p, 1, 16, 1, None) == _lib.K3_SPINE_E_INVALID
    assert lib.k3_hip_spine_bf16_decode_bits(p, p, 0, None) == _lib.K3_SPINE_E_INVALID
    assert lib.k3_hip_rms_norm(p, p, p, 1, 0, 1e-5, None) == _lib.K3_SPINE_E_INVALID
    assert lib.k3_hip_rms_norm(p, p, p, 1, 8, float("nan"), None) == _lib.K3_SPINE_E_INVALID


def test_spine_available_without_device():
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    from deltafin_amd import _lib
    lib = _lib.load()
    assert lib.k3_hip_spine_bf16_available(0, None, None) < 0


# ----------------------------------------------------------- K3 router and block


def test_k3_router_zero_bias_is_topk_of_logits():
    import oracle
    rng = np.random.default_rng(11)
    logits = rng.standard_normal(896).astype(np.float32)
    ids, w = S.k3_router_f64(logits, np.zeros(896, np.float32), 16)
    ref_ids, _ = oracle.topk_softmax(logits, 16)  # sigmoid is monotone
    assert ids.tolist() == ref_ids.tolist()
    s = 1 / (1 + np.exp(-logits[ids].astype(np.float64)))
    assert np.allclose(w, s / s.sum(), rtol=1e-14)


def test_k3_router_python_sort_and_forced():
    rng = np.random.default_rng(12)
    logits = rng.standard_normal(40).astype(np.float32)
    bias = (rng.standard_normal(40) * 0.3).astype(np.float32)
    ids, w = S.k3_router_f64(logits, bias, 7)
    sc = [1 / (1 + math.exp(-float(v))) for v in logits]
    order = sorted(range(40), key=lambda i: (-(sc[i] + float(bias[i])), i))[:7]
    assert ids.tolist() == order
    tot = sum(sc[i] for i in order)
    assert np.allclose(w, [sc[i] / (tot + 1e-20) for i in order], rtol=1e-14)
    forced = np.zeros(40, np.float32)
    forced[[5, 33, 17]] = np.float32(10.0)  # dominates any sigmoid difference
    ids, w = S.k3_router_f64(logits, forced, 3)
    assert sorted(ids.tolist()) == [5, 17, 33]
    assert np.isclose(w.sum(), 1.0, rtol=1e-14)
    ties = np.zeros(8, np.float32)
    ids, _ = S.k3_router_f64(ties, ties, 4)  # all equal: lower index first
    assert ids.tolist() == [0, 1, 2, 3]


def test_tiny_expert_layout_matches_raw_v1_offsets():
    import oracle
    span = S.tiny_expert_span(3)
    off = oracle.expert_offsets(32, 32)  # w1p, w1s, w2p, w2s, w3p, w3s, span
    assert span.size == off[-1]
    # expert 3, matrix 0, row 0: columns 0 and 1 -> one byte, scale 123 + 3
    assert span[off[0]] == S.tiny_test_code(3, 0, 0, 0) | (S.tiny_test_code(3, 0, 0, 1) << 4)
    assert span[off[1]] == 123 + 3
    assert span[off[3]] == 123 + (3 + 1) % 4 and span[off[5]] == 123 + (3 + 2) % 4


def _dense_block(m, hidden):
    """The fixture block as plain float64 matmuls, the experts decoded with
    ldexp (provider_moe_test.cpp:132-153, :193-264) -- an independent path."""
    e2m1 = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0]

    def decode(span, po, so, rows, cols):
        w = np.empty((rows, cols))
        for r in range(rows):
            for c in range(cols):
                b = int(span[po + r * (cols // 2) + c // 2])
                code = b & 15 if c % 2 == 0 else b >> 4
                v = e2m1[code & 7] * (-1.0 if code & 8 else 1.0)
                w[r, c] = math.ldexp(v, int(span[so + r * (cols // 32) + c // 32]) - 127)
        return w

    def dense(name):
        return m[name].astype(np.float64) * m[name + "_scales"].astype(np.float64)[:, None]

    def situ(g, u):
        return (np.tanh(g / 4) * 4 / (1 + np.exp(-g))) * (np.tanh(u / 25) * 25)

    p13, s13, p2, s2 = 512, 32, 512, 32
    experts = {}
    for e in range(16):
        sp = S.tiny_expert_span(e)
        experts[e] = (decode(sp, 0, p13, 32, 32), decode(sp, p13 + s13, p13 + s13 + p2, 32, 32),
                      decode(sp, p13 + s13 + p2 + s2, 2 * p13 + s13 + p2 + s2, 32, 32))
    outs = []
    for x in np.atleast_2d(hidden).astype(np.float64):
        scores = 1 / (1 + np.exp(-(dense("router") @ x)))
        choice = scores + m["router_bias"].astype(np.float64)
        ids = sorted(range(16), key=lambda i: (-choice[i], i))
        w = scores[ids] / (scores[ids].sum() + 1e-20)
        rin = dense("routed_down") @ x
        routed = np.zeros(32)
        for e, we in zip(ids, w):
            w1, w2, w3 = experts[e]
            routed += we * (w2 @ situ(w1 @ rin, w3 @ rin))
        norm = m["routed_norm"].astype(np.float64) * (routed / np.sqrt(np.mean(routed ** 2) +
                                                                     float(np.float32(1e-5))))
        shared = dense("shared_down") @ situ(dense("shared_gate") @ x, dense("shared_up") @ x)
        outs.append(dense("routed_up") @ norm + shared)
    return np.array(outs)


@pytest.mark.parametrize("positions", [1, 3])
def test_block_oracle_on_reference_tiny_fixture(positions):
    m = S.tiny_spine()
    hidden = S.tiny_hidden(positions)
    out, ids, w, _ = S.moe_block_f64("int8", m, S.tiny_expert_span, hidden, 32, 16)
    want = _dense_block(m, hidden)
    assert out.shape == (positions, 32) and ids.shape == (positions, 16)
    assert np.max(np.abs(out - want)) <= 1e-10 * max(1.0, np.max(np.abs(want)))
    assert sorted(ids[0].tolist()) == list(range(16))  # top 16 of 16: every expert


@pytest.mark.parametrize("kind", ["bf16", "int8"])
def test_block_oracle_magnitude(kind):
    """The per-element scale of the block bar: the magnitude of the terms the
    last two projections sum equals the same projections over |W| and |input|
    (pinned on the reference's tiny fixture with its own row-int8 spine, and a
    random BF16 one), and bounds the output from above."""
    if kind == "int8":
        m = S.tiny_spine()
    else:
        rng = np.random.default_rng(3)
        m = {}
        for name, (rows, cols) in {"router": (16, 32), "routed_down": (32, 32),
                                   "routed_up": (32, 32), "shared_gate": (64, 32),
                                   "shared_up": (64, 32), "shared_down": (32, 64)}.items():
            v = rng.standard_normal((rows, cols), dtype=np.float32)
            m[name] = (v.view(np.uint32) >> 16).astype(np.uint16)
        m["router_bias"] = np.zeros(16, np.float32)
        m["routed_norm"] = np.ones(32, np.float32)
    hidden = S.tiny_hidden(3)
    out, ids, w, routed, mag = S.moe_block_f64(kind, m, S.tiny_expert_span, hidden, 32, 16,
                                               with_mag=True)
    assert mag.shape == out.shape and np.all(mag >= np.abs(out) - 1e-12 * np.abs(out).max())
    for p in range(3):
        norm = S.rms_norm_f64(routed[p][None, :], m["routed_norm"], S.RMS_EPS)
        h = S.situ_f64(S._linear(kind, m, "shared_gate", hidden[p:p + 1]),
                       S._linear(kind, m, "shared_up", hidden[p:p + 1]))
        if kind == "bf16":
            dense = {n: np.abs(S.bf16_to_f32(m[n]).astype(np.float64)) for n in ("routed_up", "shared_down")}
        else:
            dense = {n: np.abs(m[n].astype(np.float64)) * np.abs(m[n + "_scales"].astype(np.float64))[:, None]
                     for n in ("routed_up", "shared_down")}
        want = dense["routed_up"] @ np.abs(norm[0]) + dense["shared_down"] @ np.abs(h[0])
        assert np.allclose(mag[p], want, rtol=1e-12, atol=0)


def test_moe_spine_validation_on_host():
    """MoeSpine checks every shape before any pointer reaches the library."""
    import torch
    from deltafin_amd import spine
    H, R, Sh, E = 64, 32, 48, 8

    def bf(r, c):
        return torch.zeros((r, c), dtype=torch.int16)
    args = dict(router=bf(E, H), router_bias=torch.zeros(E), routed_down=bf(R, H),
                routed_norm=torch.ones(R), routed_up=bf(H, R), shared_gate=bf(Sh, H),
                shared_up=bf(Sh, H), shared_down=bf(H, Sh))
    bad = dict(args, routed_up=bf(H, R + 1))
    with pytest.raises(ValueError, match="routed_up must be"):
        spine.MoeSpine("bf16", **bad)
    bad = dict(args, router_bias=torch.zeros(E + 1))
    with pytest.raises(ValueError, match="router_bias"):
        spine.MoeSpine("bf16", **bad)
    with pytest.raises(ValueError, match="device tensor"):
        spine.MoeSpine("bf16", **args)  # host tensors: refused, not passed on
    bad = dict(args, router=torch.zeros((E, H), dtype=torch.int8))
    with pytest.raises(ValueError):
        spine.MoeSpine("bf16", **bad)
