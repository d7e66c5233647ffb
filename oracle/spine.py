"""CPU oracle for the spine projections -- TEST INFRASTRUCTURE ONLY.

Only tests/ and bench.py's cpu_baseline leg use this module, as the checker.
The product library never loads it.

Restates, in float64 numpy:
  bf16_to_f32_bits   the exact BF16 widening `uint32(bits) << 16`
                     (native/provider_gate/provider_spine_bf16_cuda.cu:60-62,
                     :280-303 decode_bits)
  spine_bf16_f64     out[p, r] = sum_c bf16(W[r, c]) * x[p, c] in float64, the
                     expected value of the reference's RAW_BF16 gate
                     (provider_spine_bf16_cuda_test.cpp:264-275)
  spine_int8_f64     out[p, r] = s[r] * sum_c q[r, c] * x[p, c]
                     (at::_weight_int8pack_mm in row_int8_linear,
                     provider_moe.cpp:507-516; materialize_row_int8 :496-505
                     gives the dense form q * s[:, None])
  rms_norm_f64       weight * (x / sqrt(mean(x^2) + eps)) (provider_moe.cpp:535-542)
  spine_fixture      the reference gate's deterministic matrix fixture
                     (provider_spine_bf16_cuda_test.cpp:235-276)
  k3_router_f64      top-k of sigmoid(logits) + bias, weights = the selected
                     sigmoids over their sum + 1e-20 (prepare_moe_t1,
                     provider_moe.cpp:1673-1683); descending, lower index on ties
  moe_block_f64      the whole K3 MoE block (prepare_moe_t1 + the routed expert
                     set + complete_moe_t1, provider_moe.cpp:1660-1700,
                     :1970-2014) in float64, the experts through oracle's
                     moe_layer_f64 (SiTU)
  tiny_fixture       the reference's tiny-geometry MoE fixture
                     (provider_moe_test.cpp:50-191: make_row_int8, make_spine,
                     test_code / encode_expert)

Pins (tests/test_oracle_spine.py): the BF16 decode against the closed-form
values of the sixteen fixture patterns and of IEEE special encodings; the GEMVs
against pure-Python loops on small shapes, linearity in x, one-hot columns and
the dense materialisation; the RMS norm against constant rows (closed form),
scale invariance and a hand-computed row; the K3 router against the pinned
top-k of the logits (zero bias: sigmoid is monotone), a pure-Python sort and
forced selections; the block, on the reference's tiny fixture, against an
independent dense float64 composition (the fixture's experts decoded with
ldexp as provider_moe_test.cpp:132-153 does, every step a plain matmul).
"""
from __future__ import annotations

import numpy as np

# The sixteen finite BF16 patterns of the reference gate's fixture
# (provider_spine_bf16_cuda_test.cpp:238-240).
FIXTURE_PATTERNS = np.array(
    [0x0000, 0x0001, 0x007F, 0x0080, 0x3D00, 0x3E80, 0x3F00, 0x3F80,
     0x4000, 0x4040, 0x4080, 0x8000, 0xBD00, 0xBE80, 0xBF00, 0xBF80], dtype=np.uint16)

SPINE_TOLERANCE_ABS = 2.0e-5   # provider_spine_bf16_cuda_test.cpp:307-308
SPINE_TOLERANCE_REL = 2.0e-5


def bf16_to_f32_bits(bits: np.ndarray) -> np.ndarray:
    """uint16 BF16 bits -> uint32 fp32 bits (bits << 16)."""
    return np.asarray(bits, dtype=np.uint16).astype(np.uint32) << np.uint32(16)


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return bf16_to_f32_bits(bits).view(np.float32)


def spine_bf16_f64(weights: np.ndarray, x: np.ndarray) -> np.ndarray:
    """weights uint16 [rows, cols], x float32 [positions, cols] -> float64
    [positions, rows]."""
    w = bf16_to_f32(weights).astype(np.float64)
    return np.asarray(x, dtype=np.float64) @ w.T


def spine_int8_f64(q: np.ndarray, scales: np.ndarray, x: np.ndarray) -> np.ndarray:
    """q int8 [rows, cols], scales float32 [rows], x float32 [positions, cols]
    -> float64 [positions, rows]."""
    dots = np.asarray(x, dtype=np.float64) @ np.asarray(q, np.int8).astype(np.float64).T
    return dots * np.asarray(scales, dtype=np.float32).astype(np.float64)[None, :]


def rms_norm_f64(x: np.ndarray, weight: np.ndarray, eps: float) -> np.ndarray:
    x64 = np.asarray(x, dtype=np.float64)
    var = np.mean(x64 * x64, axis=-1, keepdims=True)
    return np.asarray(weight, np.float32).astype(np.float64) * (x64 / np.sqrt(var + np.float64(
        np.float32(eps))))


def spine_fixture(rows: int, cols: int, salt: int):
    """(weights uint16 [rows, cols], activation float32 [cols], expected float32
    [rows]) of the reference gate's make_matrix."""
    index = np.arange(rows * cols, dtype=np.int64)
    weights = FIXTURE_PATTERNS[(index * 13 + salt) % 16].reshape(rows, cols)
    c = np.arange(cols, dtype=np.int64)
    activation = (((c + salt) % 29 - 14).astype(np.float32) / np.float32(31.0)).astype(np.float32)
    expected = spine_bf16_f64(weights, activation[None, :])[0].astype(np.float32)
    return weights, activation, expected


def spine_close(found: np.ndarray, expected: np.ndarray) -> bool:
    """The reference gate's bound: |found - expected| <= 2e-5 + 2e-5 |expected|,
    and found finite."""
    found = np.asarray(found, np.float64)
    expected = np.asarray(expected, np.float64)
    tol = SPINE_TOLERANCE_ABS + SPINE_TOLERANCE_REL * np.abs(expected)
    return bool(np.all(np.isfinite(found)) and np.all(np.abs(found - expected) <= tol))


# ------------------------------------------------------------ the K3 MoE block

SITU_BETA = 4.0           # kSituBeta, provider_moe.cpp:85
SITU_LINEAR_BETA = 25.0   # kSituLinearBeta, :86
RMS_EPS = 1.0e-5          # kRmsEpsilon, :87


def sigmoid_f64(v):
    return 1.0 / (1.0 + np.exp(-np.asarray(v, np.float64)))


def situ_f64(g, u):
    """[4 tanh(g/4) sigmoid(g)] [25 tanh(u/25)] (provider_moe.cpp:524-533)."""
    g = np.asarray(g, np.float64)
    u = np.asarray(u, np.float64)
    return (np.tanh(g / SITU_BETA) * SITU_BETA * sigmoid_f64(g)) * (
        np.tanh(u / SITU_LINEAR_BETA) * SITU_LINEAR_BETA)


def k3_router_f64(logits, bias, k: int):
    """(ids int32 [k], weights float64 [k]) for one position."""
    scores = sigmoid_f64(logits)
    choice = scores + np.asarray(bias, np.float64)
    order = np.lexsort((np.arange(choice.size), -choice))  # descending, lower index first
    ids = order[:k].astype(np.int32)
    sel = scores[ids]
    return ids, sel / (sel.sum() + 1e-20)


def _linear(kind: str, m: dict, name: str, x):
    if kind == "bf16":
        return spine_bf16_f64(m[name], x)
    return spine_int8_f64(m[name], m[name + "_scales"], x)


def _linear_abs(kind: str, m: dict, name: str, x):
    """sum_j |W[i, j] x[j]|: the size of the terms each output sums."""
    ax = np.abs(np.asarray(x, np.float64))
    if kind == "bf16":
        return ax @ np.abs(bf16_to_f32(m[name]).astype(np.float64)).T
    dots = ax @ np.abs(np.asarray(m[name], np.int8).astype(np.float64)).T
    return dots * np.abs(np.asarray(m[name + "_scales"], np.float32).astype(np.float64))[None, :]


def moe_block_f64(kind: str, m: dict, expert_span, hidden, inter: int, k: int,
                  with_mag: bool = False):
    """The K3 block for hidden [P, H]; m holds the spine as numpy arrays
    (router, router_bias, routed_down, routed_norm, routed_up, shared_gate,
    shared_up, shared_down, and *_scales for kind "int8"); expert_span(id)
    returns that expert's raw-v1 bytes.  Returns (out [P, H], ids [P, k],
    weights [P, k], routed [P, R]) in float64; with_mag also the size of the
    terms each output sums, [P, H]: sum_j |routed_up[i, j] norm_j| +
    sum_j |shared_down[i, j] h_j| (the scale of a condition-aware bar,
    oracle.cond_rel_err with n = R + shared)."""
    import oracle
    x = np.atleast_2d(np.asarray(hidden, np.float64))
    R = m["routed_down"].shape[0]
    outs, all_ids, all_w, routed_all, mags = [], [], [], [], []
    for p in range(x.shape[0]):
        xp = x[p:p + 1]
        logits = _linear(kind, m, "router", xp)[0]
        ids, w = k3_router_f64(logits, m["router_bias"], k)
        routed_in = _linear(kind, m, "routed_down", xp)[0]
        routed, _ = oracle.moe_layer_f64([expert_span(int(e)) for e in ids], w, R, inter,
                                         oracle.ACT_SITU, routed_in)
        norm = rms_norm_f64(routed[None, :], m["routed_norm"], RMS_EPS)
        routed_full = _linear(kind, m, "routed_up", norm)[0]
        h = situ_f64(_linear(kind, m, "shared_gate", xp), _linear(kind, m, "shared_up", xp))
        shared = _linear(kind, m, "shared_down", h)[0]
        outs.append(routed_full + shared)
        all_ids.append(ids)
        all_w.append(w)
        routed_all.append(routed)
        if with_mag:
            mags.append(_linear_abs(kind, m, "routed_up", norm)[0] +
                        _linear_abs(kind, m, "shared_down", h)[0])
    res = (np.array(outs), np.array(all_ids), np.array(all_w), np.array(routed_all))
    return res + (np.array(mags),) if with_mag else res


# The reference's tiny MoE geometry (kTestGeometry, provider_moe_test.cpp:50):
# hidden, routed_hidden, intermediate, experts, shared_intermediate.
TINY = dict(hidden=32, routed_hidden=32, intermediate=32, experts=16, shared_intermediate=64)


def row_int8_fixture(rows: int, cols: int, seed: int):
    """make_row_int8 (provider_moe_test.cpp:155-174): (q int8, scales float32)."""
    r = np.arange(rows, dtype=np.int64)[:, None]
    c = np.arange(cols, dtype=np.int64)[None, :]
    q = (((r * 3 + c * 5 + seed * 7) % 9) - 4).astype(np.int8)
    s = ((1 + (np.arange(rows) + seed) % 3).astype(np.float32) / np.float32(64.0))
    return q, s


def tiny_spine() -> dict:
    """make_spine (provider_moe_test.cpp:176-191) as numpy arrays."""
    m = {}
    for name, (rows, cols, seed) in {
            "router": (16, 32, 1), "routed_down": (32, 32, 2), "routed_up": (32, 32, 3),
            "shared_gate": (64, 32, 4), "shared_up": (64, 32, 5),
            "shared_down": (32, 64, 6)}.items():
        m[name], m[name + "_scales"] = row_int8_fixture(rows, cols, seed)
    m["router_bias"] = (np.arange(16, dtype=np.float32) * np.float32(1.0 / 4096.0))
    m["routed_norm"] = np.linspace(0.75, 1.25, 32, dtype=np.float64).astype(np.float32)
    return m


def tiny_test_code(expert: int, matrix: int, row: int, column: int) -> int:
    """test_code (provider_moe_test.cpp:98-106)."""
    mag = 1 + ((expert * 3 + matrix * 5 + row * 7 + column * 11) % 4)
    if (expert + matrix + row + column) & 1:
        mag |= 8
    return mag


def tiny_expert_span(expert: int, hidden: int = 32, inter: int = 32) -> np.ndarray:
    """encode_expert (provider_moe_test.cpp:108-130) over the raw-v1 layout of
    (routed_hidden, intermediate) = (hidden, inter): w1 [I, H], w2 [H, I],
    w3 [I, H], each packed (low nibble = even column) then its E8M0 scales."""
    p13, s13 = inter * hidden // 2, inter * hidden // 32
    p2, s2 = hidden * inter // 2, hidden * inter // 32
    layouts = [(0, p13, inter, hidden), (p13 + s13, p13 + s13 + p2, hidden, inter),
               (p13 + s13 + p2 + s2, p13 + s13 + p2 + s2 + p13, inter, hidden)]
    span = np.zeros(2 * (p13 + s13) + p2 + s2, np.uint8)
    for mat, (po, so, rows, cols) in enumerate(layouts):
        for r in range(rows):
            for c in range(0, cols, 2):
                lo = tiny_test_code(expert, mat, r, c)
                hi = tiny_test_code(expert, mat, r, c + 1)
                span[po + r * (cols // 2) + c // 2] = lo | (hi << 4)
            for gi in range(cols // 32):
                span[so + r * (cols // 32) + gi] = 123 + ((expert + mat + r + gi) % 4)
    return span


def tiny_hidden(positions: int) -> np.ndarray:
    """The fixture's hidden rows: linspace(-0.25, 0.375, 32) for one position
    (parity_test, :275-277), linspace(-0.375, 0.625, 3 * 32) for three
    (position_prepare_complete_parity_test, :299-302)."""
    if positions == 1:
        return np.linspace(-0.25, 0.375, 32, dtype=np.float64).astype(np.float32)[None, :]
    if positions == 3:
        return np.linspace(-0.375, 0.625, 96, dtype=np.float64).astype(np.float32).reshape(3, 32)
    raise ValueError("the reference fixture has 1 or 3 positions")
