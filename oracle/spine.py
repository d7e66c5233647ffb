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

Pins (tests/test_oracle_spine.py): the BF16 decode against the closed-form
values of the sixteen fixture patterns and of IEEE special encodings; the GEMVs
against pure-Python loops on small shapes, linearity in x, one-hot columns and
the dense materialisation; the RMS norm against constant rows (closed form),
scale invariance and a hand-computed row.
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
    return np.asarray(x, dtype=np.float32).astype(np.float64) @ w.T


def spine_int8_f64(q: np.ndarray, scales: np.ndarray, x: np.ndarray) -> np.ndarray:
    """q int8 [rows, cols], scales float32 [rows], x float32 [positions, cols]
    -> float64 [positions, rows]."""
    dots = np.asarray(x, dtype=np.float32).astype(np.float64) @ np.asarray(q, np.int8).astype(
        np.float64).T
    return dots * np.asarray(scales, dtype=np.float32).astype(np.float64)[None, :]


def rms_norm_f64(x: np.ndarray, weight: np.ndarray, eps: float) -> np.ndarray:
    x64 = np.asarray(x, dtype=np.float32).astype(np.float64)
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
