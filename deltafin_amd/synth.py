"""Host-side synthetic inputs from the counter-based generator the kernels use.

Draw i of stream s under seed k is mix64(key(k, s) + (i + 1) * golden), with
key(k, s) = mix64(k ^ mix64(s ^ 0xD1B54A32D192ED03)) and mix64 the SplitMix64
finaliser.  Packed MXFP4 bytes are the little-endian bytes of consecutive draws
(stream 2m); scale bytes are lo + draw mod (hi - lo + 1) (stream 2m + 1); expert
e's matrices w1, w2, w3 use m = 3e, 3e + 1, 3e + 2.  Normal values use
Box-Muller on two 53-bit uniforms in fp64, rounded to fp32.
"""
from __future__ import annotations

import numpy as np

_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)
_GOLD = np.uint64(0x9E3779B97F4A7C15)
_SKEY = np.uint64(0xD1B54A32D192ED03)


def _mix64(z: np.ndarray) -> np.ndarray:
    z = np.asarray(z, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def key(seed: int, stream: int) -> np.uint64:
    s = np.uint64(stream)
    return _mix64(np.uint64(seed) ^ _mix64(s ^ _SKEY))


def draws(seed: int, stream: int, start: int, count: int) -> np.ndarray:
    k = key(seed, stream)
    idx = np.arange(start + 1, start + count + 1, dtype=np.uint64)
    with np.errstate(over="ignore"):
        return _mix64(k + idx * _GOLD)


def mxfp4_planes(seed: int, stream: int, n_packed: int, n_scales: int, lo: int = 119,
                 hi: int = 127) -> tuple[np.ndarray, np.ndarray]:
    words = draws(seed, 2 * stream, 0, (n_packed + 7) // 8)
    packed = words.view(np.uint8)[:n_packed].copy()
    s = draws(seed, 2 * stream + 1, 0, n_scales)
    scales = (np.uint64(lo) + s % np.uint64(hi - lo + 1)).astype(np.uint8)
    return packed, scales


def span_offsets(hidden: int, inter: int) -> list[int]:
    w13p, w13s = inter * hidden // 2, inter * (hidden // 32)
    w2p, w2s = hidden * inter // 2, hidden * (inter // 32)
    off = [0, w13p]
    off.append(off[1] + w13s)
    off.append(off[2] + w2p)
    off.append(off[3] + w2s)
    off.append(off[4] + w13p)
    off.append(off[5] + w13s)
    return off


def expert_span(seed: int, expert: int, hidden: int, inter: int, lo: int = 119,
                hi: int = 127) -> np.ndarray:
    off = span_offsets(hidden, inter)
    out = np.empty(off[6], dtype=np.uint8)
    for m, (p0, s0, p1) in enumerate([(0, 1, 2), (2, 3, 4), (4, 5, 6)]):
        pk, sc = mxfp4_planes(seed, 3 * expert + m, off[s0] - off[p0], off[p1] - off[s0], lo, hi)
        out[off[p0]:off[s0]] = pk
        out[off[s0]:off[p1]] = sc
    return out


def normal(seed: int, stream: int, n: int) -> np.ndarray:
    d = draws(seed, stream, 0, 2 * n)
    u1 = ((d[0::2] >> np.uint64(11)).astype(np.float64) + 1.0) * 2.0 ** -53
    u2 = (d[1::2] >> np.uint64(11)).astype(np.float64) * 2.0 ** -53
    return (np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)).astype(np.float32)


def to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even fp32 -> bf16 bit patterns (uint16)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + np.uint64(0x7FFF) + ((u >> np.uint64(16)) & np.uint64(1))) >> np.uint64(16))
    return r.astype(np.uint16)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint32) << np.uint32(16)).view(np.float32)
