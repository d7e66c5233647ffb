"""CPU oracle for the routed-expert MXFP4 path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use
this package, and only as the checker (or, for the reference library, as the
timed CPU baseline).  The product library never loads it.

Two native libraries back it:
  liborc.so            this repository's C restatement (oracle/orc.c); every
                       function cites the reference file:line it follows.
  _ref/libref_mxfp4.so the reference's own CPU kernels (tools/fused_gemv.c and
                       tools/fused_gemv_batch.c) compiled in place by
                       oracle/Makefile; used to pin the restatement and as the
                       CPU baseline.

Pins for each oracle function (tests/test_oracle.py):
  e2m1 / e8m0         closed form of the E2M1 encoding (exhaustive 16 codes) and
                      of E8M0 = 2^(s-127) (all 256 bytes)
  gemv_f32_lanes      bit-exact against the reference's mxfp4_gemv_compat and
                      mxfp4_gemv (AVX2) on random shapes
  gemv_f64            numpy float64 dense decode + matmul; linearity in x;
                      constant-code rows (closed-form sum); the reference KATs
                      (all 0x22 rows -> 32.0; the all-codes 2x32x2 KAT)
  act (SiTU/SiLU)     numpy closed forms
  expert_f64 (SiTU)   the reference's mxfp4_moe_expert_set within 2e-4 relative
  moe_layer_f64       numpy ordered weighted sum of expert_f64 outputs; the
                      reference mxfp4_moe_expert_set (SiTU) for the full set
  topk_softmax        numpy stable argsort / exp-normalise; NaN ranked as -inf
                      and -0 equal to +0 wherever they sit (the order the
                      reference leaves open for NaN, whose route it rejects)
  synth               numpy restatement in deltafin_amd/synth.py (bit-exact)
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ORC_PATH = HERE / "liborc.so"
REF_PATH = HERE / "_ref" / "libref_mxfp4.so"

ACT_SITU = 0
ACT_SILU = 1

_orc = None
_ref = None
_u8p = C.POINTER(C.c_uint8)
_f32p = C.POINTER(C.c_float)
_f64p = C.POINTER(C.c_double)
_u32p = C.POINTER(C.c_uint32)
_i32p = C.POINTER(C.c_int)


def build() -> None:
    """Compile liborc.so (and _ref when the reference sources are present)."""
    subprocess.run(["make", "-s", "-C", str(HERE), "all"], check=True)


def orc() -> C.CDLL:
    global _orc
    if _orc is None:
        if not ORC_PATH.exists():
            build()
        lib = C.CDLL(str(ORC_PATH))
        lib.orc_e2m1.restype = C.c_double
        lib.orc_e2m1.argtypes = [C.c_uint8]
        lib.orc_e8m0.restype = C.c_double
        lib.orc_e8m0.argtypes = [C.c_uint8]
        lib.orc_gemv_f64.argtypes = [_u8p, _u8p, _f64p, _f64p, C.c_int, C.c_int, C.c_int]
        lib.orc_gemv_f64_mag.argtypes = [_u8p, _u8p, _f64p, _f64p, _f64p, C.c_int, C.c_int]
        lib.orc_gemv_f32_lanes.argtypes = [_u8p, _u8p, _f32p, _f32p, C.c_int, C.c_int]
        lib.orc_act.restype = C.c_double
        lib.orc_act.argtypes = [C.c_int, C.c_double, C.c_double]
        lib.orc_expert_offsets.argtypes = [C.c_int, C.c_int, C.POINTER(C.c_uint64)]
        lib.orc_expert_f64.argtypes = [_u8p, C.c_int, C.c_int, C.c_int, _f64p, _f64p, _f64p, _f64p]
        lib.orc_moe_layer_f64.argtypes = [C.POINTER(_u8p), C.c_int, _f64p, C.c_int, C.c_int,
                                          C.c_int, _f64p, _f64p, _f64p]
        lib.orc_topk_softmax.restype = C.c_int
        lib.orc_topk_softmax.argtypes = [_f32p, C.c_int, C.c_int, _i32p, _f64p]
        for name in ("orc_scale4_pack", "orc_scale4_unpack"):
            getattr(lib, name).restype = C.c_int
            getattr(lib, name).argtypes = [_u8p, C.c_uint64, C.c_int, _u8p]
        lib.orc_scale4_header.restype = C.c_int
        lib.orc_scale4_header.argtypes = [_u8p, _u8p, _u8p]
        lib.orc_rand_u64.restype = C.c_uint64
        lib.orc_rand_u64.argtypes = [C.c_uint64, C.c_uint64, C.c_uint64]
        lib.orc_synth_mxfp4.argtypes = [C.c_uint64, C.c_uint64, _u8p, C.c_uint64, _u8p,
                                        C.c_uint64, C.c_int, C.c_int]
        lib.orc_synth_expert.argtypes = [C.c_uint64, C.c_uint64, C.c_int, C.c_int, _u8p, C.c_int,
                                         C.c_int]
        _orc = lib
    return _orc


def ref_available() -> bool:
    return REF_PATH.exists()


def ref() -> C.CDLL:
    """The reference's own CPU library (tools/fused_gemv*.c compiled in place)."""
    global _ref
    if _ref is None:
        if not REF_PATH.exists():
            raise FileNotFoundError(f"{REF_PATH} missing: run `make -C oracle ref` where the "
                                    "reference sources are present")
        lib = C.CDLL(str(REF_PATH))
        for name in ("mxfp4_gemv", "mxfp4_gemv_compat"):
            getattr(lib, name).argtypes = [_u8p, _u8p, _f32p, _f32p, C.c_int, C.c_int]
        for name in ("mxfp4_gemv_mt", "mxfp4_gemv_mt_compat"):
            getattr(lib, name).argtypes = [_u8p, _u8p, _f32p, _f32p, C.c_int, C.c_int, C.c_int]
        lib.mxfp4_gemv_mt_scale4.argtypes = [_u8p, _u8p, _u32p, _f32p, _f32p, C.c_int, C.c_int,
                                             C.c_int]
        lib.mxfp4_have_avx2.restype = C.c_int
        lib.mxfp4_cpu_compatible.restype = C.c_int
        lib.mxfp4_pool_init.restype = C.c_int
        lib.mxfp4_pool_init.argtypes = [C.c_int]
        lib.mxfp4_gemv_batch.argtypes = [C.POINTER(_u8p), C.POINTER(_u8p), C.POINTER(_f32p),
                                         C.POINTER(_f32p), _i32p, _i32p, C.c_int, C.c_int]
        lib.mxfp4_moe_layer.argtypes = [C.POINTER(_u8p), C.POINTER(_u8p), _i32p, _i32p, C.c_int,
                                        _f32p, _f32p, C.c_int]
        lib.mxfp4_moe_expert_set.argtypes = [C.POINTER(_u8p), C.POINTER(_u8p), C.POINTER(_u8p),
                                             C.POINTER(_u8p), _f32p, _f32p, C.c_int, C.c_int,
                                             C.c_int, _f32p, _f32p, C.c_int]
        _ref = lib
    return _ref


def _p(a: np.ndarray, t):
    return a.ctypes.data_as(t)


def _u8(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.uint8)


# ------------------------------------------------------------------ oracle wrappers
def e2m1(code: int) -> float:
    return orc().orc_e2m1(code)


def e8m0(s: int) -> float:
    return orc().orc_e8m0(s)


def gemv_f64(packed, scales, x, rows: int, cols: int, nan_on_255: bool = True,
             with_mag: bool = False):
    p, s = _u8(packed), _u8(scales)
    xd = np.ascontiguousarray(x, dtype=np.float64)
    y = np.empty(rows, dtype=np.float64)
    if with_mag:
        mag = np.empty(rows, dtype=np.float64)
        orc().orc_gemv_f64_mag(_p(p, _u8p), _p(s, _u8p), _p(xd, _f64p), _p(y, _f64p),
                               _p(mag, _f64p), rows, cols)
        return y, mag
    orc().orc_gemv_f64(_p(p, _u8p), _p(s, _u8p), _p(xd, _f64p), _p(y, _f64p), rows, cols,
                       1 if nan_on_255 else 0)
    return y


def gemv_f32_lanes(packed, scales, x, rows: int, cols: int) -> np.ndarray:
    p, s = _u8(packed), _u8(scales)
    xf = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(rows, dtype=np.float32)
    orc().orc_gemv_f32_lanes(_p(p, _u8p), _p(s, _u8p), _p(xf, _f32p), _p(y, _f32p), rows, cols)
    return y


def act(kind: int, g: float, u: float) -> float:
    return orc().orc_act(kind, g, u)


def expert_offsets(hidden: int, inter: int) -> list[int]:
    off = (C.c_uint64 * 7)()
    orc().orc_expert_offsets(hidden, inter, off)
    return list(off)


def expert_f64(span, hidden: int, inter: int, kind: int, x):
    sp = _u8(span)
    xd = np.ascontiguousarray(x, dtype=np.float64)
    y = np.empty(hidden, dtype=np.float64)
    h = np.empty(inter, dtype=np.float64)
    mag = np.empty(hidden, dtype=np.float64)
    orc().orc_expert_f64(_p(sp, _u8p), hidden, inter, kind, _p(xd, _f64p), _p(y, _f64p),
                         _p(h, _f64p), _p(mag, _f64p))
    return y, h, mag


def moe_layer_f64(spans, weights, hidden: int, inter: int, kind: int, x):
    """Returns (out, mag) for out = sum_e w_e expert_e(x) in route order."""
    arrs = [_u8(s) for s in spans]
    ptrs = (_u8p * max(len(arrs), 1))(*[_p(a, _u8p) for a in arrs])
    w = np.ascontiguousarray(weights, dtype=np.float64)
    xd = np.ascontiguousarray(x, dtype=np.float64)
    out = np.empty(hidden, dtype=np.float64)
    mag = np.empty(hidden, dtype=np.float64)
    orc().orc_moe_layer_f64(ptrs, len(arrs), _p(w, _f64p), hidden, inter, kind, _p(xd, _f64p),
                            _p(out, _f64p), _p(mag, _f64p))
    return out, mag


def topk_softmax(logits, k: int):
    lg = np.ascontiguousarray(logits, dtype=np.float32)
    ids = np.empty(k, dtype=np.int32)
    w = np.empty(k, dtype=np.float64)
    if orc().orc_topk_softmax(_p(lg, _f32p), lg.size, k, _p(ids, _i32p), _p(w, _f64p)) != 0:
        raise ValueError("invalid top-k arguments")
    return ids, w


def rand_u64(seed: int, stream: int, index: int) -> int:
    return orc().orc_rand_u64(seed, stream, index)


def synth_mxfp4(seed: int, stream: int, n_packed: int, n_scales: int, lo: int = 119,
                hi: int = 127):
    p = np.empty(n_packed, dtype=np.uint8)
    s = np.empty(n_scales, dtype=np.uint8)
    orc().orc_synth_mxfp4(seed, stream, _p(p, _u8p), n_packed, _p(s, _u8p), n_scales, lo, hi)
    return p, s


def synth_expert(seed: int, expert: int, hidden: int, inter: int, lo: int = 119,
                 hi: int = 127) -> np.ndarray:
    span = np.empty(expert_offsets(hidden, inter)[6], dtype=np.uint8)
    orc().orc_synth_expert(seed, expert, hidden, inter, _p(span, _u8p), lo, hi)
    return span


# ------------------------------------------------------------------ reference wrappers
def ref_gemv(packed, scales, x, rows: int, cols: int, variant: str = "auto",
             threads: int = 1) -> np.ndarray:
    """The reference's mxfp4_gemv (variant auto|compat) or _mt."""
    p, s = _u8(packed), _u8(scales)
    xf = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(rows, dtype=np.float32)
    lib = ref()
    args = (_p(p, _u8p), _p(s, _u8p), _p(xf, _f32p), _p(y, _f32p), rows, cols)
    if threads > 1:
        (lib.mxfp4_gemv_mt if variant == "auto" else lib.mxfp4_gemv_mt_compat)(*args, threads)
    else:
        (lib.mxfp4_gemv if variant == "auto" else lib.mxfp4_gemv_compat)(*args)
    return y


def ref_expert_set(spans, weights, x, hidden: int, inter: int, threads: int = 4) -> np.ndarray:
    """The reference's whole-set SiTU call (tools/fused_gemv_batch.c:465-518)."""
    off = expert_offsets(hidden, inter)
    arrs = [_u8(s) for s in spans]
    n = len(arrs)
    p13 = (_u8p * (2 * n))()
    s13 = (_u8p * (2 * n))()
    p2 = (_u8p * n)()
    s2 = (_u8p * n)()
    for e, a in enumerate(arrs):
        base = a.ctypes.data
        p13[2 * e] = C.cast(base + off[0], _u8p)
        s13[2 * e] = C.cast(base + off[1], _u8p)
        p13[2 * e + 1] = C.cast(base + off[4], _u8p)
        s13[2 * e + 1] = C.cast(base + off[5], _u8p)
        p2[e] = C.cast(base + off[2], _u8p)
        s2[e] = C.cast(base + off[3], _u8p)
    w = np.ascontiguousarray(weights, dtype=np.float32)
    xf = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(hidden, dtype=np.float32)
    ref().mxfp4_moe_expert_set(p13, s13, p2, s2, _p(xf, _f32p), _p(w, _f32p), n, inter, hidden,
                               None, _p(out, _f32p), threads)
    return out


# ------------------------------------------------------------------ parity metrics
def cond_rel_err(y, ref_y, mag, n_terms: int) -> float:
    """max_i |y_i - ref_i| / max(|ref_i|, mag_i / sqrt(n_terms)).

    mag_i = sum of |terms| of output i, so mag_i / sqrt(n) is the size of a
    typical output of that row's term distribution; outputs that cancel to
    near zero are measured against it instead of against themselves.
    """
    y = np.asarray(y, dtype=np.float64)
    r = np.asarray(ref_y, dtype=np.float64)
    m = np.asarray(mag, dtype=np.float64)
    den = np.maximum(np.abs(r), m / np.sqrt(float(n_terms)))
    den = np.maximum(den, 1e-300)
    return float(np.max(np.abs(y - r) / den))


def plain_max_rel(y, ref_y, floor: float = 1e-6) -> float:
    """The reference harness metric (tools/fused_gemv.c:1083-1092)."""
    y = np.asarray(y, dtype=np.float64)
    r = np.asarray(ref_y, dtype=np.float64)
    return float(np.max(np.abs(y - r) / np.maximum(np.abs(r), floor)))


# ------------------------------------------------------------------ scale4-v2
# K3 geometry constants of the format (native/deltafin/src/expert_scale4.rs:17-63).
SCALE4_HEADER_BYTES = 8192
SCALE4_SPAN = 17_039_360
SCALE4_K3 = (3584, 3072)


def scale4_pack(values, base: int | None = None) -> tuple[int, np.ndarray]:
    """(base, packed) of a scale plane; base defaults to the plane's minimum
    (expert_scale4.rs:114-148).  Raises ValueError when it does not fit."""
    v = _u8(values)
    b = int(v.min()) if base is None else int(base)
    out = np.empty((v.size + 1) // 2, dtype=np.uint8)
    if orc().orc_scale4_pack(_p(v, _u8p), v.size, b, _p(out, _u8p)) != 0:
        raise ValueError(f"scale plane does not fit base {b} plus a 4-bit index")
    return b, out


def scale4_unpack(packed, base: int, n: int) -> np.ndarray:
    pk = _u8(packed)
    if pk.size != (n + 1) // 2:
        raise ValueError("packed length does not match the value count")
    out = np.empty(n, dtype=np.uint8)
    if orc().orc_scale4_unpack(_p(pk, _u8p), n, int(base), _p(out, _u8p)) != 0:
        raise ValueError(f"base {base} exceeds 240")
    return out


def scale4_header(digest: bytes, bases) -> np.ndarray:
    d = _u8(np.frombuffer(bytes(digest), dtype=np.uint8))
    b = _u8(bases)
    if d.size != 32 or b.size != 3:
        raise ValueError("digest is 32 bytes and bases 3")
    out = np.empty(SCALE4_HEADER_BYTES, dtype=np.uint8)
    if orc().orc_scale4_header(_p(d, _u8p), _p(b, _u8p), _p(out, _u8p)) != 0:
        raise ValueError("a base exceeds 240")
    return out


def scale4_span(raw_span, digest: bytes = bytes(32)) -> np.ndarray:
    """The assembled scale4-v2 span of a raw-v1 K3 span: header, then w1
    packed, w1 indices, w2 packed, w2 indices, w3 packed, w3 indices, each
    matrix's base the minimum of its scale plane (tools/metal_moe.mm:127-155)."""
    raw = _u8(raw_span)
    off = expert_offsets(*SCALE4_K3)
    if raw.size != off[6]:
        raise ValueError("not a raw-v1 K3 span")
    bases, parts = [], []
    for m in range(3):
        p0, s0, s1 = off[2 * m], off[2 * m + 1], off[2 * m + 2]
        b, pk = scale4_pack(raw[s0:s1])
        bases.append(b)
        parts += [raw[p0:s0], pk]
    return np.concatenate([scale4_header(digest, bases)] + parts)


def scale4_to_raw(span4) -> np.ndarray:
    """Inverse of scale4_span (the indices expanded to E8M0 bytes)."""
    s4 = _u8(span4)
    off = expert_offsets(*SCALE4_K3)
    bases = [int(s4[64 + m]) for m in range(3)]
    parts, pos = [], SCALE4_HEADER_BYTES
    for m in range(3):
        n_packed = off[2 * m + 1] - off[2 * m]
        n_scales = off[2 * m + 2] - off[2 * m + 1]
        parts.append(s4[pos:pos + n_packed])
        pos += n_packed
        parts.append(scale4_unpack(s4[pos:pos + (n_scales + 1) // 2], bases[m], n_scales))
        pos += (n_scales + 1) // 2
    return np.concatenate(parts)


def ref_gemv_scale4(packed, scales4, base: int, x, rows: int, cols: int, threads: int = 1):
    """The reference's mxfp4_gemv_mt_scale4 (tools/fused_gemv.c:1059-1071) with
    the 16-entry table of E8M0 float bits (base + d) << 23."""
    lib = ref()
    table = np.array([(base + d) << 23 for d in range(16)], dtype=np.uint32)
    xs = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(rows, dtype=np.float32)
    lib.mxfp4_gemv_mt_scale4(_p(_u8(packed), _u8p), _p(_u8(scales4), _u8p), _p(table, _u32p),
                             _p(xs, _f32p), _p(y, _f32p), rows, cols, threads)
    return y
