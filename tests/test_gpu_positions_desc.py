"""The descriptor surface's positions call over raw-v1 spans
(k3_hip_moe_positions_desc_v1, the k3_metal_moe_positions_desc_v1 drop-in,
tools/metal_moe.mm:852-1021) against the fp64 oracle on every verify path.

The call takes host fp32 activations [positions, hidden] and a
position_offsets partition of the edges.  Its raw-v1 spans go through the same
path selection as k3_hip_moe_verify_device (k3_hip_set_verify_mode): AUTO picks
the matrix-core union path when the unique experts are at most 92 % of the
edges (here 6 of 14), and the matrix-core, VALU-union and per-position paths
are also forced one by one.  The route repeats experts across positions and
inside one position, and has an empty position (a zero row).  Host blobs
(staged into the library's HBM cache) and device blobs (used in place) must
give the same rows.
"""
import ctypes as C

import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu

TOL = 1e-3
H, I = 3584, 3072
EDGES = [0, 1, 2, 3, 4, 2, 5, 0, 4, 1, 3, 3, 5, 3]
OFFS = [0, 5, 5, 11, 14]


def say(msg):
    print(f"[gpu-case] {msg}", flush=True)


def _weights(n, seed):
    lg = np.random.default_rng(seed).standard_normal(n)
    w = np.exp(lg - lg.max())
    return (w / w.sum()).astype(np.float32)


@pytest.fixture(scope="module")
def case(gpu):
    from deltafin_amd import _lib, moe
    g = moe.preset(1)
    assert gpu.k3_hip_configure_v1(C.byref(g)) == 0, _lib.last_error()
    raw = [oracle.synth_expert(71, e, H, I) for e in range(6)]
    w = np.concatenate([_weights(OFFS[p + 1] - OFFS[p], 10 + p) if OFFS[p + 1] > OFFS[p]
                        else np.zeros(0, np.float32) for p in range(len(OFFS) - 1)])
    x = np.random.default_rng(72).standard_normal((len(OFFS) - 1, H)).astype(np.float32)
    refs = []
    for p in range(len(OFFS) - 1):
        sl = slice(OFFS[p], OFFS[p + 1])
        if OFFS[p + 1] == OFFS[p]:
            refs.append(None)
            continue
        refs.append(oracle.moe_layer_f64([raw[e] for e in EDGES[sl]], w[sl].astype(np.float64),
                                         H, I, g.activation, x[p]))
    return g, raw, w, x, refs


def _check(out, refs):
    for p, r in enumerate(refs):
        if r is None:
            assert np.all(out[p] == 0), f"position {p} (no edges) must be a zero row"
            continue
        err = oracle.cond_rel_err(out[p], r[0], r[1], I)
        assert err <= TOL, f"position {p}: cond rel err {err:.3e}"


@pytest.mark.parametrize("mode", ["auto", "union_mfma", "union_valu", "positions"])
def test_positions_desc_raw_v1_paths(gpu, case, mode):
    from deltafin_amd import _lib, moe
    g, raw, w, x, refs = case
    code = {"auto": _lib.VERIFY_AUTO, "union_mfma": _lib.VERIFY_UNION_MFMA,
            "union_valu": _lib.VERIFY_UNION_VALU, "positions": _lib.VERIFY_POSITIONS}[mode]
    say(f"positions_desc raw-v1, mode {mode}, {len(EDGES)} edges over {len(OFFS) - 1} positions")
    prev = _lib.set_verify_mode(code)
    try:
        out = moe.moe_positions_desc([raw[e] for e in EDGES], OFFS, w, x)
    finally:
        _lib.set_verify_mode(prev)
    _check(out, refs)


def test_positions_desc_raw_v1_device_blobs(gpu, case):
    """Device-resident raw-v1 blobs on the default path equal the host-blob call."""
    import torch
    from deltafin_amd import _lib, moe
    g, raw, w, x, refs = case
    say("positions_desc raw-v1, device blobs, AUTO")
    dev = [torch.from_numpy(r).cuda() for r in raw]
    torch.cuda.synchronize()
    prev = _lib.set_verify_mode(_lib.VERIFY_AUTO)
    try:
        a = moe.moe_positions_desc([raw[e] for e in EDGES], OFFS, w, x)
        b = moe.moe_positions_desc([dev[e] for e in EDGES], OFFS, w, x)
    finally:
        _lib.set_verify_mode(prev)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    _check(b, refs)


@pytest.mark.parametrize("mode", ["auto", "positions"])
def test_positions_flat_desc_raw_v1(gpu, case, mode):
    """k3_hip_moe_positions_flat_desc_v1 (k3_metal_moe_positions_flat_desc_v1,
    tools/metal_moe.mm:1231-1243): the same rows as the positions call.  Under
    the per-position mode these positions (edge counts 5, 0, 6, 3: no single
    position batch) run on the union kernels instead, one dispatch sequence."""
    from deltafin_amd import _lib, moe
    g, raw, w, x, refs = case
    code = _lib.VERIFY_AUTO if mode == "auto" else _lib.VERIFY_POSITIONS
    say(f"positions_flat_desc raw-v1, mode {mode}")
    prev = _lib.set_verify_mode(code)
    try:
        out = moe.moe_positions_desc([raw[e] for e in EDGES], OFFS, w, x, flat=True)
    finally:
        _lib.set_verify_mode(prev)
    _check(out, refs)


def test_positions_flat_raw_pointer_form(gpu, case):
    """k3_hip_moe_positions_flat (k3_metal_moe_positions_flat, the raw-pointer
    form the provider binds first): host spans of the configured geometry."""
    from deltafin_amd import _lib
    g, raw, w, x, refs = case
    say("positions_flat raw pointers")
    lib = _lib.load()
    blobs = (C.c_void_p * len(EDGES))(*[raw[e].ctypes.data for e in EDGES])
    offs = (C.c_int * len(OFFS))(*OFFS)
    xs = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty((len(OFFS) - 1, H), dtype=np.float32)
    rc = lib.k3_hip_moe_positions_flat(blobs, len(EDGES), offs, len(OFFS) - 1,
                                       np.ascontiguousarray(w).ctypes.data, xs.ctypes.data,
                                       out.ctypes.data)
    assert rc == 0, _lib.last_error()
    _check(out, refs)


def test_positions_flat_bounds_and_step_down(gpu, case):
    """The flat form's contract: more than 16 positions, or more than
    16 x positions edges, is invalid (-2, tools/metal_moe.mm:1056-1059); a
    scale4-v2 batch whose positions have different edge counts has no
    single-dispatch form here and returns -6 with the output untouched, and
    the provider's step-down (provider_moe.cpp:1406-1478) to the positions call
    gives the rows."""
    from deltafin_amd import _lib, moe
    g, raw, w, x, refs = case
    say("positions_flat bounds and the -6 step-down")
    lib = _lib.load()
    n_pos = 17
    offs17 = (C.c_int * (n_pos + 1))(*([0] * (n_pos + 1)))
    x17 = np.zeros((n_pos, H), np.float32)
    o17 = np.zeros((n_pos, H), np.float32)
    rc = lib.k3_hip_moe_positions_flat(None, 0, offs17, n_pos, None, x17.ctypes.data,
                                       o17.ctypes.data)
    assert rc == _lib.K3_HIP_E_INVALID
    offs2 = (C.c_int * 2)(0, 17)
    blobs = (C.c_void_p * 17)(*([raw[0].ctypes.data] * 17))
    w17 = np.full(17, 1.0 / 17, np.float32)
    rc = lib.k3_hip_moe_positions_flat(blobs, 17, offs2, 1, w17.ctypes.data, x17.ctypes.data,
                                       o17.ctypes.data)
    assert rc == _lib.K3_HIP_E_INVALID
    s4 = [oracle.scale4_span(r) for r in raw]
    descs = moe._descs([s4[e] for e in EDGES], _lib.K3_SCALE4_V2_EXPERT_SPAN,
                       _lib.K3_LAYOUT_SCALE4_V2)
    offs = (C.c_int * len(OFFS))(*OFFS)
    xs = np.ascontiguousarray(x, dtype=np.float32)
    wv = np.ascontiguousarray(w, dtype=np.float32)
    out = np.full((len(OFFS) - 1, H), 7.0, np.float32)
    rc = lib.k3_hip_moe_positions_flat_desc_v1(descs, len(EDGES), offs, len(OFFS) - 1,
                                               wv.ctypes.data, xs.ctypes.data, out.ctypes.data)
    assert rc == _lib.K3_HIP_E_CAPABILITY, (rc, _lib.last_error())
    assert np.all(out == 7.0), "a capability miss must leave the output untouched"
    rc = lib.k3_hip_moe_positions_desc_v1(descs, len(EDGES), offs, len(OFFS) - 1,
                                          wv.ctypes.data, xs.ctypes.data, out.ctypes.data)
    assert rc == 0, _lib.last_error()
    _check(out, refs)
    # Equal edge counts over scale4-v2 spans are one position batch: flat runs.
    eq_edges, eq_offs = EDGES[:12], [0, 4, 8, 12]
    eq_w = np.concatenate([_weights(4, 30 + p) for p in range(3)])
    a = moe.moe_positions_desc([s4[e] for e in eq_edges], eq_offs, eq_w, x[:3],
                               layout=_lib.K3_LAYOUT_SCALE4_V2, flat=True)
    for p in range(3):
        sl = slice(eq_offs[p], eq_offs[p + 1])
        ref, mag = oracle.moe_layer_f64([raw[e] for e in eq_edges[sl]],
                                        eq_w[sl].astype(np.float64), H, I, g.activation, x[p])
        assert oracle.cond_rel_err(a[p], ref, mag, I) <= TOL, f"scale4 flat position {p}"
