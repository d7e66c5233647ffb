"""GPU parity of the whole K3 MoE block (k3_hip_moe_block_device): router,
sigmoid + bias top-16, routed_down, the routed experts, RMS norm, routed_up
and the shared SiTU expert, against the float64 oracle (oracle/spine.py
moe_block_f64):

* the reference's own tiny-geometry fixture (provider_moe_test.cpp:50-191:
  row-int8 spine, 16 closed-form experts, hidden 32 / routed 32 /
  intermediate 32 / shared 64) at one and three positions, under the
  reference's bound max |out - expected| <= 2e-4 (:291);
* the K3 geometry (hidden 7168, routed 3584, intermediate 3072, shared 6144,
  896 experts in a device bank) with BF16 spines at 1, 3, 4, 8, 11 and 16
  positions (from 3 positions the spine runs on the BF16 matrix cores from
  three-term activation splits; 11-16 take the three-tile form) and a
  row-int8 spine at 2: every output within 1e-3 of the oracle relative to
  max(|ref|, mag / sqrt(n)) (oracle.cond_rel_err, mag = the size of the terms
  the output sums, n = routed + shared widths), route ids identical;
* a small BF16 spine (hidden 576, routed 256, shared 320, 40 experts, top-8)
  at 3 and 7 positions, where the matrix-core spine's row tails, single
  column wave and zero-term padding run, under the same bar;
* the route of a hidden row does not depend on the batch: the same rows at
  1, 4 and 16 positions route to the same experts with bit-identical weights;
* 16 positions, where AUTO takes the union path: outputs equal the
  one-decode-layer-per-position path's within 1e-4 normwise, same routes;
* calls at 1, 2 and 4 positions back to back on one workspace with no
  synchronisation between them (the shared expert's gate/up runs on the
  library's side stream and joins before shared_down): every call's output
  against the oracle (the other cases exercise the side stream at every
  position count);
* two host threads, each on its own stream and workspace, issuing block calls
  at the same time (their side work shares the library's side stream): every
  output against the oracle.
"""
import zlib

import numpy as np
import pytest

import oracle
from oracle import spine as S

pytestmark = pytest.mark.gpu

K3 = dict(hidden=7168, routed=3584, inter=3072, shared=6144, experts=896, top_k=16)


def say(msg):
    print(f"[gpu-case] {msg}", flush=True)


def _dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _spine_from(kind, m):
    from deltafin_amd import spine
    mats = {}
    scales = {}
    for name in spine.MoeSpine.MATRICES:
        a = m[name]
        mats[name] = _dev(a.view(np.int16) if kind == "bf16" else a)
        if kind == "int8":
            scales[name] = _dev(m[name + "_scales"].astype(np.float32))
    return spine.MoeSpine(kind, mats["router"], _dev(m["router_bias"].astype(np.float32)),
                          mats["routed_down"], _dev(m["routed_norm"].astype(np.float32)),
                          mats["routed_up"], mats["shared_gate"], mats["shared_up"],
                          mats["shared_down"], scales=scales if kind == "int8" else None)


@pytest.mark.parametrize("positions", [1, 3])
def test_block_reference_tiny_fixture(gpu, positions):
    import torch
    from deltafin_amd import _lib, spine
    say(f"block: reference tiny fixture, positions {positions}")
    m = S.tiny_spine()
    g = _lib.geometry(32, 32, _lib.K3_ACT_SITU)
    spans = np.concatenate([S.tiny_expert_span(e) for e in range(16)])
    stride = g.expert_span
    bank = _dev(spans)
    hidden = S.tiny_hidden(positions)
    sp = _spine_from("int8", m)
    out, ids, wts = spine.moe_block(sp, g, bank, stride, _dev(hidden))
    torch.cuda.synchronize()
    want, want_ids, want_w, _ = S.moe_block_f64("int8", m, S.tiny_expert_span, hidden, 32, 16)
    assert ids.cpu().numpy().tolist() == want_ids.tolist()
    assert np.max(np.abs(wts.cpu().numpy() - want_w)) <= 1e-6
    err = np.max(np.abs(out.cpu().numpy().astype(np.float64) - want))
    assert err <= 2.0e-4, f"max abs error {err:.3e} above the reference's 2e-4"


def _k3_spine(kind, seed):
    rng = np.random.default_rng(seed)
    H, R, Sh, E = K3["hidden"], K3["routed"], K3["shared"], K3["experts"]
    shapes = {"router": (E, H), "routed_down": (R, H), "routed_up": (H, R),
              "shared_gate": (Sh, H), "shared_up": (Sh, H), "shared_down": (H, Sh)}
    m = {}
    for name, (rows, cols) in shapes.items():
        if kind == "bf16":
            v = rng.standard_normal((rows, cols), dtype=np.float32) * np.float32(0.02)
            m[name] = (v.view(np.uint32) >> 16).astype(np.uint16)
        else:
            m[name] = rng.integers(-127, 128, size=(rows, cols), dtype=np.int8)
            m[name + "_scales"] = (rng.uniform(0.5, 1.5, rows) * 0.02 / 64).astype(np.float32)
    m["router_bias"] = (rng.standard_normal(E) * 0.01).astype(np.float32)
    m["routed_norm"] = (1.0 + 0.1 * rng.standard_normal(R)).astype(np.float32)
    return m


@pytest.fixture(scope="module")
def k3_bank(gpu):
    import torch
    from deltafin_amd import _lib, moe
    g = _lib.preset(1)
    stride = g.expert_span
    bank = torch.empty(K3["experts"] * stride, dtype=torch.uint8, device="cuda")
    moe.synth_bank(g, bank, stride, K3["experts"], 0, 4242)
    torch.cuda.synchronize()
    cache = {}

    def span(e):
        if e not in cache:
            cache[e] = bank[e * stride:(e + 1) * stride].cpu().numpy()
        return cache[e]
    return g, bank, stride, span


def _normwise(got, want):
    return float(np.max(np.abs(got - want)) / np.max(np.abs(want)))


@pytest.mark.parametrize("kind,positions", [("bf16", 1), ("bf16", 3), ("bf16", 4), ("bf16", 8),
                                            ("bf16", 11), ("bf16", 16), ("int8", 2)])
def test_block_k3_geometry(gpu, k3_bank, kind, positions):
    import torch
    from deltafin_amd import spine
    g, bank, stride, span = k3_bank
    say(f"block: K3 geometry, {kind} spine, positions {positions}")
    m = _k3_spine(kind, zlib.crc32(f"{kind}{positions}".encode()))
    hidden = np.random.default_rng(positions).standard_normal(
        (positions, K3["hidden"]), dtype=np.float32)
    sp = _spine_from(kind, m)
    out, ids, wts = spine.moe_block(sp, g, bank, stride, _dev(hidden))
    torch.cuda.synchronize()
    want, want_ids, want_w, _, mag = S.moe_block_f64(kind, m, span, hidden, K3["inter"], 16,
                                                     with_mag=True)
    assert ids.cpu().numpy().tolist() == want_ids.tolist(), "route ids differ"
    assert np.max(np.abs(wts.cpu().numpy() - want_w)) <= 1e-6
    got = out.cpu().numpy().astype(np.float64)
    for p in range(positions):
        err = oracle.cond_rel_err(got[p], want[p], mag[p], K3["routed"] + K3["shared"])
        assert err <= 1e-3, f"position {p}: cond rel err {err:.3e}"


SMALL = dict(hidden=576, routed=256, inter=128, shared=320, experts=40, top_k=8)


@pytest.mark.parametrize("positions", [3, 7])
def test_block_small_bf16_spine(gpu, positions):
    """A BF16 spine whose shapes leave row tails (40 router rows), a single
    column wave (256 columns) and zero-term padding steps on the matrix-core
    spine, against the oracle per element."""
    import torch
    from deltafin_amd import _lib, moe, spine
    say(f"block: small BF16 spine (576/256/320, 40 experts), positions {positions}")
    H, R, Sh, E, I = (SMALL[k] for k in ("hidden", "routed", "shared", "experts", "inter"))
    g = _lib.geometry(R, I, _lib.K3_ACT_SITU)
    stride = g.expert_span
    bank = torch.empty(E * stride, dtype=torch.uint8, device="cuda")
    moe.synth_bank(g, bank, stride, E, 0, 77)
    rng = np.random.default_rng(100 + positions)
    shapes = {"router": (E, H), "routed_down": (R, H), "routed_up": (H, R),
              "shared_gate": (Sh, H), "shared_up": (Sh, H), "shared_down": (H, Sh)}
    m = {}
    for name, (rows, cols) in shapes.items():
        v = rng.standard_normal((rows, cols), dtype=np.float32) * np.float32(0.05)
        m[name] = (v.view(np.uint32) >> 16).astype(np.uint16)
    m["router_bias"] = (rng.standard_normal(E) * 0.01).astype(np.float32)
    m["routed_norm"] = (1.0 + 0.1 * rng.standard_normal(R)).astype(np.float32)
    sp = spine.MoeSpine("bf16", _dev(m["router"].view(np.int16)), _dev(m["router_bias"]),
                        _dev(m["routed_down"].view(np.int16)), _dev(m["routed_norm"]),
                        _dev(m["routed_up"].view(np.int16)), _dev(m["shared_gate"].view(np.int16)),
                        _dev(m["shared_up"].view(np.int16)), _dev(m["shared_down"].view(np.int16)),
                        top_k=SMALL["top_k"])
    hidden = rng.standard_normal((positions, H), dtype=np.float32)
    out, ids, wts = spine.moe_block(sp, g, bank, stride, _dev(hidden))
    torch.cuda.synchronize()
    host = bank.cpu().numpy()
    want, want_ids, want_w, _, mag = S.moe_block_f64(
        "bf16", m, lambda e: host[e * stride:(e + 1) * stride], hidden, I, SMALL["top_k"],
        with_mag=True)
    assert ids.cpu().numpy().tolist() == want_ids.tolist(), "route ids differ"
    assert np.max(np.abs(wts.cpu().numpy() - want_w)) <= 1e-6
    got = out.cpu().numpy().astype(np.float64)
    for p in range(positions):
        err = oracle.cond_rel_err(got[p], want[p], mag[p], R + Sh)
        assert err <= 1e-3, f"position {p}: cond rel err {err:.3e}"


def test_block_routes_do_not_depend_on_batch(gpu, k3_bank):
    """The same hidden rows in a 1-position call, a 4-position call (BF16
    matrix-core spine) and a 16-position call route to the same experts with
    bit-identical weights: the router logits are summed in one order at every
    batch size."""
    import torch
    from deltafin_amd import spine
    g, bank, stride, _ = k3_bank
    say("block: routes at 1, 4 and 16 positions")
    m = _k3_spine("bf16", 515)
    sp = _spine_from("bf16", m)
    rows = np.random.default_rng(515).standard_normal((16, K3["hidden"]), dtype=np.float32)
    ids1, w1 = [], []
    for p in range(4):
        _, i, w = spine.moe_block(sp, g, bank, stride, _dev(rows[p:p + 1]))
        ids1.append(i.cpu().numpy()[0])
        w1.append(w.cpu().numpy()[0])
    _, i4, w4 = spine.moe_block(sp, g, bank, stride, _dev(rows[:4]))
    _, i16, w16 = spine.moe_block(sp, g, bank, stride, _dev(rows))
    torch.cuda.synchronize()
    for p in range(4):
        assert np.array_equal(i4.cpu().numpy()[p], ids1[p]) and np.array_equal(
            i16.cpu().numpy()[p], ids1[p]), f"position {p}: routes differ across batch sizes"
        assert np.array_equal(w4.cpu().numpy()[p].view(np.uint32), w1[p].view(np.uint32))
        assert np.array_equal(w16.cpu().numpy()[p].view(np.uint32), w1[p].view(np.uint32))


def test_block_union_matches_positions(gpu, k3_bank):
    import torch
    from deltafin_amd import _lib, spine
    g, bank, stride, _ = k3_bank
    say("block: 16 positions, union path vs one decode layer per position")
    m = _k3_spine("bf16", 99)
    hidden = _dev(np.random.default_rng(16).standard_normal((16, K3["hidden"]), dtype=np.float32))
    sp = _spine_from("bf16", m)
    ws = spine.moe_block_workspace(sp, g, 16)
    out_auto, ids_auto, _ = spine.moe_block(sp, g, bank, stride, hidden, workspace=ws)
    prev = _lib.set_verify_mode(_lib.VERIFY_POSITIONS)
    try:
        out_pos, ids_pos, _ = spine.moe_block(sp, g, bank, stride, hidden, workspace=ws)
    finally:
        _lib.set_verify_mode(prev)
    torch.cuda.synchronize()
    assert torch.equal(ids_auto, ids_pos)
    a = out_auto.cpu().numpy().astype(np.float64)
    b = out_pos.cpu().numpy().astype(np.float64)
    for p in range(16):
        assert _normwise(a[p], b[p]) <= 1e-4, f"position {p}"


def test_block_rejects_bad_calls(gpu, k3_bank):
    import ctypes as C
    from deltafin_amd import _lib, spine
    g, bank, stride, _ = k3_bank
    say("block: argument checks")
    m = S.tiny_spine()
    sp = _spine_from("int8", m)
    d = sp.descriptor()
    lib = _lib.load()
    # the tiny spine's routed width (32) differs from the K3 expert geometry
    assert lib.k3_hip_moe_block_workspace_bytes(C.byref(d), C.byref(g), 1) == 0
    d.struct_bytes = 100
    g32 = _lib.geometry(32, 32, _lib.K3_ACT_SITU)
    assert lib.k3_hip_moe_block_workspace_bytes(C.byref(d), C.byref(g32), 1) == 0
    # the Python layer refuses the mismatch before the library sees it...
    with pytest.raises(ValueError):
        spine.moe_block(sp, g, bank, stride, _dev(np.zeros((1, 32), np.float32)),
                        workspace=_dev(np.zeros(1 << 20, np.uint8)))
    # ...and so does the C ABI when called directly
    d = sp.descriptor()
    hidden = _dev(np.zeros((1, 32), np.float32))
    ws = _dev(np.zeros(1 << 20, np.uint8))
    out = _dev(np.zeros((1, 32), np.float32))
    rc = lib.k3_hip_moe_block_device(C.byref(d), C.byref(g), bank.data_ptr(), stride,
                                     hidden.data_ptr(), 1, out.data_ptr(), None, None,
                                     ws.data_ptr(), ws.numel(), None)
    assert rc == _lib.K3_HIP_E_INVALID


@pytest.mark.parametrize("positions", [1, 4])
def test_block_unaligned_spine_falls_back(gpu, k3_bank, positions):
    """Spine matrices 2 bytes off a 16-byte boundary and a norm weight 4 bytes
    off: the fused and matrix-core forms do not apply, and the block runs the
    separate launches and the any-shape kernel with the same result."""
    import torch
    from deltafin_amd import spine
    g, bank, stride, span = k3_bank
    say(f"block: unaligned BF16 spine, positions {positions}")
    m = _k3_spine("bf16", 7 + positions)

    def off(a, elems):
        flat = np.zeros(a.size + elems, a.dtype)
        flat[elems:] = a.ravel()
        t = _dev(flat.view(np.int16) if a.dtype == np.uint16 else flat)
        return t[elems:].view(*a.shape)

    mats = {n: off(m[n], 1) for n in spine.MoeSpine.MATRICES}
    sp = spine.MoeSpine("bf16", mats["router"], _dev(m["router_bias"]), mats["routed_down"],
                        off(m["routed_norm"], 1), mats["routed_up"], mats["shared_gate"],
                        mats["shared_up"], mats["shared_down"])
    assert sp.routed_norm.data_ptr() % 16 == 4 and sp.router.data_ptr() % 16 == 2
    hidden = np.random.default_rng(40 + positions).standard_normal(
        (positions, K3["hidden"]), dtype=np.float32)
    out, ids, _ = spine.moe_block(sp, g, bank, stride, _dev(hidden))
    torch.cuda.synchronize()
    want, want_ids, _, _ = S.moe_block_f64("bf16", m, span, hidden, K3["inter"], 16)
    assert ids.cpu().numpy().tolist() == want_ids.tolist()
    got = out.cpu().numpy().astype(np.float64)
    for p in range(positions):
        assert _normwise(got[p], want[p]) <= 1e-3, f"position {p}"


def test_block_back_to_back_calls_share_a_workspace(gpu, k3_bank):
    """Four block calls (1, 2, 4 and 1 positions) queued back to back on one
    workspace without a synchronisation between them: each call's shared h
    comes from the side stream and is read by its own shared_down before the
    next call's side work may overwrite it, so every output matches the
    oracle as a lone call's does."""
    import torch
    from deltafin_amd import spine
    g, bank, stride, span = k3_bank
    say("block: back-to-back calls on one workspace (1, 2, 4, 1 positions)")
    m = _k3_spine("bf16", 6161)
    sp = _spine_from("bf16", m)
    ws = spine.moe_block_workspace(sp, g, 4)
    rng = np.random.default_rng(6161)
    sizes = [1, 2, 4, 1]
    hiddens = [rng.standard_normal((p, K3["hidden"]), dtype=np.float32) for p in sizes]
    dev_rows = [_dev(h) for h in hiddens]
    outs = [spine.moe_block(sp, g, bank, stride, d, workspace=ws) for d in dev_rows]
    torch.cuda.synchronize()
    for c, (h, (out, ids, wts)) in enumerate(zip(hiddens, outs)):
        want, want_ids, want_w, _, mag = S.moe_block_f64("bf16", m, span, h, K3["inter"], 16,
                                                         with_mag=True)
        assert ids.cpu().numpy().tolist() == want_ids.tolist(), f"call {c}: route ids differ"
        assert np.max(np.abs(wts.cpu().numpy() - want_w)) <= 1e-6
        got = out.cpu().numpy().astype(np.float64)
        for p in range(h.shape[0]):
            err = oracle.cond_rel_err(got[p], want[p], mag[p], K3["routed"] + K3["shared"])
            assert err <= 1e-3, f"call {c}, position {p}: cond rel err {err:.3e}"


def test_block_two_threads_two_streams(gpu, k3_bank):
    """Two host threads, each with its own torch stream and workspace, queue
    three 1-position block calls each at the same time; the library's side
    stream (shared by both) runs their shared experts.  Every output matches
    the oracle."""
    import threading

    import torch
    from deltafin_amd import spine
    g, bank, stride, span = k3_bank
    say("block: two host threads on two streams, three calls each")
    m = _k3_spine("bf16", 7272)
    sp = _spine_from("bf16", m)
    rng = np.random.default_rng(7272)
    rows = [[rng.standard_normal((1, K3["hidden"]), dtype=np.float32) for _ in range(3)]
            for _ in range(2)]
    dev_rows = [[_dev(h) for h in per] for per in rows]
    streams = [torch.cuda.Stream() for _ in range(2)]
    wss = [spine.moe_block_workspace(sp, g, 1) for _ in range(2)]
    torch.cuda.synchronize()
    results = [[None] * 3 for _ in range(2)]
    errors = []

    def worker(t):
        try:
            with torch.cuda.stream(streams[t]):
                for c in range(3):
                    results[t][c] = spine.moe_block(sp, g, bank, stride, dev_rows[t][c],
                                                    workspace=wss[t])
        except Exception as e:  # reported after the join
            errors.append(e)

    threads = [threading.Thread(target=worker, args=(t,)) for t in range(2)]
    for th in threads:
        th.start()
    for th in threads:
        th.join(timeout=60)
    assert not any(th.is_alive() for th in threads), "a host thread did not finish"
    assert not errors, errors
    torch.cuda.synchronize()
    for t in range(2):
        for c in range(3):
            out, ids, wts = results[t][c]
            want, want_ids, want_w, _, mag = S.moe_block_f64("bf16", m, span, rows[t][c],
                                                             K3["inter"], 16, with_mag=True)
            assert ids.cpu().numpy().tolist() == want_ids.tolist(), f"thread {t} call {c}: ids"
            assert np.max(np.abs(wts.cpu().numpy() - want_w)) <= 1e-6
            err = oracle.cond_rel_err(out.cpu().numpy().astype(np.float64)[0], want[0], mag[0],
                                      K3["routed"] + K3["shared"])
            assert err <= 1e-3, f"thread {t} call {c}: cond rel err {err:.3e}"
