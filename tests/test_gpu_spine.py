"""GPU parity of the spine projections (include/k3_hip_spine_abi.h) against the
float64 oracle (oracle/spine.py), under the reference gate's bound
|found - expected| <= 2e-5 + 2e-5 |expected|
(native/provider_gate/provider_spine_bf16_cuda_test.cpp:296-317):

* the reference gate's own fixtures (19 x 521 salt 5 and 7 x 129 salt 11, at
  positions 1, 2, 9, 64, with the weights at byte offsets 256 and 10,240 of one
  slab), which take the any-shape path;
* the K3 spine shapes (router 896 x 7168, routed_down 3584 x 7168, routed_up
  7168 x 3584, shared gate/up 12288 x 7168, shared_down 7168 x 6144) on the
  streaming path at 1..64 positions, and rows whose byte length leaves a short
  last 1 KB piece;
* the row-int8 form at the same shapes, all 65,536 BF16 encodings through the
  decode canary (bit-exact) and the RMS norm (fp64 closed form, in place too).
"""
import zlib

import numpy as np
import pytest

from oracle import spine as S

pytestmark = pytest.mark.gpu

K3_SHAPES = {  # name: (rows, cols) of the reference's K3 spine (provider_moe.cpp:428-447)
    "router": (896, 7168),
    "routed_down": (3584, 7168),
    "routed_up": (7168, 3584),
    "shared_gate_up": (12288, 7168),
    "shared_down": (7168, 6144),
}


def say(msg):
    print(f"[gpu-case] {msg}", flush=True)


def _bf16_weights(rng, rows, cols, scale=0.02):
    v = (rng.standard_normal((rows, cols), dtype=np.float32) * np.float32(scale))
    return (v.view(np.uint32) >> 16).astype(np.uint16)  # truncation: any BF16 pattern will do


def _close(found, expected, tag):
    found = np.asarray(found, np.float64)
    tol = S.SPINE_TOLERANCE_ABS + S.SPINE_TOLERANCE_REL * np.abs(expected)
    err = np.abs(found - expected)
    worst = np.unravel_index(np.argmax(err - tol), err.shape)
    assert np.all(np.isfinite(found)), f"{tag}: non-finite output"
    assert np.all(err <= tol), (f"{tag}: |err| {err[worst]:.3e} > tol {tol[worst]:.3e} at "
                                f"{worst} (expected {expected[worst]:.6e})")


def test_available(gpu):
    import ctypes as C
    from deltafin_amd import _lib
    major, minor = C.c_int(0), C.c_int(0)
    assert gpu.k3_hip_spine_bf16_available(0, C.byref(major), C.byref(minor)) == 1
    assert (major.value, minor.value) == (9, 5), (major.value, minor.value)
    assert "gfx950" in _lib.load().k3_hip_spine_last_error().decode()


def test_reference_gate_fixtures(gpu):
    import torch
    from deltafin_amd import spine
    first = S.spine_fixture(19, 521, 5)
    second = S.spine_fixture(7, 129, 11)
    off1 = 256
    off2 = ((off1 + first[0].nbytes + 255) // 256) * 256
    slab = np.zeros(off2 + second[0].nbytes, np.uint8)
    slab[off1:off1 + first[0].nbytes] = first[0].view(np.uint8).ravel()
    slab[off2:off2 + second[0].nbytes] = second[0].view(np.uint8).ravel()
    dev = torch.from_numpy(slab).cuda()
    for (w, act, exp), off in ((first, off1), (second, off2)):
        rows, cols = w.shape
        wt = dev[off:off + w.nbytes].view(torch.int16).view(rows, cols)
        for positions in (1, 2, 9, 64):
            say(f"reference fixture {rows}x{cols} positions {positions}")
            x = torch.from_numpy(np.tile(act, (positions, 1))).cuda()
            out = spine.bf16_gemv(wt, x)
            torch.cuda.synchronize()
            _close(out.cpu().numpy(), np.tile(exp.astype(np.float64), (positions, 1)),
                   f"fixture {rows}x{cols} p{positions}")


@pytest.mark.parametrize("name", list(K3_SHAPES))
def test_bf16_k3_shapes(gpu, name):
    import torch
    from deltafin_amd import spine
    rows, cols = K3_SHAPES[name]
    rng = np.random.default_rng(zlib.crc32(name.encode()))
    w = _bf16_weights(rng, rows, cols)
    wt = torch.from_numpy(w.view(np.int16)).cuda()
    x_all = rng.standard_normal((64, cols), dtype=np.float32)
    want_all = S.spine_bf16_f64(w, x_all)
    for positions in (1, 2, 3, 4, 5, 16, 64):
        say(f"bf16 {name} {rows}x{cols} positions {positions}")
        x = torch.from_numpy(x_all[:positions].copy()).cuda()
        out = spine.bf16_gemv(wt, x)
        torch.cuda.synchronize()
        _close(out.cpu().numpy(), want_all[:positions], f"bf16 {name} p{positions}")


@pytest.mark.parametrize("rows,cols", [(37, 3592), (5, 8), (130, 1000), (64, 8192), (8, 8200),
                                       (3, 1004)])
def test_bf16_tails_and_generic(gpu, rows, cols):
    """3592 / 1000 / 8 columns: a short last 1 KB piece on the streaming path
    (8: the only piece); 8192: 16 whole pieces, whose activation fits the LDS
    budget two positions at a time; 8200 (17 pieces) and 1004 (rows not a
    16-byte multiple): the any-shape path."""
    import torch
    from deltafin_amd import spine
    rng = np.random.default_rng(rows * 7919 + cols)
    w = _bf16_weights(rng, rows, cols, scale=0.5)
    wt = torch.from_numpy(w.view(np.int16)).cuda()
    for positions in (1, 3, 7):
        say(f"bf16 tail {rows}x{cols} positions {positions}")
        x_np = rng.standard_normal((positions, cols), dtype=np.float32)
        out = spine.bf16_gemv(wt, torch.from_numpy(x_np).cuda())
        torch.cuda.synchronize()
        _close(out.cpu().numpy(), S.spine_bf16_f64(w, x_np), f"bf16 {rows}x{cols} p{positions}")


@pytest.mark.parametrize("rows,cols", [(896, 7168), (3584, 7168), (7168, 3584), (7168, 6144),
                                       (33, 3072), (9, 48), (5, 100)])
def test_int8_shapes(gpu, rows, cols):
    import torch
    from deltafin_amd import spine
    rng = np.random.default_rng(rows + 31 * cols)
    q = rng.integers(-128, 128, size=(rows, cols), dtype=np.int8)
    s = rng.uniform(1e-4, 2e-3, size=rows).astype(np.float32)
    qt, st = torch.from_numpy(q).cuda(), torch.from_numpy(s).cuda()
    for positions in (1, 2, 4, 9, 64):
        say(f"int8 {rows}x{cols} positions {positions}")
        x_np = rng.standard_normal((positions, cols), dtype=np.float32)
        out = spine.int8_gemv(qt, st, torch.from_numpy(x_np).cuda())
        torch.cuda.synchronize()
        _close(out.cpu().numpy(), S.spine_int8_f64(q, s, x_np), f"int8 {rows}x{cols} p{positions}")


def test_decode_bits_exhaustive(gpu):
    import torch
    from deltafin_amd import spine
    say("decode bits: all 65,536 encodings")
    every = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = spine.decode_bits(torch.from_numpy(every.view(np.int16)).cuda())
    torch.cuda.synchronize()
    assert np.array_equal(got.cpu().numpy().view(np.uint32), S.bf16_to_f32_bits(every))


@pytest.mark.parametrize("rows,cols", [(1, 3584), (16, 3584), (3, 7168), (2, 5)])
def test_rms_norm(gpu, rows, cols):
    import torch
    from deltafin_amd import _lib, spine
    say(f"rms norm {rows}x{cols}")
    rng = np.random.default_rng(rows * 100 + cols)
    x_np = (rng.standard_normal((rows, cols), dtype=np.float32) * 3).astype(np.float32)
    w_np = rng.standard_normal(cols, dtype=np.float32)
    want = S.rms_norm_f64(x_np, w_np, _lib.K3_RMS_EPS)
    x, w = torch.from_numpy(x_np).cuda(), torch.from_numpy(w_np).cuda()
    out = spine.rms_norm(x, w)
    spine.rms_norm(x, w, out=x)  # in place
    torch.cuda.synchronize()
    for got, tag in ((out, "out of place"), (x, "in place")):
        g = got.cpu().numpy().astype(np.float64)
        assert np.max(np.abs(g - want) / (np.abs(want) + 1e-30)) < 2e-6 or \
            np.max(np.abs(g - want)) < 1e-6, f"rms norm {rows}x{cols} {tag}"
    assert torch.equal(out, x)


def test_rms_norm_constant_rows(gpu):
    import torch
    from deltafin_amd import _lib, spine
    say("rms norm constant rows")
    vals = np.array([0.0, 1.0, -3.0, 1e-3], np.float32)
    x_np = np.repeat(vals[:, None], 64, axis=1)
    w_np = np.arange(1, 65, dtype=np.float32)
    out = spine.rms_norm(torch.from_numpy(x_np).cuda(), torch.from_numpy(w_np).cuda())
    torch.cuda.synchronize()
    want = S.rms_norm_f64(x_np, w_np, _lib.K3_RMS_EPS)
    assert np.allclose(out.cpu().numpy(), want, rtol=2e-6, atol=0)
    assert np.all(out.cpu().numpy()[0] == 0.0)


def test_stream_and_errors(gpu):
    """Work goes to the caller's stream; invalid calls enqueue nothing and say why."""
    import torch
    from deltafin_amd import _lib, spine
    say("stream and error paths")
    rng = np.random.default_rng(5)
    w = _bf16_weights(rng, 3584, 7168)
    wt = torch.from_numpy(w.view(np.int16)).cuda()
    x_np = rng.standard_normal((1, 7168), dtype=np.float32)
    x = torch.from_numpy(x_np).cuda()
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        out = spine.bf16_gemv(wt, x)
    s.synchronize()
    _close(out.cpu().numpy(), S.spine_bf16_f64(w, x_np), "side stream")
    with pytest.raises(_lib.K3SpineError) as e:
        spine.bf16_gemv(wt, torch.zeros(65, 7168, device="cuda"))
    assert e.value.status == _lib.K3_SPINE_E_INVALID
    assert "positions" in str(e.value)
