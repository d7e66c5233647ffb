"""The allocation-free decode entry point (k3_hip_moe_route_layer_device_noalloc)
against the workspace entry point it mirrors (k3_hip_moe_route_layer_device)
and the fp64 oracle, through the C ABI.

Two calls in a row share the library's static device scratch: the benchmark
geometry at top_k 16, then a smaller geometry at top_k 4 (whose carve-up lands
on bytes the first call left behind), then the first again.  Each output must
equal the workspace entry point's bit for bit (the same kernels run), with
identical route ids and weights, and meet the oracle bar (max relative error
<= 1e-3 against the fp64 oracle, top-k ids identical).
"""
import ctypes as C

import numpy as np
import pytest

import oracle
from deltafin_amd import synth

pytestmark = pytest.mark.gpu

TOL = 1e-3


def say(msg):
    print(f"[gpu-case] {msg}", flush=True)


def _noalloc(lib, g, bank, stride, n_bank, logits, k, x, out, ids, wts):
    from deltafin_amd import _lib, moe
    return lib.k3_hip_moe_route_layer_device_noalloc(
        C.byref(g), bank.data_ptr(), stride, n_bank, logits.data_ptr(), k, x.data_ptr(),
        moe._dtype_code(x), out.data_ptr(), moe._dtype_code(out), ids.data_ptr(),
        wts.data_ptr(), moe.stream_handle())


def _case(lib, g, n_bank, k, seed, x_dtype, out_dtype):
    import torch
    from deltafin_amd import _lib, moe
    stride = g.expert_span
    bank = torch.empty(n_bank * stride, dtype=torch.uint8, device="cuda")
    moe.synth_bank(g, bank, stride, n_bank, 0, seed)
    rng = np.random.default_rng(seed)
    logits_h = rng.standard_normal(n_bank).astype(np.float32)
    x32 = synth.bf16_bits_to_f32(synth.to_bf16_bits(rng.standard_normal(g.hidden).astype(np.float32)))
    logits = torch.from_numpy(logits_h).cuda()
    x = torch.from_numpy(x32).cuda().to(x_dtype)
    out = torch.full((g.hidden,), float("nan"), dtype=out_dtype, device="cuda")
    ids = torch.full((k,), -1, dtype=torch.int32, device="cuda")
    wts = torch.zeros(k, dtype=torch.float32, device="cuda")
    rc = _noalloc(lib, g, bank, stride, n_bank, logits, k, x, out, ids, wts)
    assert rc == 0, _lib.last_error()
    ws = moe.workspace(g, k)
    ref_out, ref_ids, ref_w = moe.moe_route_layer(g, bank, stride, n_bank, logits, k, x, ws,
                                                  out_dtype=out_dtype)
    torch.cuda.synchronize()
    a = out.view(torch.int16 if out_dtype == torch.bfloat16 else torch.int32).cpu().numpy()
    b = ref_out.view(torch.int16 if out_dtype == torch.bfloat16 else torch.int32).cpu().numpy()
    assert np.array_equal(a, b), "no-alloc output differs from the workspace entry point"
    assert ids.cpu().numpy().tolist() == ref_ids.cpu().numpy().tolist()
    assert np.array_equal(wts.cpu().numpy().view(np.uint32), ref_w.cpu().numpy().view(np.uint32))
    rid, rw = oracle.topk_softmax(logits_h, k)
    assert ids.cpu().numpy().tolist() == rid.tolist()
    spans = [oracle.synth_expert(seed, int(e), g.hidden, g.intermediate) for e in rid]
    ref, mag = oracle.moe_layer_f64(spans, rw, g.hidden, g.intermediate, g.activation, x32)
    got = out.float().cpu().numpy()
    if out_dtype == torch.float32:
        err = oracle.cond_rel_err(got, ref, mag, g.intermediate)
        assert err <= TOL, f"cond rel err {err:.3e}"
    else:
        scale = np.maximum(np.abs(ref), np.asarray(mag) / np.sqrt(g.intermediate))
        ulp = np.maximum(np.abs(ref), 1e-30) * 2.0 ** -7
        assert np.all(np.abs(got - ref) <= ulp + TOL * scale)


def test_noalloc_matches_workspace_entry_two_calls(gpu):
    import torch
    from deltafin_amd import moe
    say("noalloc: preset 2, top_k 16, bf16 x, fp32 out")
    _case(gpu, moe.preset(2), 40, 16, 911, torch.bfloat16, torch.float32)
    say("noalloc: 512/256 SiLU, top_k 4, fp32 x, bf16 out (smaller, same scratch)")
    _case(gpu, moe.geometry(512, 256, moe.K3_ACT_SILU), 12, 4, 912, torch.float32, torch.bfloat16)
    say("noalloc: preset 1 (K3, SiTU), top_k 16, bf16 x, fp32 out")
    _case(gpu, moe.preset(1), 20, 16, 913, torch.bfloat16, torch.float32)


def test_noalloc_rejects_oversize_and_bad_top_k(gpu):
    import torch
    from deltafin_amd import _lib, moe
    say("noalloc: size limits")
    g = moe.preset(2)
    # top_k 32 at the benchmark geometry needs more than the static scratch:
    # refused on the host before anything is enqueued.
    assert gpu.k3_hip_moe_workspace_bytes(C.byref(g), 32, 1) > _lib.K3_HIP_NOALLOC_SCRATCH_BYTES
    assert gpu.k3_hip_moe_workspace_bytes(C.byref(g), 16, 1) <= _lib.K3_HIP_NOALLOC_SCRATCH_BYTES
    dummy = torch.empty(1 << 12, dtype=torch.uint8, device="cuda")
    p = dummy.data_ptr()
    rc = gpu.k3_hip_moe_route_layer_device_noalloc(
        C.byref(g), p, g.expert_span, 40, p, 32, p, _lib.K3_DTYPE_BF16, p, _lib.K3_DTYPE_F32,
        None, None, moe.stream_handle())
    assert rc == _lib.K3_HIP_E_INVALID
    assert "scratch" in _lib.last_error()
    g2 = moe.preset(2)
    for k in (0, 33):
        rc = gpu.k3_hip_moe_route_layer_device_noalloc(
            C.byref(g2), p, g2.expert_span, 40, p, k, p, _lib.K3_DTYPE_BF16, p,
            _lib.K3_DTYPE_F32, None, None, moe.stream_handle())
        assert rc == _lib.K3_HIP_E_INVALID
    torch.cuda.synchronize()
