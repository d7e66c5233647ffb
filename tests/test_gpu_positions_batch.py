"""Position-batched decode (one gate/up and one down launch for all positions
of a verify call, position on the grid's y axis) against one routed decode
layer per position: identical routes and outputs bit for bit, on both down
kernels (intermediate 2048: k_down_g64; intermediate 3072: k_down_g96), with
fp32 and bf16 outputs, and the first position against the oracle.

Every case runs under both gate/up dot settings (k3_hip_set_decode_mfma):
vector ALUs for every activation, and the default, where fp32 activations
take the matrix-core gate/up in the batched and the one-position launches
alike."""
import numpy as np
import pytest

import oracle
from deltafin_amd import synth

pytestmark = pytest.mark.gpu

TOL = 1e-3


def say(msg):
    print(f"[gpu-case] {msg}", flush=True)


def _t(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


@pytest.fixture(params=["valu_dots", "mfma_f32_dots"])
def positions_mode(gpu, request):
    from deltafin_amd import _lib
    prev = _lib.set_verify_mode(_lib.VERIFY_POSITIONS)
    prev_dots = _lib.set_decode_mfma(_lib.DECODE_DOTS_VALU if request.param == "valu_dots"
                                     else _lib.DECODE_DOTS_MFMA_F32)
    yield
    _lib.set_decode_mfma(prev_dots)
    _lib.set_verify_mode(prev)


@pytest.mark.parametrize("preset_id,m,odt", [(2, 5, "f32"), (2, 3, "bf16"), (1, 4, "f32"),
                                             (1, 2, "bf16")])
def test_batched_positions_equal_per_position_layers(gpu, positions_mode, preset_id, m, odt):
    import torch
    from deltafin_amd import moe
    g = moe.preset(preset_id)
    n_bank, k = 40, 16
    say(f"batched positions preset {preset_id} M={m} out={odt}")
    stride = g.expert_span
    bank = torch.empty(n_bank * stride, dtype=torch.uint8, device="cuda")
    moe.synth_bank(g, bank, stride, n_bank, 0, 515)
    rng = np.random.default_rng(60 + m + preset_id)
    logits = rng.standard_normal((m, n_bank)).astype(np.float32)
    x = synth.bf16_bits_to_f32(synth.to_bf16_bits(
        rng.standard_normal((m, g.hidden)).astype(np.float32)))
    xd = torch.from_numpy(synth.to_bf16_bits(x).view(np.int16)).view(torch.bfloat16).cuda()
    out_dtype = torch.bfloat16 if odt == "bf16" else torch.float32
    ws = moe.workspace(g, m * k, m)
    out, ids, wts = moe.moe_verify_route(g, bank, stride, n_bank, _t(logits), k, xd, ws,
                                         out_dtype=out_dtype)
    ws1 = moe.workspace(g, k)
    for p in range(m):
        o1, i1, w1 = moe.moe_route_layer(g, bank, stride, n_bank, _t(logits[p]), k,
                                         xd[p].contiguous(), ws1, out_dtype=out_dtype)
        torch.cuda.synchronize()
        assert torch.equal(ids[p], i1), f"position {p} ids"
        assert torch.equal(wts[p].view(torch.int32), w1.view(torch.int32)), f"position {p} weights"
        assert torch.equal(out[p].view(torch.int16 if odt == "bf16" else torch.int32),
                           o1.view(torch.int16 if odt == "bf16" else torch.int32)), f"position {p}"
    if odt == "f32":
        rid, rw = oracle.topk_softmax(logits[0], k)
        spans = [oracle.synth_expert(515, int(e), g.hidden, g.intermediate) for e in rid]
        ref, mag = oracle.moe_layer_f64(spans, rw, g.hidden, g.intermediate, g.activation, x[0])
        err = oracle.cond_rel_err(out[0].cpu().numpy(), ref, mag, g.intermediate)
        assert err <= TOL, f"position 0: {err:.3e}"


@pytest.mark.parametrize("preset_id,counts,odt,xdt", [
    (2, [16, 16, 16, 16], "f32", "bf16"),
    (2, [16, 16, 0, 16, 16, 8, 8, 3], "bf16", "bf16"),
    (1, [16, 16, 16], "f32", "f32"),
    (1, [4, 0, 4, 4, 16], "bf16", "f32"),
])
def test_caller_route_batched_positions_equal_per_position_layers(gpu, positions_mode, preset_id,
                                                                  counts, odt, xdt):
    """k3_hip_moe_verify_device with a caller route on the per-position path:
    each run of consecutive positions with the same edge count is one
    position-batched launch pair over a table-mode route; every position must
    equal its own single-position layer bit for bit (experts repeated across
    positions, empty positions as zero rows, lone positions and runs of
    different counts), and sampled positions match the oracle."""
    import torch
    from deltafin_amd import moe
    g = moe.preset(preset_id)
    n_bank = 40
    say(f"caller-route batched positions preset {preset_id} counts {counts} out={odt} x={xdt}")
    stride = g.expert_span
    bank = torch.empty(n_bank * stride, dtype=torch.uint8, device="cuda")
    moe.synth_bank(g, bank, stride, n_bank, 0, 616)
    rng = np.random.default_rng(70 + preset_id + len(counts))
    m = len(counts)
    ids = [rng.choice(n_bank, size=c, replace=False) for c in counts]
    wts = []
    for c in counts:
        w = rng.random(c).astype(np.float32) + 0.05
        wts.append((w / w.sum()).astype(np.float32))
    offs = np.concatenate([[0], np.cumsum(counts)]).astype(int).tolist()
    x = rng.standard_normal((m, g.hidden)).astype(np.float32)
    if xdt == "bf16":
        x = synth.bf16_bits_to_f32(synth.to_bf16_bits(x))
        xd = torch.from_numpy(synth.to_bf16_bits(x).view(np.int16)).view(torch.bfloat16).cuda()
    else:
        xd = _t(x)
    out_dtype = torch.bfloat16 if odt == "bf16" else torch.float32
    span = lambda e: bank[int(e) * stride:(int(e) + 1) * stride]
    edges = [span(e) for p in range(m) for e in ids[p]]
    ws = moe.workspace(g, sum(counts), m)
    out = moe.moe_verify(g, edges, np.concatenate(wts), offs, xd, ws, out_dtype=out_dtype)
    ws1 = moe.workspace(g, 16)
    iv = torch.int16 if odt == "bf16" else torch.int32
    for p in range(m):
        if counts[p] == 0:
            assert torch.count_nonzero(out[p].view(iv)) == 0, f"position {p} (no edges)"
            continue
        o1 = moe.moe_layer(g, [span(e) for e in ids[p]], wts[p], xd[p].contiguous(), ws1,
                           out_dtype=out_dtype)
        torch.cuda.synchronize()
        assert torch.equal(out[p].view(iv), o1.view(iv)), f"position {p} differs from its layer"
    if odt == "f32":
        for p in (0, m - 1):
            if counts[p] == 0:
                continue
            spans = [oracle.synth_expert(616, int(e), g.hidden, g.intermediate) for e in ids[p]]
            ref, mag = oracle.moe_layer_f64(spans, wts[p].astype(np.float64), g.hidden,
                                            g.intermediate, g.activation, x[p])
            err = oracle.cond_rel_err(out[p].cpu().numpy(), ref, mag, g.intermediate)
            assert err <= TOL, f"position {p}: {err:.3e}"
