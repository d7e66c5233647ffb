"""GPU tests of the in-kernel router of the decode layer (router mode of
k3_hip_moe_route_layer_device): top-k of the logits (descending, lower index
on ties, NaN ranked as -inf, -0 equal to +0) and a softmax over the selected
logits, the semantics of oracle.topk_softmax.

Every gate/up workgroup ranks the logits in LDS (block_topk: each key ranked
within its 64-key segment, then the segment candidates ranked against each
other); a bank of up to one key per thread has its logits preloaded ahead of
the activation chunk, a larger bank is read in the ranking's fill loop.  Both
must select exactly the oracle's experts, and the layer output must be
bit-identical to a caller-routed call (explicit spans and the returned
weights), which shares every kernel but the router.
"""
import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu


def say(msg):
    print(f"[gpu-case] {msg}", flush=True)


def _bank(g, n, seed):
    import torch
    from deltafin_amd import moe
    stride = g.expert_span
    bank = torch.empty(n * stride, dtype=torch.uint8, device="cuda")
    moe.synth_bank(g, bank, stride, n, 0, seed)
    return bank, stride


def _check(g, bank, stride, n_bank, logits_np, k, x, ws, tag):
    import torch
    from deltafin_amd import moe
    logits = torch.from_numpy(logits_np.astype(np.float32)).cuda()
    out, ids, wts = moe.moe_route_layer(g, bank, stride, n_bank, logits, k, x, ws)
    torch.cuda.synchronize()
    rid, rw = oracle.topk_softmax(logits_np.astype(np.float32), k)
    got_ids = ids.cpu().numpy()
    assert got_ids.tolist() == rid.tolist(), f"{tag}: ids {got_ids.tolist()} != {rid.tolist()}"
    got_w = wts.cpu().numpy()
    assert np.max(np.abs(got_w - rw)) <= 1e-6, f"{tag}: weights"
    spans = [bank.data_ptr() + int(e) * stride for e in got_ids]
    ref = moe.moe_layer(g, spans, got_w.tolist(), x, ws)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int32), ref.view(torch.int32)), f"{tag}: output"


def _x(g, seed):
    import torch
    from deltafin_amd import synth
    v = np.random.default_rng(seed).standard_normal(g.hidden).astype(np.float32)
    return torch.from_numpy(synth.to_bf16_bits(v).view(np.int16)).view(torch.bfloat16).cuda()


def test_router_edge_cases(gpu):
    from deltafin_amd import moe
    g = moe.preset(2)
    n = 24
    say(f"router edge cases over a {n}-expert bank")
    bank, stride = _bank(g, n, 555)
    ws = moe.workspace(g, 16)
    x = _x(g, 1)
    rng = np.random.default_rng(3)
    nan, inf = np.float32("nan"), np.float32("inf")
    cases = [
        ("one expert", 1, 1, rng.standard_normal(1)),
        ("two experts top-2", 2, 2, rng.standard_normal(2)),
        ("two experts top-1", 2, 1, np.array([0.25, 0.5])),
        ("normal top-16", n, 16, rng.standard_normal(n)),
        ("normal top-3", n, 3, rng.standard_normal(n)),
        ("all equal", n, 16, np.full(n, 0.75)),
        ("tied maximum", n, 16, np.where(np.arange(n) % 5 == 2, 3.0, rng.standard_normal(n))),
        ("tie for second", n, 4, np.array([9.0] + [1.0] * (n - 1))),
        ("NaN first", n, 16, np.concatenate([[nan, nan], rng.standard_normal(n - 2)])),
        ("signed zeros and -inf", n, 16,
         np.array([-0.0, 0.0, -inf, -0.0, 0.0, -inf] * 4, dtype=np.float32)),
        ("maximum last", n, 2, np.concatenate([np.zeros(n - 1), [1.0]])),
    ]
    for tag, n_bank, k, lg in cases:
        _check(g, bank, stride, n_bank, np.asarray(lg, dtype=np.float32), k, x, ws, tag)


@pytest.mark.parametrize("n_bank", [512, 513])
def test_router_bank_size_boundary(gpu, n_bank):
    """512 logits: one preloaded key per thread of the 512-thread workgroup;
    513: the key past the workgroup is read in the ranking's fill loop."""
    from deltafin_amd import moe
    g = moe.preset(2)
    say(f"router bank {n_bank}")
    bank, stride = _bank(g, n_bank, 77)
    ws = moe.workspace(g, 16)
    rng = np.random.default_rng(n_bank)
    for t in range(2):
        lg = rng.standard_normal(n_bank).astype(np.float32)
        if t == 1:
            lg[n_bank - 1] = 10.0  # rank 0 in the last segment
            lg[300] = 9.0
        _check(g, bank, stride, n_bank, lg, 16, _x(g, t), ws, f"n_bank {n_bank} token {t}")
    del bank
