"""Streamed experts (BASELINE configs[4] at test size) against the fp64 oracle.

Three layers of benchmark-geometry experts (hidden 7168, intermediate 2048,
23,396,352-byte raw-v1 spans) live in host memory: layers 0 and 2 in pinned
memory, layer 1 in pageable memory (its misses go through the cache's pinned
staging slots).  An HBM cache of 10 slots (fewer than the 36 experts of the
working set, so evictions cross layers) serves Zipf(1.1) routes of 4 distinct
experts per layer and token.  Every layer step is plan -> fetch -> resolve ->
layer kernels -> release with no host synchronisation, x chained from layer
to layer in bf16 (the fp32 layer output RMS-normalised, then rounded to
bf16).  Afterwards sampled
steps' fp32 outputs are checked against oracle.moe_layer_f64 on the host bytes
of the routed experts, with the exact bf16 input the step consumed (max
relative error <= 1e-3), and resident entries read back byte for byte.
Follows the reference's plan/upload/execute sequence
(provider_cuda_moe.cpp:757-805, :963-1164).

A second case runs config 4 at its route width: top-16 Zipf routes over 40
experts per layer (three layers, pinned / pageable / pinned), a 24-slot cache
(the working set is 120 experts, so every layer's misses evict other layers'
entries), with the same checks.
"""
import ctypes as C

import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu

TOL = 1e-3
PINNED = (True, False, True)
SEED = 4242


def say(msg):
    print(f"[gpu-case] {msg}", flush=True)


def _routes(total, layers, per_layer, k):
    rng = np.random.default_rng(SEED)
    perms = [rng.permutation(per_layer) for _ in range(layers)]
    pz = np.arange(1, per_layer + 1, dtype=np.float64) ** -1.1
    pz /= pz.sum()
    r = np.empty((total, layers, k), np.int64)
    for t in range(total):
        for layer in range(layers):
            r[t, layer] = np.sort(perms[layer][rng.choice(per_layer, k, replace=False, p=pz)])
    w = rng.random((total, layers, k)).astype(np.float32)
    w /= w.sum(axis=2, keepdims=True)
    return r, w


@pytest.mark.parametrize("PER_LAYER,K,SLOTS,TOKENS,every", [(12, 4, 10, 12, 3), (40, 16, 24, 6, 4)],
                         ids=["top4_of_12", "top16_of_40"])
def test_streamed_layers_pinned_and_pageable_vs_oracle(gpu, PER_LAYER, K, SLOTS, TOKENS, every):
    import torch
    from deltafin_amd import _lib, moe
    LAYERS = len(PINNED)
    g = moe.preset(2)
    span = g.expert_span
    say(f"streamed: {LAYERS} layers x {PER_LAYER} experts, cache {SLOTS} slots, pinned {PINNED}")
    dev = torch.empty(PER_LAYER * span, dtype=torch.uint8, device="cuda")
    hosts = []
    for layer in range(LAYERS):
        h = torch.empty(PER_LAYER * span, dtype=torch.uint8, pin_memory=PINNED[layer])
        assert h.is_pinned() == PINNED[layer]
        moe.synth_bank(g, dev, span, PER_LAYER, layer * PER_LAYER, SEED)
        h.copy_(dev)
        hosts.append(h)
    torch.cuda.synchronize()
    del dev
    routes, weights = _routes(TOKENS, LAYERS, PER_LAYER, K)
    cache = moe.ExpertCache(span, SLOTS, LAYERS, staging_slots=2)
    ws = moe.workspace(g, K)
    x = moe.synth_normal(g.hidden, torch.bfloat16, SEED, 9)
    steps = []  # (token, layer, x_in (device bf16), out (device fp32))
    plan = 0
    for t in range(TOKENS):
        for layer in range(LAYERS):
            plan += 1
            ids = routes[t, layer].tolist()
            miss = cache.plan(plan, layer, ids)
            cache.fetch(plan, [hosts[layer].data_ptr() + e * span for e in miss])
            spans = cache.resolve(plan, ids)
            out = moe.moe_layer(g, spans, weights[t, layer].tolist(), x, ws)
            cache.release(plan)
            steps.append((t, layer, x, out))
            # RMS-normalised (as between a model's layers) so the chained
            # activations stay O(1) instead of growing ~1e5x per layer.
            x = (out * torch.rsqrt(out.pow(2).mean() + 1e-6)).to(torch.bfloat16)
    torch.cuda.synchronize()
    st = cache.stats()
    say(f"streamed: stats {st}")
    assert st["evictions"] > 0 and st["misses"] > SLOTS
    worst = 0.0
    for i, (t, layer, xin, out) in enumerate(steps):
        if i % every != 1 and i != len(steps) - 1:
            continue
        hb = hosts[layer].numpy()
        sp = [hb[e * span:(e + 1) * span] for e in routes[t, layer]]
        ref, mag = oracle.moe_layer_f64(sp, weights[t, layer].astype(np.float64), g.hidden,
                                        g.intermediate, g.activation, xin.float().cpu().numpy())
        err = oracle.cond_rel_err(out.cpu().numpy(), ref, mag, g.intermediate)
        worst = max(worst, err)
        assert err <= TOL, f"token {t} layer {layer} (pinned={PINNED[layer]}): {err:.3e}"
    say(f"streamed: max cond rel err {worst:.3e}")
    # Resident entries hold exactly the host bytes of their (layer, expert).
    last_t = TOKENS - 1
    for layer in range(LAYERS):
        e = int(routes[last_t, layer][0])
        try:
            got = cache.read_back(layer, e)
        except _lib.K3HipError:
            continue  # evicted since; other layers still cover the check
        want = hosts[layer].numpy()[e * span:(e + 1) * span]
        assert np.array_equal(got, want)
    cache.close()
