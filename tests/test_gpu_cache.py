"""GPU tests of the HBM expert cache (k3_hip_cache_*), the C counterpart of
CudaMoeExpertCache (native/provider_gate/provider_cuda_moe.{h,cpp}).

* The reference's one-expert residency canary
  (provider_cuda_moe_test.cpp:189-242): capacity one, a span of bytes
  (i * 131 + 17) & 0xff, first plan misses, upload and compute, second plan
  hits with zero misses, and the D2H read-back is byte-exact.
* LRU eviction over unpinned slots and pinning by live plans
  (provider_cuda_moe.cpp:707-747, :963-1008).
* Streaming: two disjoint expert sets alternate through a cache that holds
  exactly one of them, with no host synchronisation between calls, so every
  upload overwrites slots that kernels queued on the compute stream may still
  be reading; outputs must equal direct layer calls on the same bytes.
* Qualification: the reference's device known-answer tests run before the
  first plan (provider_cuda_moe.cpp:291-420, :889-953).
* Fail-closed: a poisoned cache drops its entries and refuses later calls with
  the reason (:517-533, :1199-1201).
"""
import ctypes as C

import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu


def say(msg):
    print(f"[gpu-case] {msg}", flush=True)


def _pinned(nbytes):
    import torch
    return torch.empty(nbytes, dtype=torch.uint8).pin_memory()


def _ids(values):
    return (C.c_uint16 * len(values))(*values)


def _plan(lib, cache, plan_id, layer, ids):
    missing = (C.c_uint16 * len(ids))()
    n_missing = C.c_int(-1)
    rc = lib.k3_hip_cache_plan(cache, plan_id, layer, _ids(ids), len(ids), missing,
                               C.byref(n_missing))
    assert rc == 0, rc
    return [missing[i] for i in range(n_missing.value)]


def _stats(lib, cache):
    six = (C.c_longlong * 6)()
    lib.k3_hip_cache_stats(cache, six)
    return list(six)


def test_cache_residency_canary(gpu):
    """provider_cuda_moe_test.cpp:189-242 restated on the C cache."""
    import torch
    from deltafin_amd import _lib, moe
    lib = gpu
    g = moe.preset(1)
    span = g.expert_span
    say("cache residency canary (capacity 1, K3 span)")
    host = _pinned(span)
    host.numpy()[:] = ((np.arange(span, dtype=np.uint64) * 131 + 17) & 0xFF).astype(np.uint8)
    cache = lib.k3_hip_cache_create(0, span, 1, 1, 0)
    assert cache, _lib.last_error()
    try:
        assert _plan(lib, cache, 101, 0, [0]) == [0]
        srcs = (C.c_void_p * 1)(host.data_ptr())
        assert lib.k3_hip_cache_fetch(cache, 101, srcs, 1) == 0, _lib.last_error()
        spans = (C.c_void_p * 1)()
        st = moe.stream_handle()
        assert lib.k3_hip_cache_resolve(cache, 101, _ids([0]), 1, spans, st) == 0
        x = torch.zeros((1, g.hidden), dtype=torch.float32, device="cuda")
        out = moe.moe_layer(g, [spans[0]], [1.0 / 16.0], x, moe.workspace(g, 1))
        lib.k3_hip_cache_release(cache, 101)
        torch.cuda.synchronize()
        # The pattern puts scale byte 255 (NaN) in some groups, and zero x
        # times a NaN scale is NaN: an output row of the down matrix is NaN
        # exactly when its scales hold a 255 or the h it reads is NaN, i.e. a
        # gate/up row with a 255 scale (the reference canary checks only that
        # an output comes back, provider_cuda_moe_test.cpp:210-224).
        off = oracle.expert_offsets(g.hidden, g.intermediate)
        pat = host.numpy()
        gu_nan = any((pat[off[k]:off[k] + g.intermediate * (g.hidden // 32)] == 255).any()
                     for k in (1, 5))
        w2s = pat[off[3]:off[3] + g.hidden * (g.intermediate // 32)].reshape(g.hidden, -1)
        want_nan = np.full(g.hidden, gu_nan) | (w2s == 255).any(axis=1)
        got = out.cpu().numpy()
        assert out.shape == (g.hidden,)
        assert np.array_equal(np.isnan(got), want_nan)
        assert np.all(got[~want_nan] == 0)
        assert _plan(lib, cache, 102, 0, [0]) == []
        back = np.empty(span, dtype=np.uint8)
        rc = lib.k3_hip_cache_read_back(cache, 0, 0, back.ctypes.data, span)
        assert rc == 0, _lib.last_error()
        assert np.array_equal(back, host.numpy())
        lib.k3_hip_cache_release(cache, 102)
        hits, misses, evictions, resident, capacity, uploaded = _stats(lib, cache)
        assert (hits, misses, evictions, resident, capacity) == (1, 1, 0, 1, 1)
        assert uploaded == span
    finally:
        lib.k3_hip_cache_destroy(cache)


def test_cache_lru_and_pins(gpu):
    """Eviction takes the least-recent unpinned slot; a fetch that needs more
    slots than live plans leave free fails with the allocation status."""
    import torch
    from deltafin_amd import _lib
    lib = gpu
    span = 1 << 20
    say("cache LRU and pinning (capacity 3)")
    hosts = {e: _pinned(span) for e in range(1, 8)}
    for e, h in hosts.items():
        h.numpy()[:] = e
    cache = lib.k3_hip_cache_create(0, span, 3, 2, 0)
    assert cache, _lib.last_error()

    def fetch(plan_id, missing):
        srcs = (C.c_void_p * max(len(missing), 1))(*[hosts[e].data_ptr() for e in missing])
        return lib.k3_hip_cache_fetch(cache, plan_id, srcs, len(missing))

    def resident(layer, e):
        back = np.empty(span, dtype=np.uint8)
        rc = lib.k3_hip_cache_read_back(cache, layer, e, back.ctypes.data, span)
        return rc == 0 and bool(np.all(back == e))

    try:
        assert _plan(lib, cache, 1, 0, [1, 2, 3]) == [1, 2, 3]
        assert fetch(1, [1, 2, 3]) == 0
        lib.k3_hip_cache_release(cache, 1)
        # 3 hits, 4 misses: the least-recent unpinned slot (expert 1) goes.
        assert _plan(lib, cache, 2, 0, [3, 4]) == [4]
        assert fetch(2, [4]) == 0
        torch.cuda.synchronize()
        assert not resident(0, 1) and resident(0, 2) and resident(0, 3) and resident(0, 4)
        # Plan 2 pins 3 and 4: only one slot is free for three misses.
        assert _plan(lib, cache, 3, 1, [5, 6, 7]) == [5, 6, 7]
        assert fetch(3, [5, 6, 7]) == _lib.K3_HIP_E_ALLOC
        lib.k3_hip_cache_release(cache, 3)
        lib.k3_hip_cache_release(cache, 2)
        # Strata: the same id in another layer is a different entry.
        assert _plan(lib, cache, 4, 1, [3]) == [3]
        lib.k3_hip_cache_release(cache, 4)
        # A stale plan id is rejected.
        assert lib.k3_hip_cache_fetch(cache, 4, None, 0) == _lib.K3_HIP_E_INVALID
    finally:
        lib.k3_hip_cache_destroy(cache)


def test_cache_streaming_reuse(gpu):
    """Alternate two 16-expert sets through a 16-slot cache, queueing every
    call without a host sync; each call evicts every slot the previous call's
    kernels read."""
    import torch
    from deltafin_amd import _lib, moe
    lib = gpu
    g = moe.preset(1)
    span = g.expert_span
    n, calls = 16, 6
    say(f"cache streaming reuse: 2 x {n} experts through {n} slots, {calls} calls")
    host = _pinned(2 * n * span)
    hv = host.numpy()
    for e in range(2 * n):
        hv[e * span:(e + 1) * span] = oracle.synth_expert(61, e, g.hidden, g.intermediate)
    dev = host.cuda()
    rng = np.random.default_rng(7)
    x = torch.from_numpy(rng.standard_normal((calls, g.hidden)).astype(np.float32)).cuda()
    w = [rng.random(n).astype(np.float32) for _ in range(calls)]
    cache = lib.k3_hip_cache_create(0, span, n, 1, 0)
    assert cache, _lib.last_error()
    ws = [moe.workspace(g, n) for _ in range(calls)]
    outs = []
    try:
        st = moe.stream_handle()
        for c in range(calls):
            ids = list(range((c % 2) * n, (c % 2) * n + n))
            missing = _plan(lib, cache, 10 + c, 0, ids)
            assert missing == ids  # the other set was evicted
            srcs = (C.c_void_p * n)(*[host.data_ptr() + e * span for e in missing])
            assert lib.k3_hip_cache_fetch(cache, 10 + c, srcs, n) == 0, _lib.last_error()
            spans = (C.c_void_p * n)()
            assert lib.k3_hip_cache_resolve(cache, 10 + c, _ids(ids), n, spans, st) == 0
            outs.append(moe.moe_layer(g, [spans[i] for i in range(n)], w[c].tolist(), x[c:c + 1],
                                      ws[c]))
            lib.k3_hip_cache_release(cache, 10 + c)
        torch.cuda.synchronize()
        for c in range(calls):
            ids = range((c % 2) * n, (c % 2) * n + n)
            ref = moe.moe_layer(g, [dev.data_ptr() + e * span for e in ids], w[c].tolist(),
                                x[c:c + 1], moe.workspace(g, n))
            torch.cuda.synchronize()
            assert torch.equal(outs[c], ref), f"call {c}"
    finally:
        lib.k3_hip_cache_destroy(cache)


def _state(lib, cache):
    buf = C.create_string_buffer(256)
    return lib.k3_hip_cache_state(cache, buf, 256), buf.value.decode()


def test_cache_qualifies_on_first_plan(gpu):
    """CudaMoeExpertCache::available (provider_cuda_moe.cpp:889-953): the
    device known-answer tests run before the first use, and pass here."""
    from deltafin_amd import _lib
    lib = gpu
    say("cache qualification (device known-answer tests)")
    cache = lib.k3_hip_cache_create(0, 1 << 20, 2, 1, 0)
    assert cache, _lib.last_error()
    try:
        assert _state(lib, cache)[0] == 0
        assert _plan(lib, cache, 1, 0, [3]) == [3]
        st, why = _state(lib, cache)
        assert st == 1 and "known-answer" in why, why
        lib.k3_hip_cache_release(cache, 1)
    finally:
        lib.k3_hip_cache_destroy(cache)


def test_cache_poison_fails_closed(gpu):
    """poison_external / poison (provider_cuda_moe.cpp:517-533, :1199-1201):
    every resident entry is dropped and later calls fail with the reason."""
    import torch
    from deltafin_amd import _lib
    lib = gpu
    span = 1 << 20
    say("cache poison")
    host = _pinned(span)
    host.numpy()[:] = 7
    cache = lib.k3_hip_cache_create(0, span, 2, 1, 0)
    assert cache, _lib.last_error()
    try:
        assert _plan(lib, cache, 1, 0, [5]) == [5]
        srcs = (C.c_void_p * 1)(host.data_ptr())
        assert lib.k3_hip_cache_fetch(cache, 1, srcs, 1) == 0
        torch.cuda.synchronize()
        lib.k3_hip_cache_release(cache, 1)
        assert _stats(lib, cache)[3] == 1
        lib.k3_hip_cache_poison(cache, b"spine failure")
        st, why = _state(lib, cache)
        assert st == _lib.K3_HIP_E_EXEC and "spine failure" in why
        assert _stats(lib, cache)[3] == 0
        missing = (C.c_uint16 * 1)()
        n_missing = C.c_int(-1)
        rc = lib.k3_hip_cache_plan(cache, 2, 0, _ids([5]), 1, missing, C.byref(n_missing))
        assert rc == _lib.K3_HIP_E_EXEC and "spine failure" in _lib.last_error()
        back = np.empty(span, dtype=np.uint8)
        assert lib.k3_hip_cache_read_back(cache, 0, 5, back.ctypes.data, span) != 0
    finally:
        lib.k3_hip_cache_destroy(cache)


# ------------------------------------------------------------ budget and recovery
def _geo_small():
    from deltafin_amd import moe
    return moe.geometry(512, 256, moe.K3_ACT_SILU)


def _host_experts(g, n, seed):
    """Pinned host spans of n synthetic experts (oracle generator) + numpy views."""
    spans = [oracle.synth_expert(seed, e, g.hidden, g.intermediate) for e in range(n)]
    hosts = []
    for s in spans:
        h = _pinned(g.expert_span)
        h.numpy()[:] = s
        hosts.append(h)
    return spans, hosts


def test_cache_budget_policy(gpu):
    """CudaMoeCachePolicy (provider_cuda_moe.h:16-28): bounds checked as
    validate_cache_policy (:60-74); the budget is free memory at the first
    plan minus the reserve (:668-705); the policy is frozen from then on."""
    from deltafin_amd import _lib, moe
    g = _geo_small()
    say("cache budget and policy")
    cache = moe.ExpertCache(g.expert_span, 0, 1, staging_slots=0)
    try:
        with pytest.raises(_lib.K3HipError):
            cache.configure(True, capacity=5)        # automatic with a count
        # The reference's bound: 92 strata x 16 experts (kCudaMaximumExperts).
        assert _lib.K3_HIP_CACHE_MAX_EXPERTS == 92 * 16
        with pytest.raises(_lib.K3HipError):
            cache.configure(False, capacity=_lib.K3_HIP_CACHE_MAX_EXPERTS + 1)
        cache.configure(False, capacity=_lib.K3_HIP_CACHE_MAX_EXPERTS)
        with pytest.raises(_lib.K3HipError):
            cache.configure(True, reserve_kind=_lib.K3_CACHE_RESERVE_RATIO_PPM,
                            reserve_value=1_000_001)
        reserve = 1 << 30
        cache.configure(True, reserve_kind=_lib.K3_CACHE_RESERVE_BYTES, reserve_value=reserve)
        assert not cache.budget()["measured"]
        _, hosts = _host_experts(g, 2, 3)
        assert cache.plan(1, 0, [0, 1]) == [0, 1]
        b = cache.budget()
        slot = (g.expert_span + 4095) & ~4095
        want = min(_lib.K3_HIP_CACHE_MAX_EXPERTS, (b["free_bytes"] - reserve) // slot)
        assert b["reserve_bytes"] == reserve and b["capacity"] == want, b
        assert b["allocated_slots"] == 0 and b["rebuilds_left"] == 2
        cache.fetch(1, [h.data_ptr() for h in hosts])
        assert cache.budget()["allocated_slots"] == 32  # one segment
        cache.release(1)
        with pytest.raises(_lib.K3HipError):
            cache.configure(True)  # frozen after first use
        assert "frozen" in _lib.last_error()
    finally:
        cache.close()


def test_cache_recoverable_allocation_failure(gpu):
    """A device allocation failure while admitting misses is recoverable
    (provider_cuda_moe.cpp:545-567, :630-653): the fetch returns
    K3_HIP_E_ALLOC, the plan's hits stay pinned and are materialized to the
    host (materialize_plan_for_cpu, :1170-1196) for the caller's exact CPU
    reconstruction of the tile (provider_moe.cpp:1117-1206) -- checked here
    against the device layer on the same experts -- and the cache re-measures
    its budget and carries on; after two rebuilds the next failure disables
    it (its callers take their CPU path)."""
    import torch
    from deltafin_amd import _lib, moe
    g = _geo_small()
    say("cache recoverable allocation failure")
    n = 36
    spans, hosts = _host_experts(g, n, 11)
    cache = moe.ExpertCache(g.expert_span, 40, 1, staging_slots=0)  # segments of 32 + 8
    try:
        # Fill the first segment with experts 0..31.
        for p in range(4):
            ids = list(range(8 * p, 8 * p + 8))
            miss = cache.plan(1 + p, 0, ids)
            cache.fetch(1 + p, [hosts[e].data_ptr() for e in miss])
            cache.release(1 + p)
        torch.cuda.synchronize()
        assert cache.budget()["allocated_slots"] == 32
        # Plan 10: hits 3 and 7, misses 33 and 34, which need the second
        # segment: its allocation is refused.
        ids = [3, 7, 33, 34]
        miss = cache.plan(10, 0, ids)
        assert miss == [33, 34]
        cache.fail_allocations(1)
        rc = gpu.k3_hip_cache_fetch(cache.handle, 10,
                                    (C.c_void_p * 2)(*[hosts[e].data_ptr() for e in miss]), 2)
        assert rc == _lib.K3_HIP_E_ALLOC and "recoverable" in _lib.last_error()
        st, why = cache.state()
        assert st == 1, why
        b = cache.budget()
        assert b["rebuilds_left"] == 1 and not b["measured"]  # measured again at the next plan
        # The CPU path: hits from the device, misses from the caller's bytes.
        hits = cache.materialize_plan(10, 4)
        assert sorted(hits) == [3, 7]
        for e, b in hits.items():
            assert np.array_equal(b, spans[e])
        w = np.array([0.4, 0.3, 0.2, 0.1], np.float32)
        x = np.random.default_rng(5).standard_normal(g.hidden).astype(np.float32)
        cpu_spans = [hits[e] if e in hits else spans[e] for e in ids]
        ref, mag = oracle.moe_layer_f64(cpu_spans, w.astype(np.float64), g.hidden,
                                        g.intermediate, g.activation, x)
        dev = [torch.from_numpy(spans[e]).cuda() for e in ids]
        ws = moe.workspace(g, 4)
        out = moe.moe_layer(g, dev, w.tolist(), torch.from_numpy(x).cuda(), ws)
        torch.cuda.synchronize()
        assert oracle.cond_rel_err(out.cpu().numpy(), ref, mag, g.intermediate) <= 1e-3
        cache.release(10)
        # Unpinned entries were dropped; the cache carries on after re-measuring.
        assert cache.stats()["resident"] == 2
        miss = cache.plan(11, 0, [3, 33, 35])
        assert miss == [33, 35]
        cache.fetch(11, [hosts[e].data_ptr() for e in miss])
        got = cache.resolve(11, [3, 33, 35])
        torch.cuda.synchronize()
        cache.release(11)
        assert cache.budget()["measured"] and cache.read_back(0, 35).tobytes() == spans[35].tobytes()
        assert len(got) == 3
        # Two more failures: the second rebuild, then the cache disables itself.
        statuses = []
        for k in range(2):
            cache.fail_allocations(100)
            for p in range(40):
                pid = 100 + 50 * k + p
                miss = cache.plan(pid, 0, [p])
                srcs = (C.c_void_p * max(len(miss), 1))(*[hosts[e % n].data_ptr() for e in miss])
                rc = gpu.k3_hip_cache_fetch(cache.handle, pid, srcs, len(miss))
                cache.release(pid)
                if rc != 0:
                    statuses.append((rc, _lib.last_error()))
                    break
        assert [s[0] for s in statuses] == [_lib.K3_HIP_E_ALLOC] * 2
        assert "disabled" in statuses[1][1], statuses
        st, why = cache.state()
        assert st == _lib.K3_HIP_E_CAPABILITY and "rebuilds" in why, why
        missing = (C.c_uint16 * 1)()
        nm = C.c_int()
        assert gpu.k3_hip_cache_plan(cache.handle, 999, 0, _ids([1]), 1, missing,
                                     C.byref(nm)) == _lib.K3_HIP_E_CAPABILITY
    finally:
        cache.close()


def test_cache_release_orders_reuse_on_every_stream(gpu):
    """Two live plans hold the same slot and read it on two different streams
    (resolve on one, ready_subset on the other); after both are released a
    fetch evicts it.  The copy into the slot must wait for both streams' work:
    both layers' outputs equal the same layer on a private copy of the
    expert."""
    import torch
    from deltafin_amd import _lib, moe
    g = _geo_small()
    say("cache slot reuse after two streams")
    spans, hosts = _host_experts(g, 3, 21)
    cache = moe.ExpertCache(g.expert_span, 1, 1, staging_slots=0)
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    try:
        x = torch.from_numpy(np.random.default_rng(6).standard_normal(g.hidden)
                             .astype(np.float32)).cuda()
        ws1, ws2 = moe.workspace(g, 1), moe.workspace(g, 1)
        private = torch.from_numpy(spans[0]).cuda()
        want = moe.moe_layer(g, [private], [1.0], x, moe.workspace(g, 1))
        torch.cuda.synchronize()
        miss = cache.plan(1, 0, [0])
        cache.fetch(1, [hosts[e].data_ptr() for e in miss])
        # Wait (on the host) for the upload, so ready_subset sees it below.
        cache.resolve(1, [0])
        torch.cuda.current_stream().synchronize()
        outs = []
        with torch.cuda.stream(s1):
            sp = cache.resolve(1, [0], stream=moe.stream_handle(s1))
            for _ in range(20):
                outs.append(moe.moe_layer(g, sp, [1.0], x, ws1))
        assert cache.plan(2, 0, [0]) == []
        with torch.cuda.stream(s2):
            sp2 = cache.ready_subset(2, [0], stream=moe.stream_handle(s2))
            assert sp2 == sp
            for _ in range(20):
                outs.append(moe.moe_layer(g, sp2, [1.0], x, ws2))
        # Both plans released with their kernels still queued on s1 and s2.
        cache.release(1)
        cache.release(2)
        # Evict the slot: expert 1's bytes land where expert 0 was read.
        miss = cache.plan(3, 0, [1])
        assert miss == [1]
        cache.fetch(3, [hosts[1].data_ptr()])
        cache.release(3)
        torch.cuda.synchronize()
        ref = want.cpu().numpy().view(np.uint32)
        for o in outs:
            assert np.array_equal(o.cpu().numpy().view(np.uint32), ref)
    finally:
        cache.close()
