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
