#!/usr/bin/env python3
"""Routed-expert MXFP4 decode benchmark on one MI355X.

Workload: a bank of 384 synthetic MXFP4 experts
(hidden 7168, intermediate 2048, raw-v1 spans of 23,396,352 B, 8.98 GB) resident
in HBM; 1000 seeded tokens, each with fp32 N(0,1) router logits over the 384
experts and a bf16 N(0,1) activation.  One step = one token-layer: the device
router picks the top 16 experts (softmax weights over them), then the gate/up
projections with SiLU-GLU and the down projection with the route-ordered
weighted combine write a bf16 output row.  Inputs are resident in HBM when the
timed region starts.

Printed: one JSON line with the step throughput, the roofline of the dominant
kernel (algorithmic bytes per launch / average launch duration measured with
HIP events on the launch stream), parity of sampled tokens against the fp64
oracle, and the reference CPU path (tools/fused_gemv_batch.c, compiled from the
reference sources into oracle/_ref) timed on this host over a bounded sample of
the same tokens.

    python bench.py [--steps K] [--warmup W] [--cpu-seconds S] [--no-cpu]
    python bench.py --copy-calibration   # plain 1 GiB device copies, for scaling
                                         # rocprofv3 FETCH_SIZE / WRITE_SIZE
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

METRIC = "achieved HBM GB/s + MoE-layer decode tokens/s (16 experts, MXFP4, batch 1)"
HIDDEN, INTER, N_BANK, TOP_K, N_TOKENS = 7168, 2048, 384, 16, 1000
SEED = 20261201
HBM_PEAK_GBS = 8000.0

# Algorithmic bytes (what the computation must move at least once).
MAT_BYTES = INTER * HIDDEN // 2 + INTER * (HIDDEN // 32)  # one 2048x7168 MXFP4 matrix: 7,798,784
SPAN = 3 * MAT_BYTES                                      # 23,396,352
X_BYTES = HIDDEN * 2                                      # bf16 activation
OUT_BYTES = HIDDEN * 2                                    # bf16 output
LOGIT_BYTES = N_BANK * 4
H_BYTES = TOP_K * INTER * 4                               # fp32 h handed from gate/up to down
LAYER_BYTES = TOP_K * SPAN + X_BYTES + LOGIT_BYTES + OUT_BYTES  # 374,371,840
# Per launch of each decode kernel.  The fused kernel (the default path) reads
# the logits, x and all 48 matrices, writes h and reads it back, and writes the
# output row.  On the two-launch path gate/up (with the router folded in) reads
# the logits, x and 32 gate/up matrices and writes h; down reads 16 down
# matrices and h and writes the output row.
KERNEL_BYTES = {
    "decode_fused": 3 * TOP_K * MAT_BYTES + X_BYTES + LOGIT_BYTES + 2 * H_BYTES + OUT_BYTES,
    "glu_decode": 2 * TOP_K * MAT_BYTES + X_BYTES + LOGIT_BYTES + H_BYTES,
    "down_decode": TOP_K * MAT_BYTES + H_BYTES + OUT_BYTES,
}
KERNEL_FLOPS = {
    "decode_fused": 3 * 2 * TOP_K * INTER * HIDDEN,
    "glu_decode": 2 * 2 * TOP_K * INTER * HIDDEN,
    "down_decode": 2 * TOP_K * INTER * HIDDEN,
}


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse() -> argparse.Namespace:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=N_TOKENS)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--cpu-seconds", type=float, default=12.0,
                    help="CPU work budget for the reference CPU baseline sample")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--parity-tokens", type=int, default=2)
    ap.add_argument("--verify-only", action="store_true",
                    help="time only the config-3 verify paths (one JSON line)")
    ap.add_argument("--verify-batches", type=int, default=20,
                    help="verify batches timed per M for the config-3 line (0 skips it)")
    ap.add_argument("--streamed", action="store_true",
                    help="run BASELINE configs[4] (8 layers x 384 experts streamed from pinned host "
                         "memory through a 24 GB HBM cache) instead of the decode bench")
    ap.add_argument("--streamed-tokens", type=int, default=1000,
                    help="timed tokens of --streamed (the default bench line carries a "
                         "300-token run; 0 there skips it)")
    ap.add_argument("--streamed-line-tokens", type=int, default=300)
    ap.add_argument("--spine-only", action="store_true",
                    help="print only the spine-projection timings (K3 spine shapes)")
    ap.add_argument("--no-spine", action="store_true", help="skip the spine timings")
    ap.add_argument("--no-k3", action="store_true", help="skip the K3 caller-route decode object")
    ap.add_argument("--k3-only", action="store_true",
                    help="print only the K3 caller-route decode object (k3_decode)")
    ap.add_argument("--block-only", action="store_true",
                    help="print only the whole-K3-MoE-block timings")
    ap.add_argument("--no-block", action="store_true", help="skip the K3 MoE block timings")
    ap.add_argument("--settle-ms", type=float, default=100.0,
                    help="untimed back-to-back decode steps for this long before the warm-up "
                         "steps (0 disables)")
    ap.add_argument("--transient-probe", action="store_true",
                    help="print per-phase decode step times from idle (the load-onset "
                         "transient the settle phase waits out) and exit")
    ap.add_argument("--no-single", action="store_true",
                    help="skip the config-0 (one GEMV) and config-1 (one expert) legs")
    ap.add_argument("--single-only", action="store_true",
                    help="print only the config-0 and config-1 objects")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run 4 plain device copies of 1 GiB (the known-size kernel "
                         "the HBM byte counters are scaled by) and exit")
    return ap.parse_args()


COPY_CAL_BYTES = 1 << 30


def copy_calibration() -> int:
    """Four device-to-device copies of COPY_CAL_BYTES with torch's copy kernel:
    each reads and writes exactly 1 GiB of HBM, so FETCH_SIZE / WRITE_SIZE per
    dispatch of this kernel give the counters' scale on this device."""
    import torch

    torch.cuda.set_device(0)
    src = torch.ones(COPY_CAL_BYTES // 4, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(4):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes": COPY_CAL_BYTES, "copies": 4}), flush=True)
    return 0


def cpu_nproc() -> int:
    """CPUs this process may run on (what `nproc` prints)."""
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1


def cpu_threads() -> int:
    """Pool threads of the reference CPU path: min(nproc, 32), the reference
    pool's own cap (K3_MAX_THREADS, tools/fused_gemv_batch.c:36)."""
    return max(1, min(cpu_nproc(), 32))


MT_THREADS_CAP = 16  # mxfp4_gemv_mt splits rows over at most 16 threads (tools/fused_gemv.c:734)


def cpu_token_fn(bank_host_base: int, threads: int):
    """The reference CPU composition of one token-layer (provider_moe.cpp:867-971
    with SiLU-GLU in place of SiTU): mxfp4_moe_layer over the routed experts'
    gate/up matrices with the shared x, fp32 SiLU-GLU, mxfp4_gemv_batch over
    their down matrices, then the route-ordered combine.  Returns
    token(ids, weights, x_f32, stride) -> fp32 output, reading expert e's span
    at bank_host_base + e * stride (host memory)."""
    import oracle

    ref = oracle.ref()
    ref.mxfp4_pool_init(threads)
    u8p = C.POINTER(C.c_uint8)
    f32p = C.POINTER(C.c_float)
    off = oracle.expert_offsets(HIDDEN, INTER)
    rows13 = (C.c_int * (2 * TOP_K))(*([INTER] * (2 * TOP_K)))
    cols13 = (C.c_int * (2 * TOP_K))(*([HIDDEN] * (2 * TOP_K)))
    rows2 = (C.c_int * TOP_K)(*([HIDDEN] * TOP_K))
    cols2 = (C.c_int * TOP_K)(*([INTER] * TOP_K))
    gu = np.empty(2 * TOP_K * INTER, np.float32)
    yb = np.empty((TOP_K, HIDDEN), np.float32)

    def token(ids, w, x_f32: np.ndarray, stride: int = SPAN, base: int | None = None) -> np.ndarray:
        b0 = bank_host_base if base is None else base
        k = len(ids)
        p13 = (u8p * (2 * TOP_K))()
        s13 = (u8p * (2 * TOP_K))()
        p2 = (u8p * TOP_K)()
        s2 = (u8p * TOP_K)()
        for j, e in enumerate(ids):
            b = b0 + int(e) * stride
            p13[2 * j] = C.cast(b + off[0], u8p)
            s13[2 * j] = C.cast(b + off[1], u8p)
            p13[2 * j + 1] = C.cast(b + off[4], u8p)
            s13[2 * j + 1] = C.cast(b + off[5], u8p)
            p2[j] = C.cast(b + off[2], u8p)
            s2[j] = C.cast(b + off[3], u8p)
        xt = np.ascontiguousarray(x_f32, dtype=np.float32)
        ref.mxfp4_moe_layer(p13, s13, rows13, cols13, 2 * k, xt.ctypes.data_as(f32p),
                            gu.ctypes.data_as(f32p), threads)
        g = gu[:2 * k * INTER].reshape(k, 2, INTER)[:, 0, :]
        u = gu[:2 * k * INTER].reshape(k, 2, INTER)[:, 1, :]
        with np.errstate(over="ignore"):
            h = np.ascontiguousarray(g / (np.float32(1.0) + np.exp(-g)) * u, dtype=np.float32)
        xs = (f32p * TOP_K)(*[h[j].ctypes.data_as(f32p) for j in range(k)])
        ys = (f32p * TOP_K)(*[yb[j].ctypes.data_as(f32p) for j in range(k)])
        ref.mxfp4_gemv_batch(p2, s2, xs, ys, rows2, cols2, k, threads)
        out = np.zeros(HIDDEN, np.float32)
        for j in range(k):
            out += np.float32(w[j]) * yb[j]
        return out

    return token


def cpu_baseline(bank_host: np.ndarray, logits: np.ndarray, x_f32: np.ndarray,
                 seconds: float, threads: int) -> tuple[dict, np.ndarray, int]:
    """The reference CPU composition for config 2 (cpu_token_fn) on the same
    tokens and bank.  Tokens are run in order until `seconds` of CPU work."""
    import oracle

    ref = oracle.ref()
    run = cpu_token_fn(bank_host.ctypes.data, threads)
    outs = []

    def token(t: int) -> np.ndarray:
        ids, w64 = oracle.topk_softmax(logits[t], TOP_K)
        return run(ids, w64.astype(np.float32), x_f32[t])

    token(0)  # warm the pool and the pages of the first token's experts
    n = 0
    t0 = time.perf_counter()
    while True:
        outs.append(token(n % logits.shape[0]))
        n += 1
        el = time.perf_counter() - t0
        if el >= seconds or n >= logits.shape[0]:
            break
    rate = n / el
    res = {
        "value": rate,
        "unit": "token-layers/s",
        **_cpu_env(threads),
        "kind": "reference",
        "sample": (f"first {n} of the {logits.shape[0]} tokens of the same workload, "
                   f"384-expert bank copied to host DRAM; mxfp4_moe_layer + fp32 SiLU-GLU + "
                   f"mxfp4_gemv_batch + ordered combine per token ({el:.1f} s)"),
        "achieved_gbs": rate * LAYER_BYTES / 1e9,
        "avx2": int(ref.mxfp4_have_avx2()),
    }
    return res, np.stack(outs), n


STREAM_LAYERS = 8
STREAM_SLOTS = 1025          # 24e9 B of HBM / 23,396,352 B per expert
STREAM_ZIPF = 1.1
STREAM_WARMUP_TOKENS = 200
STREAM_STAGING_SLOTS = 4     # pinned staging slots for layers held in pageable memory
STREAM_CHECK_TOKENS = 2      # tokens whose 8 layer outputs are checked against the oracle
STREAM_CPU_TOKENS = 4        # tokens of the CPU per-token compute figure


def stream_routes(n_layers: int, n_bank: int, total: int, seed: int) -> tuple[np.ndarray, np.ndarray]:
    """Per layer a seeded rank permutation of the experts; per token and layer
    16 distinct ranks drawn Zipf(STREAM_ZIPF) without replacement, returned as
    canonical ascending expert ids [total, layers, 16] and weights summing to 1."""
    rng = np.random.default_rng(seed)
    perms = [rng.permutation(n_bank) for _ in range(n_layers)]
    pz = np.arange(1, n_bank + 1, dtype=np.float64) ** -STREAM_ZIPF
    pz /= pz.sum()
    routes = np.empty((total, n_layers, TOP_K), dtype=np.int64)
    for t in range(total):
        for layer in range(n_layers):
            routes[t, layer] = np.sort(perms[layer][rng.choice(n_bank, TOP_K, replace=False, p=pz)])
    weights = rng.random((total, n_layers, TOP_K)).astype(np.float32)
    weights /= weights.sum(axis=2, keepdims=True)
    return routes, weights


def streamed_config4(n_tokens: int, cpu: bool = True) -> dict:
    """8 distinct layers x 384 experts (71.87 GB) in host
    memory, a 1,025-slot (24 GB) HBM LRU cache, 16 distinct experts per layer
    per token drawn Zipf(1.1) over a per-layer rank permutation (seeded).
    Each layer's 8.98 GB bank is pinned host memory where the host grants it;
    layers it refuses to pin are held in pageable memory, distinct bytes, and
    their misses go through the cache's pinned staging slots (a threaded host
    copy, then the DMA).  Per layer: plan -> fetch the misses (side-stream
    copies) -> resolve (the compute stream waits per expert) -> layer kernels
    -> RMS norm of the layer output (k3_hip_rms_norm; it is the next layer's
    fp32 x, as a model normalises between layers, so activations stay O(1))
    -> release, with no host synchronisation.  Reports tokens/s, the PCIe rate of the uploads, the hit rate, the
    misses served from pinned and from pageable layers, and the copy/compute
    overlap 1 - (wall - max(copy, compute)) / min(copy, compute), where compute
    is the same token sequence over resident experts and copy the same
    plan/fetch sequence with no kernels.  Then STREAM_CHECK_TOKENS tokens run
    through all 8 layers again with each layer's output checked against the
    fp64 oracle on that layer's host bytes, and the reference CPU path's
    per-token compute time (8 layers, cpu_token_fn on the host banks)."""
    import torch

    import oracle
    from deltafin_amd import _lib, moe

    torch.cuda.set_device(0)
    lib = _lib.load()
    if lib.k3_hip_moe_available(0) != 1:
        raise _lib.K3HipError(lib.k3_hip_moe_available(0), "k3_hip_moe_available")
    g = moe.preset(2)
    L, NB = STREAM_LAYERS, N_BANK
    t0 = time.perf_counter()
    hosts, pinned = [], []
    for layer in range(L):
        h = None
        if all(pinned):
            try:
                h = torch.empty(NB * SPAN, dtype=torch.uint8, pin_memory=True)
            except Exception as e:  # torch raises its accelerator error (a RuntimeError) on OOM
                log(f"streamed: pinning layer {layer} refused ({str(e).splitlines()[0]}); "
                    f"layers {layer}..{L - 1} go to pageable memory")
        if h is None:
            h = torch.empty(NB * SPAN, dtype=torch.uint8)
        hosts.append(h)
        pinned.append(bool(h.is_pinned()))
    t_alloc = time.perf_counter() - t0
    n_pinned = sum(pinned)
    log(f"streamed: {n_pinned} pinned + {L - n_pinned} pageable x {NB * SPAN / 1e9:.2f} GB "
        f"host banks in {t_alloc:.1f} s")
    bank = torch.empty(NB * SPAN, dtype=torch.uint8, device="cuda")
    for layer, h in enumerate(hosts):
        moe.synth_bank(g, bank, SPAN, NB, layer * NB, SEED)
        h.copy_(bank)
    torch.cuda.synchronize()
    log(f"streamed: host banks filled ({time.perf_counter() - t0:.1f} s)")

    total = STREAM_WARMUP_TOKENS + n_tokens
    routes, weights = stream_routes(L, NB, total + STREAM_CHECK_TOKENS, SEED + 4)

    cache = lib.k3_hip_cache_create(0, SPAN, STREAM_SLOTS, L, STREAM_STAGING_SLOTS)
    if not cache:
        raise _lib.K3HipError(-3, f"k3_hip_cache_create: {_lib.last_error()}")
    xs = [moe.synth_normal(HIDDEN, torch.float32, SEED + 5, 0),
          torch.empty(HIDDEN, dtype=torch.float32, device="cuda")]
    x_first = xs[0].clone()
    norm_w = torch.ones(HIDDEN, dtype=torch.float32, device="cuda")
    ws = moe.workspace(g, TOP_K)
    wsb, wsn = moe._ws_args(ws)
    st = moe.stream_handle()
    gref = C.byref(g)
    host_base = [hosts[layer].data_ptr() for layer in range(L)]
    u16 = C.c_uint16 * TOP_K
    missing = u16()
    n_missing = C.c_int(0)
    spans = (C.c_void_p * TOP_K)()
    srcs = (C.c_void_p * TOP_K)()
    plan_id = [0]
    miss_by_kind = [0, 0]  # misses served from pageable / pinned layers

    def layer_kernels(spans_arr, w, x_in, y_out, x_next) -> None:
        rc = lib.k3_hip_moe_layer_device(gref, spans_arr, w, TOP_K, x_in.data_ptr(),
                                         _lib.K3_DTYPE_F32, y_out.data_ptr(), _lib.K3_DTYPE_F32,
                                         wsb, wsn, st)
        if rc != 0:
            raise _lib.K3HipError(rc, "k3_hip_moe_layer_device")
        rc = lib.k3_hip_rms_norm(y_out.data_ptr(), norm_w.data_ptr(), x_next.data_ptr(), 1,
                                 HIDDEN, C.c_float(1e-5), st)
        if rc != 0:
            raise _lib.K3HipError(rc, "k3_hip_rms_norm")

    def layer_step(c, t: int, layer: int, x_in, y_out, x_next=None) -> None:
        ids = u16(*routes[t, layer].tolist())
        plan_id[0] += 1
        pid = plan_id[0]
        rc = lib.k3_hip_cache_plan(c, pid, layer, ids, TOP_K, missing, C.byref(n_missing))
        if rc != 0:
            raise _lib.K3HipError(rc, "k3_hip_cache_plan")
        for i in range(n_missing.value):
            srcs[i] = host_base[layer] + missing[i] * SPAN
        miss_by_kind[int(pinned[layer])] += n_missing.value
        rc = lib.k3_hip_cache_fetch(c, pid, srcs, n_missing.value)
        if rc != 0:
            raise _lib.K3HipError(rc, "k3_hip_cache_fetch")
        rc = lib.k3_hip_cache_resolve(c, pid, ids, TOP_K, spans, st)
        if rc != 0:
            raise _lib.K3HipError(rc, "k3_hip_cache_resolve")
        if x_in is not None:
            w = (C.c_float * TOP_K)(*weights[t, layer].tolist())
            layer_kernels(spans, w, x_in, y_out, y_out if x_next is None else x_next)
        lib.k3_hip_cache_release(c, pid)

    def run(c, first: int, count: int, kernels: bool = True) -> float:
        cur = 0
        torch.cuda.synchronize()
        t_start = time.perf_counter()
        for t in range(first, first + count):
            for layer in range(L):
                layer_step(c, t, layer, xs[cur] if kernels else None, xs[1 - cur])
                cur = 1 - cur
        torch.cuda.synchronize()
        return time.perf_counter() - t_start

    six = (C.c_longlong * 6)()
    run(cache, 0, STREAM_WARMUP_TOKENS)
    lib.k3_hip_cache_stats(cache, six)
    before = list(six)
    miss_by_kind[:] = [0, 0]
    wall = run(cache, STREAM_WARMUP_TOKENS, n_tokens)
    lib.k3_hip_cache_stats(cache, six)
    hits, misses = six[0] - before[0], six[1] - before[1]
    uploaded = six[5] - before[5]
    miss_pageable, miss_pinned = miss_by_kind

    # Sampled outputs: tokens past the timed ones, each through all 8 layers,
    # every layer's output (before the norm) checked against the fp64 oracle
    # on the host bank's bytes, with the exact x the layer consumed.
    worst = 0.0
    x_cur = x_first.clone()
    y32 = torch.empty(HIDDEN, dtype=torch.float32, device="cuda")
    x_nxt = torch.empty(HIDDEN, dtype=torch.float32, device="cuda")
    for t in range(total, total + STREAM_CHECK_TOKENS):
        for layer in range(L):
            layer_step(cache, t, layer, x_cur, y32, x_nxt)
            torch.cuda.synchronize()
            hb = hosts[layer].numpy()
            sp = [hb[int(e) * SPAN:(int(e) + 1) * SPAN] for e in routes[t, layer]]
            xin = x_cur.cpu().numpy()
            ref, mag = oracle.moe_layer_f64(sp, weights[t, layer].astype(np.float64), HIDDEN,
                                            INTER, oracle.ACT_SILU, xin)
            worst = max(worst, oracle.cond_rel_err(y32.cpu().numpy(), ref, mag, INTER))
            x_cur, x_nxt = x_nxt, x_cur
    lib.k3_hip_cache_destroy(cache)
    log(f"streamed: checked {STREAM_CHECK_TOKENS} tokens x {L} layers, max cond rel err {worst:.2e}")

    # Compute alone: the same routes over experts resident in the device bank.
    ptrs = [[(C.c_void_p * TOP_K)(*[bank.data_ptr() + int(e) * SPAN for e in routes[t, layer]])
             for layer in range(L)] for t in range(STREAM_WARMUP_TOKENS, total)]
    torch.cuda.synchronize()
    t_start = time.perf_counter()
    cur = 0
    for i, t in enumerate(range(STREAM_WARMUP_TOKENS, total)):
        for layer in range(L):
            w = (C.c_float * TOP_K)(*weights[t, layer].tolist())
            layer_kernels(ptrs[i][layer], w, xs[cur], xs[1 - cur], xs[1 - cur])
            cur = 1 - cur
    torch.cuda.synchronize()
    compute = time.perf_counter() - t_start
    # Copy alone: the same plan/fetch/release sequence on a fresh cache with
    # no layer kernels (the side stream carries exactly the streamed run's
    # uploads), warm-up tokens included and then timed like the run.
    cache2 = lib.k3_hip_cache_create(0, SPAN, STREAM_SLOTS, L, STREAM_STAGING_SLOTS)
    if not cache2:
        raise _lib.K3HipError(-3, f"k3_hip_cache_create: {_lib.last_error()}")
    run(cache2, 0, STREAM_WARMUP_TOKENS, kernels=False)
    copy = run(cache2, STREAM_WARMUP_TOKENS, n_tokens, kernels=False)
    lib.k3_hip_cache_destroy(cache2)
    # Context: H2D rate of one 1.5 GB copy from a pinned and from a pageable bank.
    probe = 64 * SPAN
    dst = torch.empty(probe, dtype=torch.uint8, device="cuda")
    rates = {}
    for kind, layer in (("pinned", pinned.index(True) if any(pinned) else None),
                        ("pageable", pinned.index(False) if not all(pinned) else None)):
        if layer is None:
            continue
        src = hosts[layer][:probe]
        dst.copy_(src, non_blocking=True)
        torch.cuda.synchronize()
        t_start = time.perf_counter()
        for _ in range(3):
            dst.copy_(src, non_blocking=True)
        torch.cuda.synchronize()
        rates[kind] = round(3 * probe / (time.perf_counter() - t_start) / 1e9, 2)
    overlap = 1.0 - (wall - max(copy, compute)) / min(copy, compute) if min(copy, compute) > 0 else None
    res = {
        "metric": "streamed-expert MoE tokens/s (8 layers, 16-of-384 per layer, host -> 24 GB HBM cache)",
        "value": round(n_tokens / wall, 2),
        "unit": "tokens/s",
        "higher_is_better": True,
        "tokens": n_tokens,
        "warmup_tokens": STREAM_WARMUP_TOKENS,
        "ms_per_token": round(wall * 1e3 / n_tokens, 3),
        "data": "synthetic",
        "config": {
            "workload": (f"BASELINE configs[4]: 8 distinct layers x 384 MXFP4 experts (71.87 GB) "
                         f"in host memory, {n_pinned} layer banks pinned and {L - n_pinned} "
                         f"pageable (the host refused to pin more; their misses go through "
                         f"{STREAM_STAGING_SLOTS} pinned staging slots), 1,025-slot (24 GB) HBM "
                         f"LRU, Zipf(1.1) routes of 16 distinct experts per layer, fp32 x "
                         f"RMS-normalised between layers"),
            "layers": L, "experts_per_layer": NB, "top_k": TOP_K, "cache_slots": STREAM_SLOTS,
            "zipf": STREAM_ZIPF, "pinned_layers": n_pinned, "pageable_layers": L - n_pinned,
            "host_bank_bytes_pinned": n_pinned * NB * SPAN,
            "host_bank_bytes_pageable": (L - n_pinned) * NB * SPAN,
            "staging_slots": STREAM_STAGING_SLOTS,
        },
        "hit_rate": round(hits / max(hits + misses, 1), 4),
        "misses_per_token": round(misses / n_tokens, 2),
        "misses_per_token_pinned_layers": round(miss_pinned / n_tokens, 2),
        "misses_per_token_pageable_layers": round(miss_pageable / n_tokens, 2),
        "pcie_gbs": round(uploaded / wall / 1e9, 2),
        "h2d_probe_gbs": rates,
        "compute_only_ms_per_token": round(compute * 1e3 / n_tokens, 3),
        "copy_only_ms_per_token": round(copy * 1e3 / n_tokens, 3),
        "overlap": None if overlap is None else round(overlap, 3),
        "host_alloc_s": round(t_alloc, 1),
        "parity": {"tokens_checked": STREAM_CHECK_TOKENS, "layers_each": L,
                   "max_cond_rel_err_fp32": worst, "tolerance": 1e-3, "pass": bool(worst <= 1e-3)},
    }
    if cpu:
        # The reference CPU path's compute per token (8 layers) on the host
        # banks; it has no streaming analog.
        threads = cpu_threads()
        run_cpu = cpu_token_fn(host_base[0], threads)
        xh = x_first.cpu().numpy()
        run_cpu(routes[0, 0], weights[0, 0], xh, SPAN, host_base[0])  # warm the pool
        t_start = time.perf_counter()
        for t in range(STREAM_WARMUP_TOKENS, STREAM_WARMUP_TOKENS + STREAM_CPU_TOKENS):
            xt = xh
            for layer in range(L):
                y = run_cpu(routes[t, layer], weights[t, layer], xt, SPAN, host_base[layer])
                xt = (y / np.sqrt(np.mean(y * y) + np.float32(1e-5))).astype(np.float32)
        per_tok = (time.perf_counter() - t_start) / STREAM_CPU_TOKENS
        res["cpu_baseline"] = {"value": round(1.0 / per_tok, 3), "unit": "tokens/s",
                               "ms_per_token": round(per_tok * 1e3, 1), **_cpu_env(threads),
                               "kind": "reference",
                               "sample": (f"{STREAM_CPU_TOKENS} tokens x {L} layers of the same "
                                          "routes, compute only (the host banks are the CPU's "
                                          "resident weights): mxfp4_moe_layer + fp32 SiLU-GLU + "
                                          "mxfp4_gemv_batch + ordered combine per layer")}
    del hosts, bank, dst
    return res


def _cpu_model() -> str:
    """The first CPU's /proc/cpuinfo identity: model name, vendor, family /
    model / stepping, and the number of packages and logical CPUs listed."""
    info: dict[str, str] = {}
    packages: set[str] = set()
    logical = 0
    try:
        for line in open("/proc/cpuinfo"):
            if ":" not in line:
                continue
            k, v = (s.strip() for s in line.split(":", 1))
            if k == "processor":
                logical += 1
            elif k == "physical id":
                packages.add(v)
            elif k in ("model name", "vendor_id", "cpu family", "model", "stepping") and k not in info:
                info[k] = v
    except OSError:
        return "unknown"
    name = info.get("model name", "unknown")
    return (f"{name} ({info.get('vendor_id', '?')} family {info.get('cpu family', '?')} model "
            f"{info.get('model', '?')} stepping {info.get('stepping', '?')}; "
            f"{max(len(packages), 1)} package(s), {logical} logical CPUs listed)")


def _cpu_env(threads: int) -> dict:
    return {"cores": threads, "nproc": cpu_nproc(), "cpu_model": _cpu_model()}


def main() -> int:
    args = parse()
    if args.copy_calibration:
        return copy_calibration()
    if args.streamed:
        print(json.dumps(streamed_config4(args.streamed_tokens, not args.no_cpu)), flush=True)
        return 0
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only: the routed-expert path is built and measured "
              f"on a single MI355X (asked for --gpus {args.gpus}); multi-GPU sharding is a "
              f"design note, not a measured configuration.", file=sys.stderr, flush=True)
        return 2
    import torch

    import oracle
    from deltafin_amd import _lib, moe, synth

    assert torch.cuda.is_available(), "bench.py needs a HIP device"
    torch.cuda.set_device(0)
    lib = _lib.load()
    avail = lib.k3_hip_moe_available(0)
    if avail != 1:
        raise _lib.K3HipError(avail, "k3_hip_moe_available")
    props = torch.cuda.get_device_properties(0)
    log(f"device {props.name} {getattr(props, 'gcnArchName', '')} CUs={props.multi_processor_count}")

    g = moe.preset(2)
    assert g.hidden == HIDDEN and g.intermediate == INTER and g.expert_span == SPAN
    stride = SPAN
    bank = torch.empty(N_BANK * stride, dtype=torch.uint8, device="cuda")
    moe.synth_bank(g, bank, stride, N_BANK, 0, SEED)
    logits = moe.synth_normal(N_TOKENS * N_BANK, torch.float32, SEED, 1).view(N_TOKENS, N_BANK)
    x = moe.synth_normal(N_TOKENS * HIDDEN, torch.bfloat16, SEED, 2).view(N_TOKENS, HIDDEN)
    out = torch.empty((N_TOKENS, HIDDEN), dtype=torch.bfloat16, device="cuda")
    ws = moe.workspace(g, TOP_K)
    torch.cuda.synchronize()
    log(f"bank of {N_BANK} experts ({N_BANK * stride / 1e9:.2f} GB) synthesised in HBM")

    if args.verify_only:
        print(json.dumps(_verify_config3(moe, _lib, g, bank, stride, max(1, args.verify_batches))),
              flush=True)
        return 0
    if args.single_only:
        print(json.dumps(_single_configs(moe, _lib, oracle, g, bank, stride, args.cpu_seconds,
                                         args.no_cpu)), flush=True)
        return 0
    if args.k3_only:
        print(json.dumps(_k3_decode_bench(moe, _lib, oracle, 300,
                                          None if args.no_cpu else args.cpu_seconds / 2, bank)),
              flush=True)
        return 0
    if args.spine_only or args.block_only:
        del bank
        torch.cuda.empty_cache()
        print(json.dumps(_spine_bench() if args.spine_only else _k3_block_bench()), flush=True)
        return 0

    fn = lib.k3_hip_moe_route_layer_device
    gref = C.byref(g)
    ws_base, ws_bytes = moe._ws_args(ws)
    st = moe.stream_handle()
    bank_p, lg_p, x_p, o_p = bank.data_ptr(), logits.data_ptr(), x.data_ptr(), out.data_ptr()
    BF16 = _lib.K3_DTYPE_BF16

    def step(t: int) -> None:
        t %= N_TOKENS
        rc = fn(gref, bank_p, stride, N_BANK, lg_p + t * N_BANK * 4, TOP_K, x_p + t * HIDDEN * 2,
                BF16, o_p + t * HIDDEN * 2, BF16, None, None, ws_base, ws_bytes, st)
        if rc != 0:
            raise _lib.K3HipError(rc, "k3_hip_moe_route_layer_device")

    if args.transient_probe:
        print(json.dumps(_transient_probe(step)), flush=True)
        return 0

    # ---- settle (untimed): back-to-back decode steps until the GPU has run
    # them for --settle-ms.  From idle, the first ~1.5 ms of this load run at
    # full speed, the next ~10-20 ms at ~15 % lower throughput in both decode
    # kernels, then the rate holds steady (bench.py --transient-probe; the
    # same token can take 51 us in that window and 42.5 us after it).  The
    # timed window starts in the steady state.
    settle_steps = 0
    t_settle = time.perf_counter()
    while args.settle_ms > 0:
        for i in range(100):
            step(settle_steps + i)
        settle_steps += 100
        torch.cuda.synchronize()
        if (time.perf_counter() - t_settle) * 1e3 >= args.settle_ms:
            break
    settle_ms = (time.perf_counter() - t_settle) * 1e3
    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    log(f"settle {settle_steps} steps ({settle_ms:.1f} ms), warmup {args.warmup} steps done")

    # ---- timed region: exactly K steps, synchronised on both sides
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        step(args.warmup + i)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = wall * 1e3 / args.steps
    # Device time of the same K steps, in a pass of its own (events recorded
    # on the stream around them; kept out of the timed region above).
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0.record()
    for i in range(args.steps):
        step(args.warmup + i)
    ev1.record()
    torch.cuda.synchronize()
    dev_ms = ev0.elapsed_time(ev1)
    log(f"timed {args.steps} steps: wall {wall * 1e3:.2f} ms; device {dev_ms:.2f} ms (next pass)")

    # ---- per-kernel durations: the same K steps again, each launch bracketed by
    # HIP events on the launch stream
    _lib.timing_begin(4 * args.steps + 16)
    for i in range(args.steps):
        step(args.warmup + i)
    kern, dropped = _lib.timing_end()
    log("kernels: " + ", ".join(f"{k} {v['avg_ms'] * 1e3:.2f} us x{v['launches']}" for k, v in kern.items()))
    dom = max((k for k in kern if k in KERNEL_BYTES), key=lambda k: kern[k]["total_ms"])
    dom_s = kern[dom]["avg_ms"] / 1e3
    achieved = KERNEL_BYTES[dom] / dom_s / 1e9
    traffic = _traffic_from_profiles(dom)
    roofline = {
        "bound": "hbm",
        "kernel": dom,
        "achieved": round(achieved, 1),
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(achieved / HBM_PEAK_GBS, 4),
        "traffic": traffic,
        "traffic_source": (f"not measured in this run: read from "
                           f"{TRAFFIC_FILE.relative_to(ROOT)} (rocprofv3 --pmc FETCH_SIZE and "
                           f"WRITE_SIZE per dispatch, each scaled by its reading for a 1 GiB "
                           f"device copy)") if traffic is not None else None,
        "algorithmic_bytes_per_launch": KERNEL_BYTES[dom],
        "avg_launch_us": round(dom_s * 1e6, 3),
    }

    # ---- the same K steps on the other decode path, for comparison: the
    # opt-in fused single launch (k_decode_fused) when the default two-launch
    # path ran, and the reverse
    fused_ran = "decode_fused" in kern
    prev = _lib.set_fused_decode(not fused_ran)
    try:
        for i in range(20):
            step(i)
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        for i in range(args.steps):
            step(args.warmup + i)
        torch.cuda.synchronize()
        wall2 = time.perf_counter() - t1
        _lib.timing_begin(4 * args.steps + 16)
        for i in range(args.steps):
            step(args.warmup + i)
        kern2, _ = _lib.timing_end()
    finally:
        _lib.set_fused_decode(prev)
    alt = {"path": "two-launch" if fused_ran else "fused single launch",
           "value": round(args.steps / wall2, 2), "unit": "token-layers/s",
           "ms_per_step": round(wall2 * 1e3 / args.steps, 5),
           "kernels_us": {k: round(v["avg_ms"] * 1e3, 3) for k, v in kern2.items()}}
    log(f"{alt['path']} path: {alt['value']:.1f} tok/s, " +
        ", ".join(f"{k} {v} us" for k, v in alt["kernels_us"].items()))

    # ---- parity of sampled tokens (fp32 output before rounding) against the fp64 oracle
    parity = _parity(moe, oracle, synth, g, bank, stride, logits, x, ws, args.parity_tokens)

    value = args.steps / wall
    res = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "token-layers/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "settle": {"steps": settle_steps, "ms": round(settle_ms, 1),
                   "note": "untimed decode steps run back to back before the warm-up steps, "
                           "so the timed window starts after the GPU's load-onset transient "
                           "(bench.py --transient-probe; profiles/decode_config2_load_transient.md)"},
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic",
        "config": {
            "workload": ("16-of-384 routed-expert MXFP4 decode layer, batch 1 "
                         "(BASELINE configs[2]): hidden 7168, intermediate 2048, SiLU-GLU, "
                         "device top-16 + softmax router, bf16 x/out, 1000 seeded tokens"),
            "n_bank": N_BANK, "top_k": TOP_K, "hidden": HIDDEN, "intermediate": INTER,
            "bank_bytes": N_BANK * SPAN, "layer_bytes_per_token": LAYER_BYTES,
            "weights": "MXFP4 (E2M1 + E8M0 per 32)", "x_dtype": "bf16", "out_dtype": "bf16",
        },
        "achieved_gbs": round(value * LAYER_BYTES / 1e9, 1),
        "hbm_frac": round(value * LAYER_BYTES / 1e9 / HBM_PEAK_GBS, 4),
        "device_ms_per_step": round(dev_ms / args.steps, 5),
        "roofline": roofline,
        "kernels_us": {k: round(v["avg_ms"] * 1e3, 3) for k, v in kern.items()},
        "timing_dropped": dropped,
        "other_decode_path": alt,
        "parity": parity,
    }
    if not args.no_single:
        res.update(_single_configs(moe, _lib, oracle, g, bank, stride, args.cpu_seconds,
                                   args.no_cpu))
    if args.verify_batches > 0:
        res["verify"] = _verify_config3(moe, _lib, g, bank, stride, args.verify_batches,
                                        None if args.no_cpu else args.cpu_seconds)
    if not args.no_k3:
        res["k3_decode"] = _k3_decode_bench(moe, _lib, oracle, 300,
                                            None if args.no_cpu else args.cpu_seconds / 2, bank)
    if not args.no_spine:
        res["spine"] = _spine_bench()
    if not args.no_block:
        res["k3_block"] = _k3_block_bench()
    if args.streamed_line_tokens > 0:
        try:
            res["streamed"] = streamed_config4(args.streamed_line_tokens, not args.no_cpu)
        except Exception as e:  # reported in the line rather than losing the decode result
            log(f"streamed run failed: {e}")
            res["streamed"] = {"error": str(e).splitlines()[0]}
    if not args.no_cpu:
        log("cpu baseline: copying the bank to host DRAM")
        bank_host = host_bank(bank)
        lg_host = logits.cpu().numpy()
        x_host = x.float().cpu().numpy()  # bf16 -> fp32 widening outside the timed region
        threads = cpu_threads()
        cpu, cpu_out, n_cpu = cpu_baseline(bank_host, lg_host, x_host, args.cpu_seconds, threads)
        # Cross-check on exactly the tokens the CPU ran: the GPU path computes
        # them again, untimed, into their output rows.  The GPU rows are
        # bf16-rounded (relative step 2^-8): the difference is reported per
        # token against the token's largest |output|.
        for t in range(n_cpu):
            step(t)
        torch.cuda.synchronize()
        gpu_out = out[:n_cpu].float().cpu().numpy()
        scale = np.max(np.abs(cpu_out), axis=1)
        cpu["gpu_bf16_vs_cpu_max_diff_over_max_abs"] = float(
            np.max(np.max(np.abs(gpu_out - cpu_out), axis=1) / scale))
        cpu["cross_check_rows"] = n_cpu
        res["cpu_baseline"] = cpu
        log(f"cpu baseline {cpu['value']:.2f} tok/s with {threads} threads")
    else:
        res["cpu_baseline"] = None
    print(json.dumps(res), flush=True)
    return 0


CFG0_BYTES = MAT_BYTES + HIDDEN * 4 + INTER * 4    # 7,835,648: W + fp32 x + fp32 y
CFG1_BYTES = SPAN + X_BYTES + HIDDEN * 4           # 23,439,360: 3 matrices + bf16 x + fp32 out
SINGLE_ROTATE = 64                                 # distinct matrices / experts per rotation


def _roofline(nbytes: float, seconds: float) -> dict:
    gbs = nbytes / seconds / 1e9
    return {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None}


def _single_configs(moe, _lib, oracle, g, bank, stride, cpu_seconds: float, no_cpu: bool,
                    launches: int = 640) -> dict:
    """BASELINE configs[0] and [1] on the resident bank.

    Config 0: one 2048 x 7168 MXFP4 GEMV, fp32 x ~N(0,1), fp32 y, batch 1
    (k3_hip_mxfp4_gemv, the k3_cuda_mxfp4_gemv counterpart).  The matrices
    are the gate matrices of SINGLE_ROTATE distinct experts of the bank (501
    MB, above the 256 MB Infinity Cache), launched round-robin back to back so
    no launch finds its matrix in a cache.  Config 1: one expert's SwiGLU FFN,
    y = down(silu(gate x) * (up x)), bf16 x, fp32 y, with fp32 accumulation
    (k3_hip_moe_layer_device with one expert of weight 1.0, exact), over
    SINGLE_ROTATE distinct experts (1.5 GB).  Each leg reports the host-timed
    rate of the back-to-back calls and the kernels' device time per call
    (dispatch stamps), GB/s over the algorithmic bytes, one call checked
    against the fp64 oracle, and the reference CPU path on the same matrices
    copied to host memory: config 0 through mxfp4_gemv_mt (threads created per
    call, at most 16) and the pooled mxfp4_gemv_batch with one matrix; config 1
    through mxfp4_moe_layer (gate and up) -> fp32 SiLU-GLU -> mxfp4_gemv_batch
    (down), the reference CPU composition (provider_moe.cpp:867-971)."""
    import torch

    lib = _lib.load()
    st = moe.stream_handle()
    off = moe.span_offsets(g)
    base = bank.data_ptr()
    n_rot = SINGLE_ROTATE
    res: dict = {}

    # ---------------- config 0
    x0 = moe.synth_normal(HIDDEN, torch.float32, SEED + 70, 1)
    y0 = torch.empty(INTER, dtype=torch.float32, device="cuda")
    mats = [(base + e * stride + off["w1p"], base + e * stride + off["w1s"]) for e in range(n_rot)]

    def gemv(i: int) -> None:
        p, s = mats[i % n_rot]
        rc = lib.k3_hip_mxfp4_gemv(p, s, x0.data_ptr(), y0.data_ptr(), INTER, HIDDEN, 1, st)
        if rc != 0:
            raise _lib.K3HipError(rc, "k3_hip_mxfp4_gemv")

    def timed_calls(fn, cls: list[str]) -> tuple[float, float]:
        for i in range(n_rot):
            fn(i)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(launches):
            fn(i)
        torch.cuda.synchronize()
        wall = (time.perf_counter() - t0) / launches
        _lib.timing_begin(4 * launches)
        for i in range(launches):
            fn(i)
        torch.cuda.synchronize()
        kern, _ = _lib.timing_end()
        dev = sum(kern[k]["total_ms"] for k in cls if k in kern) / 1e3 / launches
        seen[fn.__name__] = sorted(k for k in cls if k in kern)
        return wall, dev

    seen: dict[str, list[str]] = {}

    wall0, dev0 = timed_calls(gemv, ["gemv"])
    gemv(0)
    torch.cuda.synchronize()
    h_p = bank[off["w1p"]: off["w1p"] + INTER * HIDDEN // 2].cpu().numpy()
    h_s = bank[off["w1s"]: off["w1s"] + INTER * HIDDEN // 32].cpu().numpy()
    x0h = x0.cpu().numpy()
    ref0, mag0 = oracle.gemv_f64(h_p, h_s, x0h, INTER, HIDDEN, with_mag=True)
    err0 = oracle.cond_rel_err(y0.cpu().numpy(), ref0, mag0, HIDDEN)
    c0 = {
        "workload": ("BASELINE configs[0]: one 2048x7168 MXFP4 GEMV, fp32 x ~N(0,1), fp32 y, "
                     f"batch 1, round-robin over {n_rot} distinct matrices "
                     f"({n_rot * MAT_BYTES / 1e6:.0f} MB) so every launch streams HBM"),
        "algorithmic_bytes": CFG0_BYTES,
        "launches": launches,
        "us_per_call_wall": round(wall0 * 1e6, 3),
        "us_per_call_device": round(dev0 * 1e6, 3),
        "gemvs_per_s": round(1 / wall0, 1),
        "achieved_gbs_wall": round(CFG0_BYTES / wall0 / 1e9, 1),
        "roofline": _roofline(CFG0_BYTES, dev0),
        "parity": {"max_cond_rel_err": err0, "tolerance": 1e-3, "pass": bool(err0 <= 1e-3)},
    }
    log(f"config 0: {wall0 * 1e6:.2f} us/GEMV wall, {dev0 * 1e6:.2f} us device "
        f"({CFG0_BYTES / dev0 / 1e9:.0f} GB/s), parity {err0:.2e}")

    # ---------------- config 1
    x1 = moe.synth_normal(HIDDEN, torch.bfloat16, SEED + 71, 1)
    y1 = torch.empty(HIDDEN, dtype=torch.float32, device="cuda")
    ws = moe.workspace(g, 1)
    wsb, wsn = moe._ws_args(ws)
    one = (C.c_float * 1)(1.0)
    experts = [(C.c_void_p * 1)(base + e * stride) for e in range(n_rot)]
    gref = C.byref(g)

    def expert(i: int) -> None:
        rc = lib.k3_hip_moe_layer_device(gref, experts[i % n_rot], one, 1, x1.data_ptr(),
                                         _lib.K3_DTYPE_BF16, y1.data_ptr(), _lib.K3_DTYPE_F32,
                                         wsb, wsn, st)
        if rc != 0:
            raise _lib.K3HipError(rc, "k3_hip_moe_layer_device")

    wall1, dev1 = timed_calls(expert, ["glu_decode", "down_decode", "decode_fused", "decode_chain"])
    expert(0)
    torch.cuda.synchronize()
    span0 = bank[:SPAN].cpu().numpy()
    x1h = x1.float().cpu().numpy()
    ref1, _, mag1 = oracle.expert_f64(span0, HIDDEN, INTER, oracle.ACT_SILU, x1h)
    err1 = oracle.cond_rel_err(y1.cpu().numpy(), ref1, mag1, INTER)
    c1 = {
        "workload": ("BASELINE configs[1]: one expert SwiGLU FFN at batch 1, gate/up 2048x7168 "
                     "and down 7168x2048 MXFP4, bf16 x ~N(0,1), fp32 y, fp32 accumulation, "
                     f"round-robin over {n_rot} distinct experts ({n_rot * SPAN / 1e9:.2f} GB)"),
        "algorithmic_bytes": CFG1_BYTES,
        "launches": launches,
        "kernels": seen.get("expert", []),
        "us_per_call_wall": round(wall1 * 1e6, 3),
        "us_per_call_device": round(dev1 * 1e6, 3),
        "experts_per_s": round(1 / wall1, 1),
        "achieved_gbs_wall": round(CFG1_BYTES / wall1 / 1e9, 1),
        "roofline": _roofline(CFG1_BYTES, dev1),
        "parity": {"max_cond_rel_err": err1, "tolerance": 1e-3, "pass": bool(err1 <= 1e-3)},
    }
    log(f"config 1: {wall1 * 1e6:.2f} us/expert wall, {dev1 * 1e6:.2f} us device "
        f"({CFG1_BYTES / dev1 / 1e9:.0f} GB/s), parity {err1:.2e}")

    if not no_cpu:
        c0["cpu_baseline"], c1["cpu_baseline"] = _single_cpu(
            oracle, bank, stride, off, x0h, x1h, cpu_seconds)
    res["config0"] = c0
    res["config1"] = c1
    return res


def _single_cpu(oracle, bank, stride, off, x0h: np.ndarray, x1h: np.ndarray,
                seconds: float) -> tuple[dict, dict]:
    """The reference CPU kernels on the config-0 matrices and config-1 experts
    (host copies of the same bytes), each timed for about seconds / 3."""
    ref = oracle.ref()
    u8p, f32p = C.POINTER(C.c_uint8), C.POINTER(C.c_float)
    threads = cpu_threads()
    mt = min(cpu_nproc(), MT_THREADS_CAP)
    ref.mxfp4_pool_init(threads)
    n_rot = SINGLE_ROTATE
    hb = host_bank(bank)
    host = [hb[e * stride: e * stride + SPAN] for e in range(n_rot)]
    y0 = np.empty(INTER, np.float32)
    x0 = np.ascontiguousarray(x0h, dtype=np.float32)

    def rate(fn, budget: float) -> tuple[float, int]:
        fn(0)
        n, t0 = 0, time.perf_counter()
        while True:
            fn(n)
            n += 1
            el = time.perf_counter() - t0
            if el >= budget:
                return el / n, n

    def gemv_mt(i: int) -> None:
        h = host[i % n_rot]
        ref.mxfp4_gemv_mt(h[off["w1p"]:].ctypes.data_as(u8p), h[off["w1s"]:].ctypes.data_as(u8p),
                          x0.ctypes.data_as(f32p), y0.ctypes.data_as(f32p), INTER, HIDDEN, mt)

    rows1 = (C.c_int * 1)(INTER)
    cols1 = (C.c_int * 1)(HIDDEN)
    ys = (f32p * 1)(y0.ctypes.data_as(f32p))
    xs = (f32p * 1)(x0.ctypes.data_as(f32p))

    def gemv_pool(i: int) -> None:
        h = host[i % n_rot]
        ps = (u8p * 1)(h[off["w1p"]:].ctypes.data_as(u8p))
        ss = (u8p * 1)(h[off["w1s"]:].ctypes.data_as(u8p))
        ref.mxfp4_gemv_batch(ps, ss, xs, ys, rows1, cols1, 1, threads)

    t_mt, n_mt = rate(gemv_mt, seconds / 3)
    t_pool, n_pool = rate(gemv_pool, seconds / 6)
    env = _cpu_env(threads)
    c0 = {"value": round(CFG0_BYTES / t_mt / 1e9, 2), "unit": "GB/s", **env, "mt_threads": mt,
          "kind": "reference",
          "sample": (f"{n_mt} mxfp4_gemv_mt calls ({mt} threads, created per call) round-robin "
                     f"over the same {n_rot} matrices in host DRAM"),
          "us_per_call": round(t_mt * 1e6, 1),
          "pool_batch1": {"us_per_call": round(t_pool * 1e6, 1),
                          "gbs": round(CFG0_BYTES / t_pool / 1e9, 2), "threads": threads,
                          "calls": n_pool},
          "avx2": int(ref.mxfp4_have_avx2())}

    x1 = np.ascontiguousarray(x1h, dtype=np.float32)  # bf16 -> fp32 outside the timed region
    gu = np.empty(2 * INTER, np.float32)
    y1 = np.empty(HIDDEN, np.float32)
    rows13 = (C.c_int * 2)(INTER, INTER)
    cols13 = (C.c_int * 2)(HIDDEN, HIDDEN)
    rows2 = (C.c_int * 1)(HIDDEN)
    cols2 = (C.c_int * 1)(INTER)
    y1s = (f32p * 1)(y1.ctypes.data_as(f32p))

    def expert(i: int) -> None:
        h = host[i % n_rot]
        p13 = (u8p * 2)(h[off["w1p"]:].ctypes.data_as(u8p), h[off["w3p"]:].ctypes.data_as(u8p))
        s13 = (u8p * 2)(h[off["w1s"]:].ctypes.data_as(u8p), h[off["w3s"]:].ctypes.data_as(u8p))
        ref.mxfp4_moe_layer(p13, s13, rows13, cols13, 2, x1.ctypes.data_as(f32p),
                            gu.ctypes.data_as(f32p), threads)
        g_, u_ = gu[:INTER], gu[INTER:]
        with np.errstate(over="ignore"):
            hh = np.ascontiguousarray(g_ / (np.float32(1.0) + np.exp(-g_)) * u_, dtype=np.float32)
        p2 = (u8p * 1)(h[off["w2p"]:].ctypes.data_as(u8p))
        s2 = (u8p * 1)(h[off["w2s"]:].ctypes.data_as(u8p))
        hs = (f32p * 1)(hh.ctypes.data_as(f32p))
        ref.mxfp4_gemv_batch(p2, s2, hs, y1s, rows2, cols2, 1, threads)

    t_e, n_e = rate(expert, seconds / 2)
    c1 = {"value": round(CFG1_BYTES / t_e / 1e9, 2), "unit": "GB/s", **env, "kind": "reference",
          "sample": (f"{n_e} experts round-robin over the same {n_rot} experts in host DRAM: "
                     f"mxfp4_moe_layer (gate, up) + fp32 SiLU-GLU + mxfp4_gemv_batch (down)"),
          "us_per_call": round(t_e * 1e6, 1), "avx2": int(ref.mxfp4_have_avx2())}
    log(f"config 0/1 cpu: gemv_mt {t_mt * 1e6:.0f} us, pool {t_pool * 1e6:.0f} us, "
        f"expert {t_e * 1e6:.0f} us")
    return c0, c1


def _transient_probe(step) -> dict:
    """Decode step rates in phases from a cold start, to show the GPU's
    load-onset transient: host-timed µs per step of each phase (the per-launch
    kernel durations come from running this under rocprofv3 --kernel-trace).
    Tokens are those of the config-2 workload; `same` phases repeat tokens 5-24,
    `new` ones take tokens never run before in the process."""
    import torch

    phases = (("warm5", 0, 5, 0.0), ("first20", 5, 20, 0.0), ("same20", 5, 20, 0.0),
              ("same20_after_idle_0.5s", 5, 20, 0.5), ("new20", 500, 20, 0.0),
              ("run1000", 0, 1000, 0.0), ("same20_after_run", 5, 20, 0.0),
              ("same20_after_idle_1s", 5, 20, 1.0), ("new20_after_idle_1s", 300, 20, 1.0))
    out = []
    for name, first, n, idle in phases:
        if idle:
            time.sleep(idle)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(n):
            step(first + i)
        torch.cuda.synchronize()
        us = (time.perf_counter() - t0) * 1e6 / n
        log(f"transient probe {name}: {us:.2f} us/step")
        out.append({"phase": name, "first_token": first, "steps": n, "idle_before_s": idle,
                    "us_per_step": round(us, 2)})
    return {"transient_probe": out}


TRAFFIC_FILE = ROOT / "profiles" / "hbm_traffic_decode_config2.txt"


def _traffic_from_profiles(kernel: str):
    """HBM bytes per launch measured by rocprofv3 PMC runs (FETCH_SIZE + WRITE_SIZE,
    each scaled by what the counter reads for a plain copy of known size),
    recorded as `<kernel> <bytes_per_launch>` lines; '#' lines are comments.
    None when the file or the kernel's line is absent."""
    if not TRAFFIC_FILE.exists():
        return None
    for line in TRAFFIC_FILE.read_text().splitlines():
        if line.startswith("#"):
            continue
        f = line.split()
        if len(f) >= 2 and f[0] == kernel:
            try:
                return int(float(f[1]))
            except ValueError:
                return None
    return None


# The verify matrix-core path multiplies fp4 weights by fp8 activation terms:
# v_mfma_scale_f32_16x16x128_f8f6f4 with one fp8 operand runs at the dense fp8
# rate of MI355X (5.0 PFLOP/s).
MFMA_PEAK_FP8_TFLOPS = 5000.0
MFMA_FLOPS = 2 * 16 * 16 * 128  # one 16x16x128 block-scaled MFMA
X_TERMS, H_TERMS = 2, 3         # fp8 terms per bf16 x row / fp32 h row
PARITY_SPLIT = 2                # MFMA rows per weight row in a parity-split tile


def _mfma_issued_per_expert() -> int:
    """MFMA instructions the union kernels issue per unique expert: gate and up
    (I/16 row tiles each, H/128 K steps, one per x term) and down (H/16 row
    tiles, I/128 K steps, one per h term), times 2 for the parity split (a
    tile's 16 MFMA rows hold 8 weight rows, each as an even and an odd K
    step).  Each covers 16 token columns."""
    glu = 2 * (INTER // 16) * (HIDDEN // 128) * X_TERMS
    down = (HIDDEN // 16) * (INTER // 128) * H_TERMS
    return PARITY_SPLIT * (glu + down)


VERIFY_SETTLE_S = 0.05


def _verify_batches(moe, _lib, g, bank, stride, logits, x, batches: int) -> dict:
    """Time `batches` verify calls (after a 50 ms settle phase and 3 warm-up
    calls) on each path:
    AUTO (the library's choice), the matrix-core union path and one decode
    layer per position; per-kernel stamps for the union path."""
    import torch

    n, m = logits.shape[0], logits.shape[1]
    y = torch.empty((n, m, HIDDEN), dtype=torch.bfloat16, device="cuda")
    ws = moe.workspace(g, m * TOP_K, m)
    base, nbytes = moe._ws_args(ws)
    st = moe.stream_handle()
    lib = _lib.load()
    ids = torch.empty((n, m, TOP_K), dtype=torch.int32, device="cuda")
    wts = torch.empty((n, m, TOP_K), dtype=torch.float32, device="cuda")

    def routed(i: int) -> None:
        rc = lib.k3_hip_moe_verify_route_device(
            C.byref(g), bank.data_ptr(), stride, N_BANK, logits[i].data_ptr(), m, TOP_K,
            x[i].data_ptr(), _lib.K3_DTYPE_BF16, y[i].data_ptr(), _lib.K3_DTYPE_BF16,
            ids[i].data_ptr(), wts[i].data_ptr(), base, nbytes, st)
        if rc != 0:
            raise _lib.K3HipError(rc, "k3_hip_moe_verify_route_device")

    call = routed

    def timed(stamps: bool):
        # Settle: the batches back to back for VERIFY_SETTLE_S of host time
        # (past the load-onset transient a cold GPU shows), then 3 warm-up
        # calls, then the timed window.
        t_end = time.perf_counter() + VERIFY_SETTLE_S
        i = 0
        while time.perf_counter() < t_end:
            call(i % n)
            i += 1
            if i % n == 0:
                torch.cuda.synchronize()
        for i in range(3):
            call(i)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(3, n):
            call(i)
        torch.cuda.synchronize()
        sec = (time.perf_counter() - t0) / batches
        kern = None
        if stamps:
            _lib.timing_begin(64 * n)
            for i in range(3, n):
                call(i)
            torch.cuda.synchronize()
            kern, _ = _lib.timing_end()
        return sec, kern

    res = {}
    for path, mode in (("auto", _lib.VERIFY_AUTO), ("union_mfma", _lib.VERIFY_UNION_MFMA),
                       ("positions", _lib.VERIFY_POSITIONS)):
        prev = _lib.set_verify_mode(mode)
        try:
            res[path] = timed(path != "positions")
        finally:
            _lib.set_verify_mode(prev)
    # The same routes handed over as caller routes (k3_hip_moe_verify_device:
    # span tables and weights, the provider's execute_positions call), on
    # AUTO and on the per-position path (runs of equal edge counts batched).
    ids_h, w_h = ids.cpu().numpy(), wts.cpu().numpy()
    tables = []
    for i in range(n):
        ptrs = (C.c_void_p * (m * TOP_K))(*[bank.data_ptr() + int(e) * stride
                                             for e in ids_h[i].ravel()])
        ww = (C.c_float * (m * TOP_K))(*[float(v) for v in w_h[i].ravel()])
        tables.append((ptrs, ww))
    offs = (C.c_int * (m + 1))(*[p * TOP_K for p in range(m + 1)])

    def caller(i: int) -> None:
        rc = lib.k3_hip_moe_verify_device(C.byref(g), tables[i][0], tables[i][1], offs, m,
                                          x[i].data_ptr(), _lib.K3_DTYPE_BF16, y[i].data_ptr(),
                                          _lib.K3_DTYPE_BF16, base, nbytes, st)
        if rc != 0:
            raise _lib.K3HipError(rc, "k3_hip_moe_verify_device")

    call = caller
    for path, mode in (("caller_auto", _lib.VERIFY_AUTO), ("caller_positions", _lib.VERIFY_POSITIONS)):
        prev = _lib.set_verify_mode(mode)
        try:
            res[path] = timed(True)
        finally:
            _lib.set_verify_mode(prev)
    union = float(np.mean([len(set(ids[i].cpu().numpy().ravel().tolist())) for i in range(3, n)]))
    auto_path = "union_mfma" if "glu_mfma" in res["auto"][1] else "positions"
    sec = res["auto"][0]
    nbytes_alg = union * SPAN + m * (X_BYTES + LOGIT_BYTES + OUT_BYTES)
    useful = m * (KERNEL_FLOPS["glu_decode"] + KERNEL_FLOPS["down_decode"])
    issued = union * _mfma_issued_per_expert() * MFMA_FLOPS
    usec, kern = res["union_mfma"]
    kus = {k: round(v["total_ms"] * 1e3 / batches, 2) for k, v in kern.items()}
    mfma_s = (kus.get("glu_mfma", 0.0) + kus.get("down_mfma", 0.0)) * 1e-6
    out = {
        "default_path": auto_path,
        "us_per_batch": round(sec * 1e6, 1),
        "token_layers_per_s": round(m / sec, 1),
        "union_experts": round(union, 1),
        "edges": m * TOP_K,
        "algorithmic_bytes": int(nbytes_alg),
        "achieved_gbs": round(nbytes_alg / sec / 1e9, 1),
        "hbm_frac": round(nbytes_alg / sec / 1e9 / HBM_PEAK_GBS, 4),
        "union_mfma_us_per_batch": round(usec * 1e6, 1),
        "union_mfma_gbs": round(nbytes_alg / usec / 1e9, 1),
        "positions_us_per_batch": round(res["positions"][0] * 1e6, 1),
        "union_mfma_speedup_vs_positions": round(res["positions"][0] / usec, 3),
        "union_mfma_kernels_us": kus,
        "glu_mfma_gbs": round(union * 2 * MAT_BYTES / (kus["glu_mfma"] * 1e-6) / 1e9, 1)
        if kus.get("glu_mfma") else None,
        "down_mfma_gbs": round(union * MAT_BYTES / (kus["down_mfma"] * 1e-6) / 1e9, 1)
        if kus.get("down_mfma") else None,
        # Useful = the layer's own multiply-adds (2 flops per weight and real
        # token) over the two matrix-core kernels' time; issued = every MFMA
        # the kernels issue (16 token columns each, padding and parity split
        # included), which is what keeps the matrix cores busy.
        "mfma_util": round(useful / mfma_s / (MFMA_PEAK_FP8_TFLOPS * 1e12), 5) if mfma_s else None,
        "mfma_useful_tflops": round(useful / mfma_s / 1e12, 2) if mfma_s else None,
        "mfma_issued_tflops": round(issued / mfma_s / 1e12, 1) if mfma_s else None,
        "mfma_issued_util": round(issued / mfma_s / (MFMA_PEAK_FP8_TFLOPS * 1e12), 4)
        if mfma_s else None,
        "useful_tflops_union_mfma": round(useful / usec / 1e12, 2),
        "caller_route": _caller_summary(res, nbytes_alg, batches),
    }
    log(f"verify M={m}: auto -> {auto_path} {sec * 1e6:.1f} us/batch (union {union:.1f} of "
        f"{m * TOP_K} edges); union/mfma {usec * 1e6:.1f} us, per-position "
        f"{res['positions'][0] * 1e6:.1f} us; mfma kernels {kus}")
    return out


# The reference's own routed layer (provider_moe.h:40-42; K3 preset): 16 of
# 896 experts, hidden 3584, intermediate 3072, SiTU, fp32 activations in and
# out, caller routes.
K3_BANK, K3_HIDDEN, K3_INTER = 896, 3584, 3072
K3_MAT = K3_INTER * K3_HIDDEN // 2 + K3_INTER * (K3_HIDDEN // 32)  # 5,849,088 per matrix
K3_SPAN = 3 * K3_MAT                                                 # 17,547,264
K3_H_BYTES = TOP_K * K3_INTER * 4
K3_KERNEL_BYTES = {
    "glu_decode": 2 * TOP_K * K3_MAT + K3_HIDDEN * 4 + K3_H_BYTES,
    "down_decode": TOP_K * K3_MAT + K3_H_BYTES + K3_HIDDEN * 4,
}
K3_LAYER_BYTES = TOP_K * K3_SPAN + 2 * K3_HIDDEN * 4                  # 280,784,896


def _decode_caller(moe, _lib, g, bank, stride: int, n_bank: int, x_dtype, tokens: int,
                   seed: int, settle_s: float = 0.05):
    """Decode layers with caller routes through k3_hip_moe_layer_device (the
    provider's per-token call): `tokens` tokens, each 16 distinct experts
    drawn uniformly from the bank with positive weights summing to one, x
    N(0,1) in x_dtype, fp32 out.  Returns (result, ids, weights, x, out) after
    a settle phase, a timed pass and a kernel-stamp pass."""
    import torch

    lib = _lib.load()
    rng = np.random.default_rng(seed)
    ids = np.stack([rng.choice(n_bank, TOP_K, replace=False) for _ in range(tokens)])
    w = rng.random((tokens, TOP_K)).astype(np.float32) + 0.05
    w = (w / w.sum(axis=1, keepdims=True)).astype(np.float32)
    x = moe.synth_normal(tokens * g.hidden, x_dtype, seed, 2).view(tokens, g.hidden)
    out = torch.empty((tokens, g.hidden), dtype=torch.float32, device="cuda")
    ws = moe.workspace(g, TOP_K)
    base, nbytes = moe._ws_args(ws)
    st = moe.stream_handle()
    xb = 2 if x_dtype == torch.bfloat16 else 4
    xcode = _lib.K3_DTYPE_BF16 if x_dtype == torch.bfloat16 else _lib.K3_DTYPE_F32
    tables = [((C.c_void_p * TOP_K)(*[bank.data_ptr() + int(e) * stride for e in ids[t]]),
               (C.c_float * TOP_K)(*[float(v) for v in w[t]])) for t in range(tokens)]
    gref = C.byref(g)
    x_p, o_p = x.data_ptr(), out.data_ptr()

    def step(t: int) -> None:
        t %= tokens
        rc = lib.k3_hip_moe_layer_device(gref, tables[t][0], tables[t][1], TOP_K,
                                         x_p + t * g.hidden * xb, xcode, o_p + t * g.hidden * 4,
                                         _lib.K3_DTYPE_F32, base, nbytes, st)
        if rc != 0:
            raise _lib.K3HipError(rc, "k3_hip_moe_layer_device")

    t_end = time.perf_counter() + settle_s
    i = 0
    while time.perf_counter() < t_end:
        step(i)
        i += 1
        if i % 100 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for t in range(tokens):
        step(t)
    torch.cuda.synchronize()
    sec = (time.perf_counter() - t0) / tokens
    _lib.timing_begin(4 * tokens + 16)
    for t in range(tokens):
        step(t)
    kern, _ = _lib.timing_end()
    return sec, kern, ids, w, x, out


def _k3_decode_bench(moe, _lib, oracle, tokens: int = 300, cpu_seconds: float | None = None,
                     bank_cfg2=None) -> dict:
    """The drop-in's own workload: the K3 routed decode layer (16 of 896
    experts, 3584 / 3072, SiTU, fp32 x and out) with caller routes through
    k3_hip_moe_layer_device, as the provider calls it
    (provider_moe.cpp:1664-1669); roofline per decode kernel; the reference
    CPU path beside it (the whole-set mxfp4_moe_expert_set,
    tools/fused_gemv_batch.c:465-518, on host copies of the same experts).
    With bank_cfg2, also the benchmark geometry (preset 2) with caller routes
    and fp32 / bf16 x, against its router-mode kernels."""
    import torch

    g = moe.preset(1)
    assert g.hidden == K3_HIDDEN and g.intermediate == K3_INTER and g.expert_span == K3_SPAN
    bank = torch.empty(K3_BANK * K3_SPAN, dtype=torch.uint8, device="cuda")
    moe.synth_bank(g, bank, K3_SPAN, K3_BANK, 0, SEED + 80)
    torch.cuda.synchronize()
    sec, kern, ids, w, x, out = _decode_caller(moe, _lib, g, bank, K3_SPAN, K3_BANK,
                                               torch.float32, tokens, SEED + 81)
    kus = {k: round(v["avg_ms"] * 1e3, 3) for k, v in kern.items()}
    roof = {k: {"us": kus[k], "gbs": round(K3_KERNEL_BYTES[k] / (kus[k] * 1e-6) / 1e9, 1),
                "frac": round(K3_KERNEL_BYTES[k] / (kus[k] * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                "algorithmic_bytes": K3_KERNEL_BYTES[k]}
            for k in K3_KERNEL_BYTES if k in kus}
    res = {
        "workload": (f"K3 routed decode layer: {TOP_K} of {K3_BANK} experts ({K3_BANK * K3_SPAN / 1e9:.1f}"
                     f" GB bank in HBM), hidden {K3_HIDDEN}, intermediate {K3_INTER}, SiTU, fp32 x "
                     f"and out, caller routes (16 distinct uniform experts, positive weights) "
                     f"through k3_hip_moe_layer_device, {tokens} seeded tokens"),
        "us_per_token": round(sec * 1e6, 2),
        "token_layers_per_s": round(1.0 / sec, 1),
        "layer_bytes_per_token": K3_LAYER_BYTES,
        "achieved_gbs": round(K3_LAYER_BYTES / sec / 1e9, 1),
        "hbm_frac": round(K3_LAYER_BYTES / sec / 1e9 / HBM_PEAK_GBS, 4),
        "kernels_us": kus,
        "roofline": roof,
    }
    # Oracle check of two tokens (fp32 out against the fp64 oracle).
    errs = []
    for t in (0, tokens - 1):
        spans = [oracle.synth_expert(SEED + 80, int(e), K3_HIDDEN, K3_INTER) for e in ids[t]]
        ref, mag = oracle.moe_layer_f64(spans, w[t].astype(np.float64), K3_HIDDEN, K3_INTER,
                                        g.activation, x[t].cpu().numpy())
        errs.append(oracle.cond_rel_err(out[t].cpu().numpy(), ref, mag, K3_INTER))
    res["oracle_max_cond_rel_err"] = float(max(errs))
    if cpu_seconds:
        threads = cpu_threads()
        ref = oracle.ref()
        ref.mxfp4_pool_init(threads)
        host = {}
        n, el, diffs = 0, 0.0, []
        xh = x.cpu().numpy()
        outh = out.cpu().numpy()
        while n < tokens and el < cpu_seconds:
            for e in ids[n]:
                if int(e) not in host:
                    host[int(e)] = bank[int(e) * K3_SPAN:(int(e) + 1) * K3_SPAN].cpu().numpy()
            spans = [host[int(e)] for e in ids[n]]
            if n == 0:
                oracle.ref_expert_set(spans, w[n], xh[n], K3_HIDDEN, K3_INTER, threads)  # warm
            t0 = time.perf_counter()
            y = oracle.ref_expert_set(spans, w[n], xh[n], K3_HIDDEN, K3_INTER, threads)
            el += time.perf_counter() - t0
            diffs.append(float(np.max(np.abs(y - outh[n])) / np.max(np.abs(y))))
            n += 1
        rate = n / el
        res["cpu_baseline"] = {
            "value": round(rate, 2), "unit": "token-layers/s", **_cpu_env(threads),
            "kind": "reference",
            "sample": (f"first {n} tokens of the same workload: mxfp4_moe_expert_set (SiTU, "
                       f"{threads} pool threads) on host copies of their experts ({el:.1f} s of "
                       f"calls)"),
            "achieved_gbs": round(rate * K3_LAYER_BYTES / 1e9, 1),
            "gpu_vs_cpu_max_diff_over_max_abs": float(max(diffs)),
        }
    del bank
    torch.cuda.empty_cache()
    if bank_cfg2 is not None:
        g2 = moe.preset(2)
        cmp = {}
        for name, dt in (("fp32_x", torch.float32), ("bf16_x", torch.bfloat16)):
            s2, k2, *_ = _decode_caller(moe, _lib, g2, bank_cfg2, SPAN, N_BANK, dt, tokens,
                                        SEED + 82)
            cmp[name] = {"us_per_token": round(s2 * 1e6, 2),
                         "kernels_us": {k: round(v["avg_ms"] * 1e3, 3) for k, v in k2.items()}}
        res["preset2_caller_routes"] = cmp
    return res


def _caller_summary(res: dict, nbytes_alg: float, batches: int) -> dict:
    """k3_hip_moe_verify_device over the routes the device router chose, as a
    provider hands them over (span tables + weights): AUTO and the per-position
    path, whose runs of equal edge counts are one position-batched launch
    pair; the kernel split shows which path AUTO took."""
    out = {}
    for path in ("caller_auto", "caller_positions"):
        sec, kern = res[path]
        kus = {k: round(v["total_ms"] * 1e3 / batches, 2) for k, v in (kern or {}).items()}
        out[path[len("caller_"):]] = {
            "us_per_batch": round(sec * 1e6, 1),
            "achieved_gbs": round(nbytes_alg / sec / 1e9, 1),
            "hbm_frac": round(nbytes_alg / sec / 1e9 / HBM_PEAK_GBS, 4),
            "kernels_us": kus,
        }
    out["auto_path"] = "union_mfma" if "glu_mfma" in out["auto"]["kernels_us"] else "positions"
    return out


# The K3 spine around the routed experts (provider_moe.cpp:428-447): rows x
# columns of each resident matrix, in the order one token runs them.
SPINE_SHAPES = (("router", 896, 7168), ("routed_down", 3584, 7168), ("routed_up", 7168, 3584),
                ("shared_gate_up", 12288, 7168), ("shared_down", 7168, 6144))
SPINE_POSITIONS = (1, 4, 16)
SPINE_ROTATE_BYTES = 600_000_000  # > the 256 MB Infinity Cache: every pass streams HBM


def _spine_bench(launches: int = 24) -> dict:
    """Spine projections at the K3 shapes, BF16 and row-int8, at 1, 4 and 16
    positions: each shape is launched `launches` times over enough distinct
    copies that no launch finds its matrix in the Infinity Cache; `us` is the
    kernel's device time per launch (the library's dispatch stamps).
    Algorithmic bytes = matrix (+ int8 row scales) + activation + output."""
    import torch

    from deltafin_amd import _lib, spine

    out = {"positions": list(SPINE_POSITIONS), "launches": launches}
    gen = torch.Generator(device="cuda")
    gen.manual_seed(SEED)
    for kind in ("bf16", "int8"):
        per_kind = {}
        tok_us = {p: 0.0 for p in SPINE_POSITIONS}
        tok_bytes = {p: 0 for p in SPINE_POSITIONS}
        for name, rows, cols in SPINE_SHAPES:
            mat_bytes = rows * cols * (2 if kind == "bf16" else 1) + (rows * 4 if kind == "int8" else 0)
            copies = max(2, -(-SPINE_ROTATE_BYTES // mat_bytes))
            if kind == "bf16":
                mats = [(torch.randn(rows, cols, device="cuda", generator=gen) * 0.02)
                        .to(torch.bfloat16).view(torch.int16) for _ in range(copies)]
            else:
                mats = [torch.randint(-128, 128, (rows, cols), dtype=torch.int8, device="cuda",
                                      generator=gen) for _ in range(copies)]
                scales = torch.rand(rows, device="cuda", generator=gen) * 1e-3
            xs = torch.randn(max(SPINE_POSITIONS), cols, device="cuda", generator=gen)
            y = torch.empty(max(SPINE_POSITIONS), rows, device="cuda")
            res = {}
            for p in SPINE_POSITIONS:
                x = xs[:p]

                def run(i):
                    if kind == "bf16":
                        spine.bf16_gemv(mats[i % copies], x, out=y[:p])
                    else:
                        spine.int8_gemv(mats[i % copies], scales, x, out=y[:p])

                for i in range(copies):
                    run(i)
                torch.cuda.synchronize()
                _lib.timing_begin(launches)
                for i in range(launches):
                    run(i)
                torch.cuda.synchronize()
                kern, _ = _lib.timing_end()
                us = kern["spine_gemv"]["total_ms"] * 1e3 / kern["spine_gemv"]["launches"]
                alg = mat_bytes + p * cols * 4 + p * rows * 4
                res[f"p{p}"] = {"us": round(us, 2), "gbs": round(alg / us / 1e3, 1),
                                "hbm_frac": round(alg / us / 1e3 / HBM_PEAK_GBS, 4)}
                tok_us[p] += us
                tok_bytes[p] += alg
            per_kind[name] = {"rows": rows, "cols": cols, "matrix_bytes": mat_bytes, **res}
            del mats
            torch.cuda.empty_cache()
        per_kind["all_five"] = {f"p{p}": {"us": round(tok_us[p], 2),
                                          "gbs": round(tok_bytes[p] / tok_us[p] / 1e3, 1),
                                          "hbm_frac": round(tok_bytes[p] / tok_us[p] / 1e3
                                                            / HBM_PEAK_GBS, 4)}
                                for p in SPINE_POSITIONS}
        out[kind] = per_kind
        log(f"spine {kind}: " + ", ".join(
            f"{n} {per_kind[n]['p1']['us']}us/{per_kind[n]['p1']['gbs']}GB/s" for n, _, _ in
            SPINE_SHAPES) + f"; all five p1 {per_kind['all_five']['p1']}")
    return out


K3_BLOCK_EXPERTS = 896
K3_BLOCK_POSITIONS = (1, 4, 8, 16)


def _k3_block_bench(calls: int = 20) -> dict:
    """The whole K3 MoE block (k3_hip_moe_block_device) at the reference's
    geometry: BF16 spine (router 896 x 7168, routed_down, routed_up, shared
    gate / up / down; 380 MB) and a bank of 896 raw-v1 K3 experts (15.7 GB),
    fresh N(0,1) hidden rows per call (so the routes move).  `device_us` sums
    the kernels' dispatch stamps per call; `wall_us` is the host-timed call
    rate.  Algorithmic bytes per position-batch = spine + unique routed
    experts x 17,547,264 + activations."""
    import torch

    from deltafin_amd import _lib, moe, spine

    g = _lib.preset(1)
    stride = g.expert_span
    bank = torch.empty(K3_BLOCK_EXPERTS * stride, dtype=torch.uint8, device="cuda")
    moe.synth_bank(g, bank, stride, K3_BLOCK_EXPERTS, 0, SEED)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(SEED + 1)
    H, R, S = 7168, 3584, 6144

    def mat(rows, cols):
        return (torch.randn(rows, cols, device="cuda", generator=gen) * 0.02).to(
            torch.bfloat16).view(torch.int16)

    sp = spine.MoeSpine("bf16", mat(K3_BLOCK_EXPERTS, H),
                        torch.randn(K3_BLOCK_EXPERTS, device="cuda", generator=gen) * 0.01,
                        mat(R, H), 1 + 0.1 * torch.randn(R, device="cuda", generator=gen),
                        mat(H, R), mat(S, H), mat(S, H), mat(H, S))
    spine_bytes = 2 * (K3_BLOCK_EXPERTS * H + 2 * R * H + 3 * S * H)
    out = {"experts": K3_BLOCK_EXPERTS, "spine_bytes": spine_bytes, "calls": calls,
           "expert_span": stride}
    for P in K3_BLOCK_POSITIONS:
        ws = spine.moe_block_workspace(sp, g, P)
        xs = torch.randn(calls + 3, P, H, device="cuda", generator=gen)
        for i in range(3):
            spine.moe_block(sp, g, bank, stride, xs[i], workspace=ws)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        ids_all = []
        for i in range(3, calls + 3):
            _, ids, _ = spine.moe_block(sp, g, bank, stride, xs[i], workspace=ws)
            ids_all.append(ids)
        torch.cuda.synchronize()
        wall = (time.perf_counter() - t0) / calls
        _lib.timing_begin(64 * calls)
        for i in range(3, calls + 3):
            spine.moe_block(sp, g, bank, stride, xs[i], workspace=ws)
        torch.cuda.synchronize()
        kern, _ = _lib.timing_end()
        kus = {k: round(v["total_ms"] * 1e3 / calls, 2) for k, v in kern.items()}
        dev = sum(kus.values())
        union = float(np.mean([len(set(t.cpu().numpy().ravel().tolist())) for t in ids_all]))
        alg = spine_bytes + union * stride + P * (2 * H + R) * 4
        out[f"p{P}"] = {
            "wall_us": round(wall * 1e6, 1), "device_us": round(dev, 1),
            "token_layers_per_s": round(P / wall, 1), "union_experts": round(union, 1),
            "algorithmic_bytes": int(alg), "achieved_gbs": round(alg / wall / 1e9, 1),
            "hbm_frac": round(alg / wall / 1e9 / HBM_PEAK_GBS, 4), "kernels_us": kus}
        log(f"k3 block P={P}: {wall * 1e6:.1f} us/call (device {dev:.1f}), "
            f"{alg / wall / 1e9:.0f} GB/s, kernels {kus}")
    del bank
    torch.cuda.empty_cache()
    return out


def _verify_config3(moe, _lib, g, bank, stride, batches: int,
                    cpu_seconds: float | None = None) -> dict:
    """batched speculative verify over the same resident
    bank: M positions, each with its own top-16 of 384 N(0,1) logits and bf16
    x.  Each M is timed on the library's default path (AUTO: the matrix-core
    union kernels when the expected union is under 92% of the edges, else one
    decode layer per position) and on both paths explicitly.  A second case,
    `shared_M16`, gives 16 positions logits with a common N(0,1) component
    (logits = z_common + 0.5 z_position, as consecutive draft tokens of one
    sequence share much of their routing): there the union is small and the
    matrix cores carry a real small-M contraction.

    With cpu_seconds, each M also carries `cpu_per_row`: the reference CPU
    path as the reference runs a verify tile, one token's expert-set
    composition per position with no union amortisation (provider_moe.cpp:
    1092-1105; cpu_token_fn), timed on the same batches (about cpu_seconds / 4
    per M), beside the bytes that composition reads (M x 16 experts) and the
    union bytes the GPU reads."""
    import torch

    out = {}
    for m in (4, 8, 16):
        n = batches + 3
        logits = moe.synth_normal(n * m * N_BANK, torch.float32, SEED + 30 + m, 1).view(n, m, N_BANK)
        x = moe.synth_normal(n * m * HIDDEN, torch.bfloat16, SEED + 30 + m, 2).view(n, m, HIDDEN)
        out[f"M{m}"] = _verify_batches(moe, _lib, g, bank, stride, logits, x, batches)
        if cpu_seconds:
            out[f"M{m}"]["cpu_per_row"] = _verify_cpu(bank, logits, x, out[f"M{m}"],
                                                      cpu_seconds / 4)
    m = 16
    n = batches + 3
    common = moe.synth_normal(n * N_BANK, torch.float32, SEED + 60, 1).view(n, 1, N_BANK)
    own = moe.synth_normal(n * m * N_BANK, torch.float32, SEED + 60, 2).view(n, m, N_BANK)
    logits = (common + 0.5 * own).contiguous()
    x = moe.synth_normal(n * m * HIDDEN, torch.bfloat16, SEED + 60, 3).view(n, m, HIDDEN)
    out["shared_M16"] = _verify_batches(moe, _lib, g, bank, stride, logits, x, batches)
    return {"config": "BASELINE configs[3]: M positions each routing top-16 of 384, bf16 x/out; "
                      "us_per_batch on the default path; union_mfma_* on the matrix-core union "
                      "kernels (every routed expert read once per batch); mfma_util = the "
                      "layer's useful flops (2 per weight and routed token) / (gate/up + down "
                      "matrix-core kernel time x 5.0 PFLOP/s dense fp8); mfma_issued_util counts "
                      "every issued block-scaled MFMA (16 token columns each, padding and the "
                      "parity split included)",
            **out}


_HOST_BANK: dict = {}


def host_bank(bank) -> np.ndarray:
    """Host copy of the resident bank (made once per process)."""
    key = (bank.data_ptr(), bank.numel())
    if key not in _HOST_BANK:
        log("copying the bank to host DRAM for the CPU legs")
        _HOST_BANK.clear()
        _HOST_BANK[key] = bank.cpu().numpy()
    return _HOST_BANK[key]


def _verify_cpu(bank, logits, x, gpu: dict, seconds: float) -> dict:
    """The reference CPU composition of a verify tile: per position, that
    position's own top-16 through cpu_token_fn, batches in order (from batch 3,
    the GPU's first timed batch) until `seconds` of work."""
    import oracle

    threads = cpu_threads()
    hb = host_bank(bank)
    run = cpu_token_fn(hb.ctypes.data, threads)
    lg = logits.cpu().numpy()
    xf = x.float().cpu().numpy()  # bf16 -> fp32 widening outside the timed region
    n, m = lg.shape[0], lg.shape[1]
    routes = [[oracle.topk_softmax(lg[i, p], TOP_K) for p in range(m)] for i in range(n)]
    run(routes[0][0][0], routes[0][0][1].astype(np.float32), xf[0, 0])  # warm the pool
    done, t0 = 0, time.perf_counter()
    while True:
        i = 3 + done % max(n - 3, 1)
        for p in range(m):
            ids, w = routes[i][p]
            run(ids, w.astype(np.float32), xf[i, p])
        done += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    per_batch = el / done
    nbytes = m * LAYER_BYTES
    return {"ms_per_batch": round(per_batch * 1e3, 2), "token_layers_per_s": round(m / per_batch, 1),
            "bytes_read_per_batch": nbytes, "achieved_gbs": round(nbytes / per_batch / 1e9, 1),
            "union_bytes_per_batch_gpu": gpu["algorithmic_bytes"],
            "gpu_speedup": round(per_batch * 1e6 / gpu["us_per_batch"], 1),
            "batches": done, **_cpu_env(threads), "kind": "reference",
            "sample": (f"{done} verify batches of {m} positions: per position "
                       "mxfp4_moe_layer + fp32 SiLU-GLU + mxfp4_gemv_batch + ordered combine "
                       "(no union amortisation, as the reference CPU path)")}


def _parity(moe, oracle, synth, g, bank, stride, logits, x, ws, n_tokens: int) -> dict:
    import torch

    if n_tokens <= 0:
        return {"tokens_checked": 0}
    worst = 0.0
    ids_ok = True
    host_bank = {}
    for t in range(n_tokens):
        o32, ids, wts = moe.moe_route_layer(g, bank, stride, N_BANK, logits[t], TOP_K, x[t], ws,
                                            out_dtype=torch.float32)
        torch.cuda.synchronize()
        lg = logits[t].cpu().numpy()
        rid, rw = oracle.topk_softmax(lg, TOP_K)
        ids_ok &= ids.cpu().numpy().tolist() == rid.tolist()
        spans = []
        for e in rid:
            e = int(e)
            if e not in host_bank:
                host_bank[e] = bank[e * stride: e * stride + SPAN].cpu().numpy()
            spans.append(host_bank[e])
        xf = x[t].float().cpu().numpy()
        ref, mag = oracle.moe_layer_f64(spans, rw, HIDDEN, INTER, oracle.ACT_SILU, xf)
        worst = max(worst, oracle.cond_rel_err(o32.cpu().numpy(), ref, mag, INTER))
    log(f"parity: {n_tokens} tokens, max cond rel err {worst:.3e}, top-k identical {ids_ok}")
    return {"tokens_checked": n_tokens, "max_cond_rel_err_fp32": worst, "tolerance": 1e-3,
            "topk_ids_identical": bool(ids_ok), "pass": bool(ids_ok and worst <= 1e-3)}


if __name__ == "__main__":
    sys.exit(main())
