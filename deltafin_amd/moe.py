"""Host-side operators over the gfx950 library, mirroring the reference's
interface for the routed-expert path.

Reference counterparts:
  mxfp4_gemv          k3_cuda_mxfp4_gemv (tools/cuda_moe_kernels.cu:331-339) /
                      mxfp4_gemv (tools/fused_gemv.c:1021-1043)
  moe_launch          k3_cuda_moe_launch (tools/cuda_moe_kernels.cu:341-417)
  moe_layer           k3_metal_moe_layer (tools/metal_moe.mm:829-837) and the
                      per-expert loop + ordered_route_reduce of
                      provider_cuda_moe.cpp:1203-1258, :252-289
  moe_layer_desc      k3_metal_moe_layer_desc_v1 (tools/metal_moe_abi.h:59-61)
  moe_positions_desc  k3_metal_moe_positions_desc_v1 (tools/metal_moe_abi.h:63-66),
                      flat=True: k3_metal_moe_positions_flat_desc_v1
                      (tools/metal_moe.mm:1231-1243)
  ExpertCache         CudaMoeExpertCache (provider_cuda_moe.h:83-132)

Device tensors are torch tensors on the current HIP device; the current torch
stream is the launch stream.  Every call runs the HIP kernels; a failure raises
K3HipError with the library's message.  There is no CPU fallback.
"""
from __future__ import annotations

import ctypes as C
from typing import Sequence

import numpy as np
import torch

from . import _lib
from ._lib import (K3_ACT_SILU, K3_ACT_SITU, K3_DTYPE_BF16, K3_DTYPE_F32, K3HipError,
                   K3HipExpertDescriptorV1, K3HipGeometryV1, check, geometry, load, preset)

__all__ = [
    "K3_ACT_SILU", "K3_ACT_SITU", "K3HipError", "geometry", "preset", "span_offsets",
    "mxfp4_gemv", "moe_launch", "workspace", "moe_layer", "moe_route_layer",
    "moe_verify_route", "moe_verify", "moe_layer_desc", "moe_positions_desc",
    "ExpertCache", "synth_bank", "synth_normal", "stream_handle",
]


def stream_handle(stream: torch.cuda.Stream | None = None) -> int:
    s = stream if stream is not None else torch.cuda.current_stream()
    return int(s.cuda_stream)


def _dtype_code(t: torch.Tensor) -> int:
    if t.dtype == torch.float32:
        return K3_DTYPE_F32
    if t.dtype == torch.bfloat16:
        return K3_DTYPE_BF16
    raise TypeError(f"unsupported dtype {t.dtype}; expected float32 or bfloat16")


def _torch_dtype(code: int) -> torch.dtype:
    return torch.float32 if code == K3_DTYPE_F32 else torch.bfloat16


def _ptr(t: torch.Tensor) -> int:
    return int(t.data_ptr())


def span_offsets(g: K3HipGeometryV1) -> dict[str, int]:
    """Raw-v1 offsets w1p,w1s,w2p,w2s,w3p,w3s,span (provider_moe.cpp:217-243)."""
    h, i = g.hidden, g.intermediate
    w13p, w13s = i * h // 2, i * (h // 32)
    w2p, w2s = h * i // 2, h * (i // 32)
    off = {"w1p": 0, "w1s": w13p}
    off["w2p"] = off["w1s"] + w13s
    off["w2s"] = off["w2p"] + w2p
    off["w3p"] = off["w2s"] + w2s
    off["w3s"] = off["w3p"] + w13p
    off["span"] = off["w3s"] + w13s
    return off


def mxfp4_gemv(packed: torch.Tensor, scales: torch.Tensor, x: torch.Tensor, rows: int,
               cols: int, out_dtype: torch.dtype = torch.float32,
               out: torch.Tensor | None = None) -> torch.Tensor:
    """out[b, r] = sum_c W[r, c] x[b, c]; x is [cols] or [batches, cols]."""
    lib = load()
    batches = 1 if x.dim() == 1 else x.shape[0]
    if out is None:
        shape = (rows,) if x.dim() == 1 else (batches, rows)
        out = torch.empty(shape, dtype=out_dtype, device=x.device)
    rc = lib.k3_hip_mxfp4_gemv_ex(_ptr(packed), _ptr(scales), _ptr(x), _dtype_code(x), _ptr(out),
                                  _dtype_code(out), rows, cols, batches, stream_handle())
    check(rc, "k3_hip_mxfp4_gemv_ex")
    return out


def moe_launch(g: K3HipGeometryV1, span: torch.Tensor, x: torch.Tensor
               ) -> tuple[torch.Tensor, torch.Tensor]:
    """One expert for x [batches, hidden] fp32: returns (h, out)."""
    lib = load()
    x2 = x if x.dim() == 2 else x.unsqueeze(0)
    b = x2.shape[0]
    gate = torch.empty((b, g.intermediate), dtype=torch.float32, device=x.device)
    up = torch.empty_like(gate)
    out = torch.empty((b, g.hidden), dtype=torch.float32, device=x.device)
    rc = lib.k3_hip_moe_launch(C.byref(g), _ptr(span), _ptr(x2), b, _ptr(gate), _ptr(up),
                               _ptr(out), stream_handle())
    check(rc, "k3_hip_moe_launch")
    return gate, out


def workspace(g: K3HipGeometryV1, max_edges: int, max_positions: int = 1,
              device: str | torch.device = "cuda") -> torch.Tensor:
    """Zero-filled device workspace for the layer / verify calls."""
    n = int(load().k3_hip_moe_workspace_bytes(C.byref(g), max_edges, max_positions))
    if n == 0:
        raise K3HipError(-2, "k3_hip_moe_workspace_bytes")
    ws = torch.zeros(n + 256, dtype=torch.uint8, device=device)
    return ws


def _ws_args(ws: torch.Tensor) -> tuple[int, int]:
    base = _ptr(ws)
    aligned = (base + 255) & ~255
    return aligned, ws.numel() - (aligned - base)


def moe_layer(g: K3HipGeometryV1, experts: Sequence[int | torch.Tensor],
              weights: Sequence[float], x: torch.Tensor, ws: torch.Tensor,
              out_dtype: torch.dtype = torch.float32,
              out: torch.Tensor | None = None) -> torch.Tensor:
    """out = sum_e weights[e] * expert_e(x) (route order), experts = device spans."""
    lib = load()
    n = len(experts)
    ptrs = (C.c_void_p * max(n, 1))(*[e if isinstance(e, int) else _ptr(e) for e in experts])
    w = (C.c_float * max(n, 1))(*[float(v) for v in weights])
    if out is None:
        out = torch.empty(g.hidden, dtype=out_dtype, device=x.device)
    base, nbytes = _ws_args(ws)
    rc = lib.k3_hip_moe_layer_device(C.byref(g), ptrs, w, n, _ptr(x), _dtype_code(x), _ptr(out),
                                     _dtype_code(out), base, nbytes, stream_handle())
    check(rc, "k3_hip_moe_layer_device")
    return out


def moe_route_layer(g: K3HipGeometryV1, bank: torch.Tensor, stride: int, n_bank: int,
                    logits: torch.Tensor, top_k: int, x: torch.Tensor, ws: torch.Tensor,
                    out_dtype: torch.dtype = torch.float32,
                    out: torch.Tensor | None = None, want_route: bool = True):
    """Device router (top-k + softmax) + layer; returns (out, ids, weights)."""
    lib = load()
    if out is None:
        out = torch.empty(g.hidden, dtype=out_dtype, device=x.device)
    ids = torch.empty(top_k, dtype=torch.int32, device=x.device) if want_route else None
    wts = torch.empty(top_k, dtype=torch.float32, device=x.device) if want_route else None
    base, nbytes = _ws_args(ws)
    rc = lib.k3_hip_moe_route_layer_device(
        C.byref(g), _ptr(bank), stride, n_bank, _ptr(logits), top_k, _ptr(x), _dtype_code(x),
        _ptr(out), _dtype_code(out), _ptr(ids) if want_route else None,
        _ptr(wts) if want_route else None, base, nbytes, stream_handle())
    check(rc, "k3_hip_moe_route_layer_device")
    return out, ids, wts


def moe_verify_route(g: K3HipGeometryV1, bank: torch.Tensor, stride: int, n_bank: int,
                     logits: torch.Tensor, top_k: int, x: torch.Tensor, ws: torch.Tensor,
                     out_dtype: torch.dtype = torch.float32):
    """Batched verify with device routing; logits [M, n_bank], x [M, hidden]."""
    lib = load()
    m = x.shape[0]
    out = torch.empty((m, g.hidden), dtype=out_dtype, device=x.device)
    ids = torch.empty((m, top_k), dtype=torch.int32, device=x.device)
    wts = torch.empty((m, top_k), dtype=torch.float32, device=x.device)
    base, nbytes = _ws_args(ws)
    rc = lib.k3_hip_moe_verify_route_device(
        C.byref(g), _ptr(bank), stride, n_bank, _ptr(logits), m, top_k, _ptr(x),
        _dtype_code(x), _ptr(out), _dtype_code(out), _ptr(ids), _ptr(wts), base, nbytes,
        stream_handle())
    check(rc, "k3_hip_moe_verify_route_device")
    return out, ids, wts


def moe_verify(g: K3HipGeometryV1, edge_experts: Sequence[int | torch.Tensor],
               edge_weights: Sequence[float], position_offsets: Sequence[int],
               x: torch.Tensor, ws: torch.Tensor,
               out_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """Batched verify with a caller route (edges partitioned by position_offsets)."""
    lib = load()
    n = len(edge_experts)
    m = len(position_offsets) - 1
    ptrs = (C.c_void_p * max(n, 1))(*[e if isinstance(e, int) else _ptr(e) for e in edge_experts])
    w = (C.c_float * max(n, 1))(*[float(v) for v in edge_weights])
    offs = (C.c_int * (m + 1))(*[int(v) for v in position_offsets])
    out = torch.empty((m, g.hidden), dtype=out_dtype, device=x.device)
    base, nbytes = _ws_args(ws)
    rc = lib.k3_hip_moe_verify_device(C.byref(g), ptrs, w, offs, m, _ptr(x), _dtype_code(x),
                                      _ptr(out), _dtype_code(out), base, nbytes, stream_handle())
    check(rc, "k3_hip_moe_verify_device")
    return out


# ----------------------------------------------------------------- surface 1
def _descs(blobs: Sequence[np.ndarray | torch.Tensor | int], span: int,
           layout: int = _lib.K3_LAYOUT_RAW_V1):
    arr = (K3HipExpertDescriptorV1 * max(len(blobs), 1))()
    for i, b in enumerate(blobs):
        d = arr[i]
        d.abi_version = _lib.K3_DESCRIPTOR_ABI_V1
        d.struct_bytes = C.sizeof(K3HipExpertDescriptorV1)
        d.layout_id = layout
        d.reserved = 0
        d.blob_bytes = span
        if isinstance(b, np.ndarray):
            d.blob = b.ctypes.data
        elif isinstance(b, torch.Tensor):
            d.blob = _ptr(b)
        else:
            d.blob = int(b)
    return arr


def _layout_span(layout: int, raw_span: int) -> int:
    return _lib.K3_SCALE4_V2_EXPERT_SPAN if layout == _lib.K3_LAYOUT_SCALE4_V2 else raw_span


def moe_layer_desc(blobs: Sequence, weights: Sequence[float], x: np.ndarray,
                   layout: int = _lib.K3_LAYOUT_RAW_V1) -> np.ndarray:
    """Host-synchronous descriptor call (surface 1); x fp32 [hidden] on host;
    every blob in `layout` (raw-v1, or scale4-v2 at the K3 geometry)."""
    lib = load()
    h, i, span = C.c_int(), C.c_int(), C.c_longlong()
    lib.k3_hip_shapes(C.byref(h), C.byref(i), C.byref(span))
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(h.value, dtype=np.float32)
    w = np.ascontiguousarray(weights, dtype=np.float32)
    rc = lib.k3_hip_moe_layer_desc_v1(_descs(blobs, _layout_span(layout, span.value), layout),
                                      len(blobs), w.ctypes.data, x.ctypes.data, out.ctypes.data)
    check(rc, "k3_hip_moe_layer_desc_v1")
    return out


def moe_positions_desc(blobs: Sequence, position_offsets: Sequence[int],
                       weights: Sequence[float], x: np.ndarray,
                       layout: int = _lib.K3_LAYOUT_RAW_V1, flat: bool = False) -> np.ndarray:
    """k3_hip_moe_positions_desc_v1, or with flat=True its flat form
    k3_hip_moe_positions_flat_desc_v1 (one batched dispatch sequence; a
    K3HipError with status K3_HIP_E_CAPABILITY where the batch has none)."""
    lib = load()
    h, i, span = C.c_int(), C.c_int(), C.c_longlong()
    lib.k3_hip_shapes(C.byref(h), C.byref(i), C.byref(span))
    x = np.ascontiguousarray(x, dtype=np.float32)
    m = len(position_offsets) - 1
    out = np.empty((m, h.value), dtype=np.float32)
    w = np.ascontiguousarray(weights, dtype=np.float32)
    offs = np.ascontiguousarray(position_offsets, dtype=np.int32)
    fn = lib.k3_hip_moe_positions_flat_desc_v1 if flat else lib.k3_hip_moe_positions_desc_v1
    rc = fn(_descs(blobs, _layout_span(layout, span.value), layout), len(blobs),
            offs.ctypes.data, m, w.ctypes.data, x.ctypes.data, out.ctypes.data)
    check(rc, "k3_hip_moe_positions_flat_desc_v1" if flat else "k3_hip_moe_positions_desc_v1")
    return out


# ----------------------------------------------------------------- staging cache
class ExpertCache:
    """HBM LRU of expert spans with plan -> fetch -> resolve -> release."""

    def __init__(self, span_bytes: int, capacity: int, n_layers: int, staging_slots: int = 2,
                 device: int = 0):
        lib = load()
        self._lib = lib
        self.handle = lib.k3_hip_cache_create(device, span_bytes, capacity, n_layers,
                                              staging_slots)
        if not self.handle:
            raise K3HipError(-3, "k3_hip_cache_create")
        self.span = span_bytes

    def close(self) -> None:
        if self.handle:
            self._lib.k3_hip_cache_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def plan(self, plan_id: int, layer: int, ids: Sequence[int]) -> list[int]:
        n = len(ids)
        a = (C.c_uint16 * n)(*ids)
        miss = (C.c_uint16 * n)()
        nm = C.c_int()
        check(self._lib.k3_hip_cache_plan(self.handle, plan_id, layer, a, n, miss, C.byref(nm)),
              "k3_hip_cache_plan")
        return [miss[i] for i in range(nm.value)]

    def fetch(self, plan_id: int, sources: Sequence[int]) -> None:
        n = len(sources)
        a = (C.c_void_p * max(n, 1))(*sources)
        check(self._lib.k3_hip_cache_fetch(self.handle, plan_id, a, n), "k3_hip_cache_fetch")

    def resolve(self, plan_id: int, ids: Sequence[int], stream: int | None = None) -> list[int]:
        n = len(ids)
        a = (C.c_uint16 * n)(*ids)
        out = (C.c_void_p * n)()
        check(self._lib.k3_hip_cache_resolve(self.handle, plan_id, a, n, out,
                                             stream if stream is not None else stream_handle()),
              "k3_hip_cache_resolve")
        return [int(out[i]) for i in range(n)]

    def ready_subset(self, plan_id: int, ids: Sequence[int],
                     stream: int | None = None) -> list[int | None]:
        n = len(ids)
        a = (C.c_uint16 * n)(*ids)
        out = (C.c_void_p * n)()
        rc = self._lib.k3_hip_cache_ready_subset_v2(self.handle, plan_id, a, n, out,
                                                 stream if stream is not None else stream_handle())
        if rc < 0:
            raise K3HipError(rc, "k3_hip_cache_ready_subset_v2")
        return [int(out[i]) if out[i] else None for i in range(n)]

    def configure(self, automatic: bool, capacity: int = 0,
                  reserve_kind: int = _lib.K3_CACHE_RESERVE_AUTO, reserve_value: int = 0) -> None:
        """CudaMoeExpertCache::configure (provider_cuda_moe.h:97-98); before the first plan."""
        p = _lib.K3HipCachePolicyV1(1, C.sizeof(_lib.K3HipCachePolicyV1), int(automatic),
                                    reserve_kind, capacity, reserve_value)
        check(self._lib.k3_hip_cache_configure(self.handle, C.byref(p)), "k3_hip_cache_configure")

    def budget(self) -> dict[str, int]:
        """The budget (measured: False before the first plan and after a
        recovery, until the next plan measures it again)."""
        s = (C.c_longlong * 5)()
        rc = self._lib.k3_hip_cache_budget(self.handle, s)
        if rc < 0:
            raise K3HipError(rc, "k3_hip_cache_budget")
        return dict(zip(["capacity", "allocated_slots", "free_bytes", "reserve_bytes",
                         "rebuilds_left"], list(s)), measured=rc == 1)

    def materialize_plan(self, plan_id: int, max_hits: int) -> dict[int, np.ndarray]:
        """Host copies of the plan's pinned hits (materialize_plan_for_cpu,
        provider_cuda_moe.cpp:1170-1196): {expert id: span bytes}."""
        ids = (C.c_uint16 * max(max_hits, 1))()
        host = np.empty(max(max_hits, 1) * self.span, dtype=np.uint8)
        n = C.c_int()
        check(self._lib.k3_hip_cache_materialize_plan(self.handle, plan_id, ids, max_hits,
                                                      host.ctypes.data, host.nbytes, C.byref(n)),
              "k3_hip_cache_materialize_plan")
        return {int(ids[i]): host[i * self.span:(i + 1) * self.span] for i in range(n.value)}

    def fail_allocations(self, count: int) -> None:
        """Test hook: the next `count` device allocations report out-of-memory."""
        check(self._lib.k3_hip_cache_fail_allocations(self.handle, count),
              "k3_hip_cache_fail_allocations")

    def state(self) -> tuple[int, str]:
        buf = C.create_string_buffer(512)
        rc = self._lib.k3_hip_cache_state(self.handle, buf, 512)
        return rc, buf.value.decode(errors="replace")

    def release(self, plan_id: int) -> None:
        self._lib.k3_hip_cache_release(self.handle, plan_id)

    def stats(self) -> dict[str, int]:
        s = (C.c_longlong * 6)()
        self._lib.k3_hip_cache_stats(self.handle, s)
        return dict(zip(["hits", "misses", "evictions", "resident", "capacity", "bytes_uploaded"],
                        list(s)))

    def read_back(self, layer: int, expert: int) -> np.ndarray:
        out = np.empty(self.span, dtype=np.uint8)
        check(self._lib.k3_hip_cache_read_back(self.handle, layer, expert, out.ctypes.data,
                                               self.span), "k3_hip_cache_read_back")
        return out


# ----------------------------------------------------------------- synthetic inputs
def synth_bank(g: K3HipGeometryV1, bank: torch.Tensor, stride: int, n_experts: int,
               first_expert: int, seed: int, scale_lo: int = 119, scale_hi: int = 127) -> None:
    check(load().k3_hip_synth_bank(C.byref(g), _ptr(bank), stride, n_experts, first_expert, seed,
                                   scale_lo, scale_hi, stream_handle()), "k3_hip_synth_bank")


def synth_normal(n: int, dtype: torch.dtype, seed: int, stream_id: int,
                 device: str | torch.device = "cuda") -> torch.Tensor:
    out = torch.empty(n, dtype=dtype, device=device)
    check(load().k3_hip_synth_normal(_ptr(out), _dtype_code(out), n, seed, stream_id,
                                     stream_handle()), "k3_hip_synth_normal")
    return out
