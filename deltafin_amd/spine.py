"""Host interface of the spine projections on torch device tensors.

Mirrors the reference's RAW_BF16 projection entry (k3_cuda_spine_bf16_launch_v1,
native/provider_gate/provider_spine_bf16_cuda.cu:253-278, as its projector
calls it) and the ATen steps either side of the routed experts
(provider_moe.cpp:1673-1688 and :1997-2014): every call enqueues gfx950 work on
the current torch stream through include/k3_hip_spine_abi.h and raises
K3SpineError with the library's reason on a non-zero status.  There is no CPU
path.
"""
from __future__ import annotations

import ctypes as C

import torch

from . import _lib


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _dense(t: torch.Tensor, dtype: torch.dtype, what: str) -> None:
    if t.device.type != "cuda" or t.dtype != dtype or not t.is_contiguous():
        raise ValueError(f"{what} must be a contiguous {dtype} device tensor")


def bf16_gemv(weights: torch.Tensor, x: torch.Tensor, out: torch.Tensor | None = None
              ) -> torch.Tensor:
    """out[p, r] = sum_c bf16(weights[r, c]) * x[p, c] in fp32.  weights: BF16
    bits as int16/uint16/bfloat16 [rows, cols]; x: fp32 [positions, cols]."""
    if weights.dtype not in (torch.int16, torch.uint16, torch.bfloat16):
        raise ValueError("weights must hold BF16 bits (int16, uint16 or bfloat16)")
    if weights.device.type != "cuda" or not weights.is_contiguous() or weights.dim() != 2:
        raise ValueError("weights must be a contiguous 2-D device tensor")
    x2 = x if x.dim() == 2 else x.view(1, -1)
    _dense(x2, torch.float32, "x")
    rows, cols = weights.shape
    if x2.shape[1] != cols:
        raise ValueError(f"x has {x2.shape[1]} columns, weights {cols}")
    if out is None:
        out = torch.empty(x2.shape[0], rows, dtype=torch.float32, device=x.device)
    _dense(out, torch.float32, "out")
    lib = _lib.load()
    _lib.check_spine(lib.k3_hip_spine_bf16_launch_v1(
        weights.data_ptr(), x2.data_ptr(), out.data_ptr(), rows, cols, x2.shape[0], _stream()),
        "k3_hip_spine_bf16_launch_v1")
    return out


def int8_gemv(quantized: torch.Tensor, row_scales: torch.Tensor, x: torch.Tensor,
              out: torch.Tensor | None = None) -> torch.Tensor:
    """out[p, r] = row_scales[r] * sum_c quantized[r, c] * x[p, c] in fp32."""
    _dense(quantized, torch.int8, "quantized")
    _dense(row_scales, torch.float32, "row_scales")
    x2 = x if x.dim() == 2 else x.view(1, -1)
    _dense(x2, torch.float32, "x")
    rows, cols = quantized.shape
    if x2.shape[1] != cols or row_scales.numel() != rows:
        raise ValueError("x / row_scales do not match the matrix")
    if out is None:
        out = torch.empty(x2.shape[0], rows, dtype=torch.float32, device=x.device)
    _dense(out, torch.float32, "out")
    lib = _lib.load()
    _lib.check_spine(lib.k3_hip_spine_int8_launch_v1(
        quantized.data_ptr(), row_scales.data_ptr(), x2.data_ptr(), out.data_ptr(), rows, cols,
        x2.shape[0], _stream()), "k3_hip_spine_int8_launch_v1")
    return out


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float = _lib.K3_RMS_EPS,
             out: torch.Tensor | None = None) -> torch.Tensor:
    """weight * (x * rsqrt(mean(x^2, -1) + eps)) over the last dimension, fp32."""
    x2 = x if x.dim() == 2 else x.view(1, -1)
    _dense(x2, torch.float32, "x")
    _dense(weight, torch.float32, "weight")
    if weight.numel() != x2.shape[1]:
        raise ValueError("weight length differs from the row length")
    if out is None:
        out = torch.empty_like(x2)
    _dense(out, torch.float32, "out")
    lib = _lib.load()
    _lib.check_spine(lib.k3_hip_rms_norm(x2.data_ptr(), weight.data_ptr(), out.data_ptr(),
                                         x2.shape[0], x2.shape[1], float(eps), _stream()),
                     "k3_hip_rms_norm")
    return out


def decode_bits(bits: torch.Tensor) -> torch.Tensor:
    """fp32 bit patterns (int32) of BF16 bits (bits << 16)."""
    if bits.dtype not in (torch.int16, torch.uint16) or bits.device.type != "cuda":
        raise ValueError("bits must be an int16/uint16 device tensor")
    bits = bits.contiguous()
    out = torch.empty(bits.numel(), dtype=torch.int32, device=bits.device)
    lib = _lib.load()
    _lib.check_spine(lib.k3_hip_spine_bf16_decode_bits(bits.data_ptr(), out.data_ptr(),
                                                       bits.numel(), _stream()),
                     "k3_hip_spine_bf16_decode_bits")
    return out


class MoeSpine:
    """The eight resident spine slots of one MoE layer on the device
    (MoeSpineT1, native/provider_gate/provider_moe.h:66-100), as the
    K3HipMoeSpineV1 descriptor of k3_hip_moe_block_device.

    Matrices are row-major device tensors: BF16 bits (int16 / uint16 /
    bfloat16) for kind "bf16", int8 with fp32 row scales for kind "int8"."""

    MATRICES = ("router", "routed_down", "routed_up", "shared_gate", "shared_up", "shared_down")

    def __init__(self, kind: str, router, router_bias, routed_down, routed_norm, routed_up,
                 shared_gate, shared_up, shared_down, scales: dict | None = None,
                 top_k: int = 16):
        if kind not in ("bf16", "int8"):
            raise ValueError("kind must be 'bf16' or 'int8'")
        self.kind = kind
        self.router, self.router_bias = router, router_bias
        self.routed_down, self.routed_norm, self.routed_up = routed_down, routed_norm, routed_up
        self.shared_gate, self.shared_up, self.shared_down = shared_gate, shared_up, shared_down
        self.scales = dict(scales or {})
        self.top_k = top_k
        if router.dim() != 2 or routed_down.dim() != 2 or shared_gate.dim() != 2:
            raise ValueError("router, routed_down and shared_gate must be 2-D [rows, columns]")
        self.hidden = router.shape[1]
        self.routed_hidden = routed_down.shape[0]
        self.shared_intermediate = shared_gate.shape[0]
        self.experts = router.shape[0]
        if kind == "int8" and set(self.scales) != set(self.MATRICES):
            raise ValueError("row-int8 spines need a scale vector for every matrix")
        # Every shape, element type and layout is checked here, before a
        # pointer reaches the library (a wrong one would be an out-of-bounds
        # device read).
        H, R, S, E = self.hidden, self.routed_hidden, self.shared_intermediate, self.experts
        want = {"router": (E, H), "routed_down": (R, H), "routed_up": (H, R),
                "shared_gate": (S, H), "shared_up": (S, H), "shared_down": (H, S)}
        mdt = (torch.int16, torch.uint16, torch.bfloat16) if kind == "bf16" else (torch.int8,)
        for name, shape in want.items():
            t = getattr(self, name)
            if tuple(t.shape) != shape:
                raise ValueError(f"{name} must be {list(shape)}, got {list(t.shape)}")
        if tuple(router_bias.shape) != (E,):
            raise ValueError(f"router_bias must hold {E} values")
        if tuple(routed_norm.shape) != (R,):
            raise ValueError(f"routed_norm must hold {R} values")
        for name, shape in want.items():
            t = getattr(self, name)
            if t.dtype not in mdt or t.device.type != "cuda" or not t.is_contiguous():
                raise ValueError(f"{name} must be a contiguous device tensor of "
                                 f"{'BF16 bits' if kind == 'bf16' else 'int8'}")
            if kind == "int8":
                sc = self.scales[name]
                if tuple(sc.shape) != (shape[0],):
                    raise ValueError(f"{name} scales must hold {shape[0]} values")
                _dense(sc, torch.float32, f"{name} scales")
        _dense(router_bias, torch.float32, "router_bias")
        _dense(routed_norm, torch.float32, "routed_norm")
        if not 1 <= top_k <= min(E, 32):
            raise ValueError(f"top_k must be in [1, min(experts, 32)], got {top_k}")

    def descriptor(self) -> _lib.K3HipMoeSpineV1:
        d = _lib.K3HipMoeSpineV1()
        d.abi_version = _lib.K3_MOE_SPINE_ABI_V1
        d.struct_bytes = C.sizeof(_lib.K3HipMoeSpineV1)
        d.matrix_kind = _lib.K3_SPINE_MATRIX_BF16 if self.kind == "bf16" else _lib.K3_SPINE_MATRIX_INT8
        d.hidden, d.routed_hidden = self.hidden, self.routed_hidden
        d.shared_intermediate, d.experts, d.top_k = self.shared_intermediate, self.experts, self.top_k
        d.router_bias = self.router_bias.data_ptr()
        d.routed_norm = self.routed_norm.data_ptr()
        for name in self.MATRICES:
            setattr(d, name, getattr(self, name).data_ptr())
            if self.kind == "int8":
                setattr(d, name + "_scales", self.scales[name].data_ptr())
        return d


def moe_block_workspace(spine: MoeSpine, g, max_positions: int) -> torch.Tensor:
    lib = _lib.load()
    d = spine.descriptor()
    n = lib.k3_hip_moe_block_workspace_bytes(C.byref(d), C.byref(g), max_positions)
    if n == 0:
        raise ValueError(f"invalid spine / geometry / positions: {_lib.last_error()}")
    return torch.empty(n, dtype=torch.uint8, device="cuda")


def moe_block(spine: MoeSpine, g, bank: torch.Tensor, stride: int, hidden: torch.Tensor,
              workspace: torch.Tensor | None = None, out: torch.Tensor | None = None):
    """The K3 MoE block on the device for hidden [P, H] fp32; returns (out,
    route_ids [P, top_k], route_weights [P, top_k])."""
    h2 = hidden if hidden.dim() == 2 else hidden.view(1, -1)
    _dense(h2, torch.float32, "hidden")
    P = h2.shape[0]
    if h2.shape[1] != spine.hidden:
        raise ValueError(f"hidden rows must hold {spine.hidden} values, got {h2.shape[1]}")
    if g.hidden != spine.routed_hidden:
        raise ValueError(f"the expert geometry's hidden ({g.hidden}) must equal the spine's "
                         f"routed width ({spine.routed_hidden})")
    if bank.dtype != torch.uint8 or bank.device.type != "cuda" or not bank.is_contiguous():
        raise ValueError("bank must be a contiguous uint8 device tensor")
    if stride < g.expert_span or bank.numel() < (spine.experts - 1) * stride + g.expert_span:
        raise ValueError(f"bank holds {bank.numel()} bytes; {spine.experts} experts at stride "
                         f"{stride} need {(spine.experts - 1) * stride + g.expert_span}")
    if workspace is None:
        workspace = moe_block_workspace(spine, g, P)
    if out is None:
        out = torch.empty(P, spine.hidden, dtype=torch.float32, device=hidden.device)
    ids = torch.empty(P, spine.top_k, dtype=torch.int32, device=hidden.device)
    wts = torch.empty(P, spine.top_k, dtype=torch.float32, device=hidden.device)
    lib = _lib.load()
    d = spine.descriptor()
    _lib.check(lib.k3_hip_moe_block_device(
        C.byref(d), C.byref(g), bank.data_ptr(), stride, h2.data_ptr(), P, out.data_ptr(),
        ids.data_ptr(), wts.data_ptr(), workspace.data_ptr(), workspace.numel(), _stream()),
        "k3_hip_moe_block_device")
    return out, ids, wts
