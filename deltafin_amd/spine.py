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
