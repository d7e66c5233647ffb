"""ctypes binding of libk3hipmoe.so (the C ABI in include/k3_hip_moe_abi.h and
include/k3_hip_spine_abi.h).

The library is loaded after torch so that it binds to the HIP runtime torch
already mapped (both carry the SONAME libamdhip64.so.7); loading fails loudly if
the library is missing or two HIP runtimes end up in the process.  There is no
CPU fallback: every entry point runs the gfx950 code or returns an error.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "lib" / "libk3hipmoe.so"

K3_HIP_OK = 0
K3_HIP_E_INIT = -1
K3_HIP_E_INVALID = -2
K3_HIP_E_ALLOC = -3
K3_HIP_E_COPY = -4
K3_HIP_E_EXEC = -5
K3_HIP_E_CAPABILITY = -6
K3_HIP_E_DESCRIPTOR = -7

K3_LAYOUT_RAW_V1 = 1
K3_LAYOUT_SCALE4_V2 = 2
K3_DESCRIPTOR_ABI_V1 = 1
K3_RAW_V1_EXPERT_SPAN = 17547264
K3_SCALE4_V2_EXPERT_SPAN = 17039360
K3_CAP_RAW_V1 = 1 << K3_LAYOUT_RAW_V1
K3_CAP_SCALE4_V2 = 1 << K3_LAYOUT_SCALE4_V2

K3_ACT_SITU = 0
K3_ACT_SILU = 1
K3_DTYPE_F32 = 0
K3_DTYPE_BF16 = 1
K3_HIP_MAX_TOKEN_EXPERTS = 32
K3_HIP_MAX_POSITIONS = 16
K3_HIP_MAX_EDGES = 256
K3_HIP_NOALLOC_SCRATCH_BYTES = 1 << 20


class K3HipExpertDescriptorV1(C.Structure):
    _fields_ = [
        ("abi_version", C.c_uint32),
        ("struct_bytes", C.c_uint32),
        ("layout_id", C.c_uint32),
        ("reserved", C.c_uint32),
        ("blob_bytes", C.c_uint64),
        ("blob", C.c_void_p),
    ]


class K3HipGeometryV1(C.Structure):
    _fields_ = [
        ("abi_version", C.c_uint32),
        ("struct_bytes", C.c_uint32),
        ("hidden", C.c_uint32),
        ("intermediate", C.c_uint32),
        ("activation", C.c_uint32),
        ("reserved", C.c_uint32),
        ("expert_span", C.c_uint64),
    ]


class K3HipKernelTimingV1(C.Structure):
    _fields_ = [
        ("kernel", C.c_char * 32),
        ("launches", C.c_int64),
        ("total_ms", C.c_double),
        ("min_ms", C.c_double),
        ("max_ms", C.c_double),
    ]


class K3HipMoeSpineV1(C.Structure):
    _fields_ = [
        ("abi_version", C.c_uint32),
        ("struct_bytes", C.c_uint32),
        ("matrix_kind", C.c_uint32),
        ("hidden", C.c_uint32),
        ("routed_hidden", C.c_uint32),
        ("shared_intermediate", C.c_uint32),
        ("experts", C.c_uint32),
        ("top_k", C.c_uint32),
        ("router", C.c_void_p),
        ("router_scales", C.c_void_p),
        ("router_bias", C.c_void_p),
        ("routed_down", C.c_void_p),
        ("routed_down_scales", C.c_void_p),
        ("routed_norm", C.c_void_p),
        ("routed_up", C.c_void_p),
        ("routed_up_scales", C.c_void_p),
        ("shared_gate", C.c_void_p),
        ("shared_gate_scales", C.c_void_p),
        ("shared_up", C.c_void_p),
        ("shared_up_scales", C.c_void_p),
        ("shared_down", C.c_void_p),
        ("shared_down_scales", C.c_void_p),
    ]


K3_SPINE_MATRIX_BF16 = 0
K3_SPINE_MATRIX_INT8 = 1
K3_MOE_SPINE_ABI_V1 = 1


class K3HipCachePolicyV1(C.Structure):
    _fields_ = [
        ("abi_version", C.c_uint32),
        ("struct_bytes", C.c_uint32),
        ("automatic_capacity", C.c_uint32),
        ("reserve_kind", C.c_uint32),
        ("capacity_experts", C.c_uint64),
        ("reserve_value", C.c_uint64),
    ]


K3_CACHE_RESERVE_AUTO, K3_CACHE_RESERVE_BYTES, K3_CACHE_RESERVE_RATIO_PPM = 0, 1, 2
K3_HIP_CACHE_MAX_EXPERTS = 1472  # 92 strata x 16 (provider_cuda_moe.cpp:55-57)
assert C.sizeof(K3HipCachePolicyV1) == 32

assert C.sizeof(K3HipMoeSpineV1) == 144
assert C.sizeof(K3HipKernelTimingV1) == 64
assert C.sizeof(K3HipExpertDescriptorV1) == 32
assert C.sizeof(K3HipGeometryV1) == 32

_vp = C.c_void_p
_i32 = C.c_int
_u32 = C.c_uint32
_u64 = C.c_uint64
_i64 = C.c_int64
_GP = C.POINTER(K3HipGeometryV1)
_DP = C.POINTER(K3HipExpertDescriptorV1)

# name -> (restype, argtypes); every symbol declared in include/*.h
SIGNATURES = {
    "k3_hip_geometry_span": (_u64, [_u32, _u32]),
    "k3_hip_geometry_preset": (_i32, [_i32, _GP]),
    "k3_hip_last_error": (C.c_char_p, []),
    "k3_hip_init": (_i32, [C.c_char_p]),
    "k3_hip_available": (_i32, []),
    "k3_hip_descriptor_abi_version": (_u32, []),
    "k3_hip_layout_capabilities": (_u64, []),
    "k3_hip_configure_v1": (_i32, [_GP]),
    "k3_hip_shapes": (None, [C.POINTER(_i32), C.POINTER(_i32), C.POINTER(C.c_longlong)]),
    "k3_hip_stats": (None, [C.POINTER(C.c_longlong)]),
    "k3_hip_mode": (_i32, []),
    "k3_hip_set_mode": (_i32, [_i32]),
    "k3_hip_drop": (None, [_vp]),
    "k3_hip_flush": (None, []),
    "k3_hip_moe_layer_desc_v1": (_i32, [_DP, _i32, _vp, _vp, _vp]),
    "k3_hip_moe_positions_desc_v1": (_i32, [_DP, _i32, _vp, _i32, _vp, _vp, _vp]),
    "k3_hip_moe_layer": (_i32, [_vp, _i32, _vp, _vp, _vp]),
    "k3_hip_moe_positions": (_i32, [_vp, _i32, _vp, _i32, _vp, _vp, _vp]),
    "k3_hip_moe_positions_flat": (_i32, [_vp, _i32, _vp, _i32, _vp, _vp, _vp]),
    "k3_hip_moe_positions_flat_desc_v1": (_i32, [_DP, _i32, _vp, _i32, _vp, _vp, _vp]),
    "k3_hip_moe_abi_version": (_u32, []),
    "k3_hip_moe_shapes": (None, [C.POINTER(_i32), C.POINTER(_i32), C.POINTER(_i64), C.POINTER(_u32)]),
    "k3_hip_moe_available": (_i32, [_i32]),
    "k3_hip_mxfp4_gemv": (_i32, [_vp, _vp, _vp, _vp, _i32, _i32, _i32, _vp]),
    "k3_hip_mxfp4_gemv_ex": (_i32, [_vp, _vp, _vp, _i32, _vp, _i32, _i32, _i32, _i32, _vp]),
    "k3_hip_moe_launch": (_i32, [_GP, _vp, _vp, _i32, _vp, _vp, _vp, _vp]),
    "k3_hip_moe_workspace_bytes": (_u64, [_GP, _i32, _i32]),
    "k3_hip_moe_layer_device": (_i32, [_GP, _vp, _vp, _i32, _vp, _i32, _vp, _i32, _vp, _u64, _vp]),
    "k3_hip_moe_route_layer_device": (
        _i32, [_GP, _vp, _u64, _i32, _vp, _i32, _vp, _i32, _vp, _i32, _vp, _vp, _vp, _u64, _vp]),
    "k3_hip_moe_route_layer_device_noalloc": (
        _i32, [_GP, _vp, _u64, _i32, _vp, _i32, _vp, _i32, _vp, _i32, _vp, _vp, _vp]),
    "k3_hip_moe_verify_route_device": (
        _i32, [_GP, _vp, _u64, _i32, _vp, _i32, _i32, _vp, _i32, _vp, _i32, _vp, _vp, _vp, _u64, _vp]),
    "k3_hip_moe_verify_device": (
        _i32, [_GP, _vp, _vp, _vp, _i32, _vp, _i32, _vp, _i32, _vp, _u64, _vp]),
    "k3_hip_cache_create": (_vp, [_i32, _u64, _i32, _i32, _i32]),
    "k3_hip_cache_destroy": (None, [_vp]),
    "k3_hip_cache_plan": (_i32, [_vp, _u64, _i32, _vp, _i32, _vp, C.POINTER(_i32)]),
    "k3_hip_cache_fetch": (_i32, [_vp, _u64, _vp, _i32]),
    "k3_hip_cache_resolve": (_i32, [_vp, _u64, _vp, _i32, _vp, _vp]),
    "k3_hip_cache_ready_subset": (_i32, [_vp, _u64, _vp, _i32, _vp]),
    "k3_hip_cache_ready_subset_v2": (_i32, [_vp, _u64, _vp, _i32, _vp, _vp]),
    "k3_hip_cache_release": (None, [_vp, _u64]),
    "k3_hip_cache_configure": (_i32, [_vp, C.POINTER(K3HipCachePolicyV1)]),
    "k3_hip_cache_budget": (_i32, [_vp, C.POINTER(C.c_longlong)]),
    "k3_hip_cache_materialize_plan": (_i32, [_vp, _u64, _vp, _i32, _vp, _u64, C.POINTER(_i32)]),
    "k3_hip_cache_fail_allocations": (_i32, [_vp, _i32]),
    "k3_hip_cache_stats": (None, [_vp, C.POINTER(C.c_longlong)]),
    "k3_hip_cache_read_back": (_i32, [_vp, _i32, C.c_uint16, _vp, _u64]),
    "k3_hip_cache_state": (_i32, [_vp, C.c_char_p, _u64]),
    "k3_hip_cache_poison": (None, [_vp, C.c_char_p]),
    "k3_hip_timing_begin": (_i32, [_i32]),
    "k3_hip_timing_end": (_i32, [C.POINTER(K3HipKernelTimingV1), _i32, C.POINTER(_i32),
                                 C.POINTER(C.c_longlong)]),
    "k3_hip_set_fused_decode": (_i32, [_i32]),
    "k3_hip_set_decode_chain": (_i32, [_i32]),
    "k3_hip_set_decode_mfma": (_i32, [_i32]),
    "k3_hip_set_verify_mode": (_i32, [_i32]),
    "k3_hip_scale4_check_header": (_i32, [_vp, _u64]),
    "k3_hip_synth_bank": (_i32, [_GP, _vp, _u64, _i32, _u64, _u64, _i32, _i32, _vp]),
    "k3_hip_synth_normal": (_i32, [_vp, _i32, _u64, _u64, _u64, _vp]),
    "k3_hip_moe_block_workspace_bytes": (_u64, [C.POINTER(K3HipMoeSpineV1), _GP, _i32]),
    "k3_hip_moe_block_device": (
        _i32, [C.POINTER(K3HipMoeSpineV1), _GP, _vp, _u64, _vp, _i32, _vp, _vp, _vp, _vp, _u64,
               _vp]),
    # include/k3_hip_spine_abi.h
    "k3_hip_spine_bf16_abi_version": (_u32, []),
    "k3_hip_spine_last_error": (C.c_char_p, []),
    "k3_hip_spine_bf16_available": (_i32, [_i32, C.POINTER(_i32), C.POINTER(_i32)]),
    "k3_hip_spine_bf16_launch_v1": (_i32, [_vp, _vp, _vp, _i32, _i32, _i32, _vp]),
    "k3_hip_spine_bf16_decode_bits": (_i32, [_vp, _vp, _i32, _vp]),
    "k3_hip_spine_int8_launch_v1": (_i32, [_vp, _vp, _vp, _vp, _i32, _i32, _i32, _vp]),
    "k3_hip_rms_norm": (_i32, [_vp, _vp, _vp, _i32, _i32, C.c_float, _vp]),
}

_LIB: C.CDLL | None = None


class K3HipError(RuntimeError):
    def __init__(self, status: int, what: str):
        super().__init__(f"{what} failed with status {status}: {last_error()}")
        self.status = status


def _hip_runtimes_mapped() -> set[str]:
    paths = set()
    try:
        with open("/proc/self/maps") as f:
            for line in f:
                if "libamdhip64.so" in line:
                    paths.add(os.path.realpath(line.split()[-1]))
    except OSError:
        pass
    return paths


def load() -> C.CDLL:
    """Load the library once; raises if it is missing (run deltafin_amd.build)."""
    global _LIB
    if _LIB is not None:
        return _LIB
    try:  # bind to torch's HIP runtime when torch is present
        import torch  # noqa: F401
    except ImportError:
        pass
    if not LIB_PATH.exists():
        raise ImportError(
            f"{LIB_PATH} is missing: build it with `python -m deltafin_amd.build` "
            "(the gfx950 library has no CPU fallback)")
    lib = C.CDLL(str(LIB_PATH))
    runtimes = _hip_runtimes_mapped()
    if len(runtimes) > 1:
        raise ImportError(f"two HIP runtimes are mapped in this process: {sorted(runtimes)}")
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _LIB = lib
    return lib


def last_error() -> str:
    lib = _LIB if _LIB is not None else load()
    msg = lib.k3_hip_last_error()
    return msg.decode(errors="replace") if msg else ""


def check(status: int, what: str) -> None:
    if status != K3_HIP_OK:
        raise K3HipError(status, what)


K3_SPINE_OK = 0
K3_SPINE_E_INVALID = -1
K3_SPINE_E_RUNTIME = -2
K3_SPINE_E_UNSUPPORTED = -3
K3_SPINE_MAX_POSITIONS = 64
K3_RMS_EPS = 1.0e-5  # the reference's kRmsEpsilon (provider_moe.cpp:87)


class K3SpineError(RuntimeError):
    def __init__(self, status: int, what: str):
        lib = _LIB if _LIB is not None else load()
        msg = lib.k3_hip_spine_last_error()
        super().__init__(f"{what} failed with status {status}: "
                         f"{msg.decode(errors='replace') if msg else ''}")
        self.status = status


def check_spine(status: int, what: str) -> None:
    if status != K3_SPINE_OK:
        raise K3SpineError(status, what)


def geometry(hidden: int, intermediate: int, activation: int) -> K3HipGeometryV1:
    g = K3HipGeometryV1()
    g.abi_version = 1
    g.struct_bytes = C.sizeof(K3HipGeometryV1)
    g.hidden = hidden
    g.intermediate = intermediate
    g.activation = activation
    g.reserved = 0
    g.expert_span = load().k3_hip_geometry_span(hidden, intermediate)
    return g


def preset(which: int) -> K3HipGeometryV1:
    g = K3HipGeometryV1()
    check(load().k3_hip_geometry_preset(which, C.byref(g)), "k3_hip_geometry_preset")
    return g


def set_fused_decode(enabled: bool) -> bool:
    """Select the fused single-launch decode path or the two-launch path (the
    default) for later layer calls; returns the previous setting."""
    return bool(load().k3_hip_set_fused_decode(1 if enabled else 0))


DECODE_CHAIN_OFF, DECODE_CHAIN_ON, DECODE_CHAIN_FALLBACK = 0, 1, 2


def set_decode_chain(mode: int) -> int:
    """Run one-expert layer calls as one launch (DECODE_CHAIN_ON, the
    default), as the two launches (DECODE_CHAIN_OFF), or as one launch whose
    workgroups compute missing gate/up shares at once (DECODE_CHAIN_FALLBACK);
    returns the previous mode."""
    prev = load().k3_hip_set_decode_chain(int(mode))
    check(min(prev, 0), "k3_hip_set_decode_chain")
    return prev


DECODE_DOTS_VALU, DECODE_DOTS_MFMA_F32, DECODE_DOTS_MFMA_ALL = 0, 1, 2


def set_decode_mfma(mode: int) -> int:
    """Select where the single-token gate/up dots run (DECODE_DOTS_*) for
    later layer calls; returns the previous setting."""
    rc = load().k3_hip_set_decode_mfma(int(mode))
    if rc < 0:
        raise K3HipError(rc, "k3_hip_set_decode_mfma")
    return rc


VERIFY_AUTO, VERIFY_POSITIONS, VERIFY_UNION_MFMA, VERIFY_UNION_VALU = 0, 1, 2, 3


def set_verify_mode(mode: int) -> int:
    """Select the verify path process-wide (K3_VERIFY_*); returns the previous mode."""
    prev = load().k3_hip_set_verify_mode(int(mode))
    check(min(prev, 0), "k3_hip_set_verify_mode")
    return prev


def timing_begin(max_launches: int) -> None:
    """Open a per-launch timing window (k3_hip_timing_begin)."""
    check(load().k3_hip_timing_begin(max_launches), "k3_hip_timing_begin")


def timing_end() -> tuple[dict[str, dict[str, float]], int]:
    """Close the window; returns ({kernel: {launches, total_ms, min_ms, max_ms, avg_ms}}, dropped)."""
    rows = (K3HipKernelTimingV1 * 32)()
    n = C.c_int()
    dropped = C.c_longlong()
    check(load().k3_hip_timing_end(rows, 32, C.byref(n), C.byref(dropped)), "k3_hip_timing_end")
    out = {}
    for r in rows[: n.value]:
        out[r.kernel.decode()] = {
            "launches": int(r.launches), "total_ms": r.total_ms, "min_ms": r.min_ms,
            "max_ms": r.max_ms, "avg_ms": r.total_ms / max(r.launches, 1)}
    return out, int(dropped.value)
