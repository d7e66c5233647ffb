"""CPU checks of the C-ABI boundary (no GPU, no kernel launches).

* every function declared in include/*.h is exported by the built library and
  bound by deltafin_amd._lib;
* the header compiles as plain C11 and a C caller links against the library
  and gets the documented host-side answers (tests/c/abi_probe.c);
* struct layouts match the Metal descriptor ABI (tools/metal_moe_abi.h:35-50).
"""
import ctypes as C
import re
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADERS = sorted((ROOT / "include").glob("*.h"))
DECL = re.compile(r"^\s*(?:const\s+)?[A-Za-z_][\w\s\*]*?\b(k3_hip_\w+)\s*\(", re.M)


def declared() -> set[str]:
    names = set()
    for h in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names |= set(DECL.findall(text))
    return names


def test_header_declares_entry_points():
    names = declared()
    for must in ("k3_hip_moe_layer_desc_v1", "k3_hip_moe_positions_desc_v1", "k3_hip_init",
                 "k3_hip_mxfp4_gemv", "k3_hip_moe_launch", "k3_hip_moe_route_layer_device",
                 "k3_hip_moe_verify_device", "k3_hip_cache_plan", "k3_hip_timing_begin"):
        assert must in names
    assert len(names) >= 40


def test_library_exports_every_declared_symbol():
    from deltafin_amd import _lib
    lib = _lib.load()
    missing = [n for n in sorted(declared()) if not hasattr(lib, n)]
    assert not missing, f"declared but not exported: {missing}"
    nm = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)], capture_output=True,
                        text=True, check=True).stdout
    exported = {ln.split()[-1] for ln in nm.splitlines() if " T " in ln}
    assert declared() <= exported


def test_bindings_cover_every_declared_symbol():
    from deltafin_amd import _lib
    assert declared() == set(_lib.SIGNATURES)


def test_struct_layouts():
    from deltafin_amd import _lib
    D = _lib.K3HipExpertDescriptorV1
    assert C.sizeof(D) == 32 and D.blob_bytes.offset == 16 and D.blob.offset == 24
    assert C.sizeof(_lib.K3HipGeometryV1) == 32
    assert C.sizeof(_lib.K3HipKernelTimingV1) == 64


def test_c_caller_probe(tmp_path):
    from deltafin_amd import _lib
    exe = tmp_path / "abi_probe"
    subprocess.run(["gcc", "-std=c11", "-Wall", "-Wextra", "-Werror", f"-I{ROOT / 'include'}",
                    str(ROOT / "tests" / "c" / "abi_probe.c"), "-o", str(exe),
                    f"-L{_lib.LIB_PATH.parent}", "-lk3hipmoe",
                    f"-Wl,-rpath,{_lib.LIB_PATH.parent}"], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    assert r.stdout.strip() == "ok"


def test_presets_and_spans_from_python():
    from deltafin_amd import _lib
    lib = _lib.load()
    assert lib.k3_hip_geometry_span(3584, 3072) == _lib.K3_RAW_V1_EXPERT_SPAN
    g = _lib.preset(2)
    assert (g.hidden, g.intermediate, g.activation, g.expert_span) == (7168, 2048, 1, 23396352)
    with pytest.raises(_lib.K3HipError):
        _lib.preset(9)


def test_no_device_fails_loudly():
    """Without a GPU the device entry points report an error; nothing falls back
    to a CPU path."""
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    from deltafin_amd import _lib
    lib = _lib.load()
    assert lib.k3_hip_moe_available(0) < 0
    assert lib.k3_hip_available() == 0
    assert lib.k3_hip_init(None) == -1
