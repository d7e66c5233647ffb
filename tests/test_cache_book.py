"""CPU test of the expert cache's host bookkeeping (deltafin_amd/csrc/k3_cache_book.h,
the same header the library compiles): policy bounds (validate_cache_policy,
provider_cuda_moe.cpp:60-74), the budget arithmetic and the reference's own
clamp_cache_capacity checks (:76-97), global LRU over layer strata with plan
pinning (:707-747, :963-1008), and the bounded recovery from a forced
allocation failure: undo the fetch, drop unpinned entries, give back segments,
keep the plan's hits for materialization, two rebuilds, then disable
(:545-567, :630-653).  Compiled with g++ and run; no GPU.
"""
import subprocess
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def test_cache_book(tmp_path):
    exe = tmp_path / "cache_book_test"
    subprocess.run(["g++", "-std=c++17", "-O1", "-Wall", "-Wextra", "-Werror",
                    "-fsanitize=address,undefined", "-o", str(exe),
                    str(ROOT / "tests" / "c" / "cache_book_test.cpp")], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.strip() == "ok"
