"""CPU checks of the scale4-v2 expert format (no GPU).

* The oracle's codec and header builder against the reference's own test
  vectors (native/deltafin/src/expert_scale4.rs:559-630): nibble order of an
  even and an odd plane, the rejected ranges and bases, the SHA-256 of the
  canonical header and of a whole sidecar record.
* The oracle's index expansion against the reference's scale4 CPU consumer
  (mxfp4_gemv_mt_scale4, tools/fused_gemv.c:416-480, compiled into
  oracle/_ref): bit-identical to the reference raw kernel on the expanded
  scales and to the oracle's lane-order restatement.
* The library's header checks (k3_hip_scale4_check_header, the checks its
  descriptor calls run, tools/metal_moe.mm:353-405): a canonical header
  passes, the source digest is free, and each corrupted field is rejected.
"""
import hashlib

import numpy as np
import pytest

import oracle

SCALE_BYTES = 344_064  # one K3 matrix's E8M0 plane (expert_scale4.rs:23)


def test_codec_reference_vectors():
    even = np.array([17, 18, 31, 17, 22, 25], np.uint8)
    base, packed = oracle.scale4_pack(even)
    assert base == 17 and packed.tolist() == [0x10, 0x0E, 0x85]
    assert oracle.scale4_unpack(packed, base, even.size).tolist() == even.tolist()
    odd = np.array([240, 255, 241], np.uint8)
    base, packed = oracle.scale4_pack(odd, 240)
    assert packed.tolist() == [0xF0, 0x01]
    assert oracle.scale4_unpack(packed, base, odd.size).tolist() == odd.tolist()


def test_codec_rejects_lossy_ranges_and_bases():
    with pytest.raises(ValueError):
        oracle.scale4_pack(np.array([1, 17], np.uint8))
    with pytest.raises(ValueError):
        oracle.scale4_pack(np.array([239, 240], np.uint8), 241)
    with pytest.raises(ValueError):
        oracle.scale4_unpack(np.array([0], np.uint8), 241, 1)
    with pytest.raises(ValueError):
        oracle.scale4_unpack(np.array([0], np.uint8), 0, 3)


def test_header_digest_matches_reference():
    header = oracle.scale4_header(bytes(range(32)), [7, 100, 240])
    assert header.size == 8192
    assert (hashlib.sha256(header.tobytes()).hexdigest()
            == "826d7d4a29872614e6298e05be15f7637db041ce762a806ec606ccf573ee3f4b")
    with pytest.raises(ValueError):
        oracle.scale4_header(bytes(32), [7, 241, 0])


def test_sidecar_record_digest_matches_reference():
    """A record is the header then the three index planes (the on-disk
    sidecar layout of expert_scale4.rs:62-63)."""
    values = np.full(SCALE_BYTES, 120, np.uint8)
    planes = [oracle.scale4_pack(values)[1] for _ in range(3)]
    header = oracle.scale4_header(bytes([9] * 32), [120, 120, 120])
    record = np.concatenate([header] + planes)
    assert record.size == 8192 + 3 * SCALE_BYTES // 2
    assert (hashlib.sha256(record.tobytes()).hexdigest()
            == "8b50b1d82b5a7a0fd22f12826ad900e7d675ae4a89ff85921499b7e780f60f9f")


def test_span_round_trip_and_offsets():
    raw = oracle.synth_expert(5, 3, 3584, 3072)
    span4 = oracle.scale4_span(raw)
    assert span4.size == oracle.SCALE4_SPAN
    # payload table of the header = the assembled offsets (tools/metal_moe.mm:133-138)
    table = span4[72:120].view(np.uint32).tolist()
    assert table[0::2] == [8192, 5513216, 5685248, 11190272, 11362304, 16867328]
    assert np.array_equal(oracle.scale4_to_raw(span4), raw)


@pytest.mark.skipif(not oracle.ref_available(), reason="reference CPU library not built")
def test_expansion_matches_reference_scale4_consumer():
    rng = np.random.default_rng(11)
    rows, cols = 48, 3584
    groups = cols // 32
    packed = rng.integers(0, 256, rows * cols // 2, dtype=np.uint8)
    idx = rng.integers(0, 16, rows * groups, dtype=np.uint8)
    base = 113
    _, s4 = oracle.scale4_pack(idx.astype(np.int32) + base, base)
    x = rng.standard_normal(cols).astype(np.float32)
    y4 = oracle.ref_gemv_scale4(packed, s4, base, x, rows, cols)
    scales = oracle.scale4_unpack(s4, base, rows * groups)
    assert np.array_equal(scales, idx + base)
    y_raw = oracle.ref_gemv(packed, scales, x, rows, cols)
    assert np.array_equal(y4.view(np.uint32), y_raw.view(np.uint32))
    y_orc = oracle.gemv_f32_lanes(packed, scales, x, rows, cols)
    assert np.array_equal(y4.view(np.uint32), y_orc.view(np.uint32))


def _check(header) -> int:
    from deltafin_amd import _lib
    h = np.ascontiguousarray(header, dtype=np.uint8)
    return _lib.load().k3_hip_scale4_check_header(h.ctypes.data, h.size)


def test_library_header_checks():
    from deltafin_amd import _lib
    good = oracle.scale4_header(bytes(range(32)), [7, 100, 240])
    assert _check(good) == 0
    assert _check(oracle.scale4_header(bytes([0xAB] * 32), [0, 0, 0])) == 0  # digest is free
    assert _check(good[:4096]) == _lib.K3_HIP_E_INVALID
    bad_at = [0, 8, 12, 16, 24, 67, 72, 100, 120, 127, 128 + 4, 192 + 9, 256 + 63, 319, 320,
              340, 344, 8191]
    for off in bad_at:
        h = good.copy()
        h[off] ^= 1
        assert _check(h) == _lib.K3_HIP_E_DESCRIPTOR, f"offset {off}"
    h = good.copy()
    h[65] = 241  # base above 240 (its table rewritten to match)
    h[192:256] = np.array([(241 + d) << 23 for d in range(16)], np.uint32).view(np.uint8)
    assert _check(h) == _lib.K3_HIP_E_DESCRIPTOR
    assert "base" in _lib.last_error()
