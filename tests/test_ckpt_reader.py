"""Reader checks that run without a GPU: unit metadata read from a .ansc v3 file
is validated on the host before anything is uploaded, so a corrupt offset or
lane header is CKR_E_CORRUPT, not a kernel reading outside its buffer.

The files are assembled here from the documented layout (include/checkers_amd.h,
ckr_ckpt_write): header {magic, 3, rank, n, u64 unit_bytes}, 568-byte index
entries, per-tensor metadata (n_units * 256 headers, then n_units + 1 u64
offsets), data; tables in tables/rank_<r>_tables.dict (v1, 2308-byte entries).
Without a GPU, a file that passes validation fails later at the first device
allocation (CKR_E_HIP), which is how the valid case shows it got past the checks.
"""
import os
import struct

import numpy as np
import pytest

import checkers_amd as ck

UNIT = 256


def _write(d, headers, offsets, data, n_elems=512, dtype=ck.I8):
    os.makedirs(os.path.join(d, "tables"), exist_ok=True)
    nu = len(offsets) - 1
    name = b"t0"
    entry = name.ljust(256, b"\0")
    entry += struct.pack("<BBB5x", dtype, 0, 1)
    entry += struct.pack("<QQQQ", n_elems * ck.element_size(dtype), n_elems, 0, len(data))
    entry += b"".ljust(256, b"\0")
    entry += struct.pack("<QQ", nu, 0)
    assert len(entry) == 568
    meta = headers.astype(ck.HEADER_DTYPE).tobytes() + np.asarray(offsets, np.uint64).tobytes()
    with open(os.path.join(d, "rank_0_states.ansc"), "wb") as f:
        f.write(struct.pack("<IIIIQ", 0x414E5343, 3, 0, 1, UNIT) + entry + meta + bytes(data))
    norm = np.full(256, 16, np.uint32)
    cum = np.concatenate([[0], np.cumsum(norm)]).astype(np.uint32)
    with open(os.path.join(d, "tables", "rank_0_tables.dict"), "wb") as f:
        f.write(struct.pack("<IIII", 0x44494354, 1, 0, 1) + name.ljust(256, b"\0") + norm.tobytes() + cum.tobytes())


def _raw_units(nu=2):
    """nu raw (passthrough) units of UNIT bytes: header 0 of each holds the length."""
    h = np.zeros(nu * 256, ck.HEADER_DTYPE)
    for u in range(nu):
        h[u * 256]["byte_count"] = UNIT
    return h, [UNIT * u for u in range(nu + 1)], bytes(range(256)) * nu


def _restore(d):
    """ckr_ckpt_restore on the C ABI (null stream, a destination that is never
    written: validation or the first allocation fails before it is used)."""
    import ctypes
    c = ck.Checkpoint(d)
    try:
        rc = ck.lib().ckr_ckpt_restore(c._h, 0, ctypes.c_void_p(0x10000), None)
        ck._check(rc)
    finally:
        c.close()


def _code(exc):
    return exc.value.code


def test_valid_v3_metadata_passes_the_checks(tmp_path):
    _write(tmp_path, *_raw_units())
    with pytest.raises(ck.CkrError) as e:
        _restore(str(tmp_path))
    assert _code(e) != ck.CKR_E_CORRUPT


@pytest.mark.parametrize("case", ["first_offset", "decreasing", "past_unit_length", "last_offset",
                                  "lane_past_unit", "raw_unit_with_lanes"])
def test_corrupt_v3_metadata_is_rejected_on_the_host(tmp_path, case):
    h, off, data = _raw_units()
    if case == "first_offset":
        off = [8, 256, 512]
    elif case == "decreasing":
        off = [0, 300, 290]
        data = data[:290]
    elif case == "past_unit_length":
        off = [0, 300, 512]
    elif case == "last_offset":
        off = [0, 256, 511]
    elif case == "lane_past_unit":
        h[0]["byte_count"] = 100  # unit 0 no longer raw: its lanes must lie inside it
        h[1]["byte_count"] = 100
        h[1]["buf_offset"] = 200
    elif case == "raw_unit_with_lanes":
        h[257]["byte_count"] = 3
    _write(tmp_path, h, off, data)
    with pytest.raises(ck.CkrError) as e:
        _restore(str(tmp_path))
    assert _code(e) == ck.CKR_E_CORRUPT, str(e.value)


def test_truncated_metadata_and_oversized_unit_count(tmp_path):
    h, off, data = _raw_units()
    _write(tmp_path, h, off, data)
    p = os.path.join(tmp_path, "rank_0_states.ansc")
    b = open(p, "rb").read()
    # n_units field of the index entry (offset 24 + 552) claims 2^40 units
    b2 = b[:24 + 552] + struct.pack("<Q", 1 << 40) + b[24 + 560:]
    open(p, "wb").write(b2)
    with pytest.raises(ck.CkrError) as e:
        _restore(str(tmp_path))
    assert _code(e) == ck.CKR_E_CORRUPT
