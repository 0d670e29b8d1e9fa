"""The .ansc v4 unit records without a GPU: the Python restatement of the
format (tests/ckpt_format.py) against the oracle's streams, and the reader's
host-side checks on files assembled from the layout — a corrupt record or
size is CKR_E_CORRUPT before anything is uploaded.

Layout (include/checkers_amd.h, ckr_ckpt_write): header {magic, 4, rank, n,
u64 unit_bytes, u64 records offset}, 576-byte index entries (name, dtype, raw,
owns, original bytes, elements, data offset, data size, anchor, n_units,
records offset, records size), stored bytes, unit records; tables in
tables/rank_<r>_tables.dict (v1, 2308-byte entries).  Without a GPU, a file
that passes validation fails later at the first device allocation
(CKR_E_HIP), which is how the valid cases show they got past the checks.
"""
import os
import struct

import numpy as np
import pytest

import checkers_amd as ck
import oracle as oc
from tests import ckpt_format as cf
from tests import datagen as dg

UNIT = 256
L_ = 1 << 23


@pytest.mark.parametrize("tag,unit", [(dg.F32, 4096), (dg.BF16, 65536), (dg.I8, 4096), (dg.BF16, 1024)])
def test_unit_records_round_trip_the_oracle_streams(tag, unit):
    n = 40_001
    arr = {dg.F32: dg.normal_f32(n, 1e-3, 1), dg.BF16: dg.normal_bf16(n, 0.02, 2),
           dg.I8: np.random.default_rng(3).integers(-20, 20, n).astype(np.int8)}[tag]
    raw = np.ascontiguousarray(arr).view(np.uint8).reshape(-1)
    ref = oc.compress_tensor(raw, n, tag, unit)
    es, spe = oc.ES[tag], oc.SPE[tag]
    norm0 = int(ref["table"]["norm_freq"][0])
    rec, stored = cf.pack_tensor(ref["headers"], ref["unit_offsets"], ref["data"].tobytes(), raw.size, unit, es,
                                 spe, norm0)
    nu = oc.num_units(raw.size, unit)
    kinds = []
    p = 0
    for _ in range(nu):   # walk the records: every unit of this data is packed
        kinds.append(rec[p])
        p += 1 if rec[p] == 1 else 2049 if rec[p] == 2 else 0
        if kinds[-1] == 0:
            G = es - spe
            w = sum(rec[p + 5 + 5 * g] for g in range(G))
            p += 1 + 5 * G + (31 * (256 // es) * G + (256 // es) * w + 7) // 8
    assert p == len(rec) and set(kinds) == {0}
    if spe:   # the zero-plane lanes' bytes are not stored (4 symbols a lane emit none)
        assert len(stored) < ref["data"].size or unit < 4096
    else:
        assert len(stored) == ref["data"].size
    hdr, uoff, data = cf.expand_tensor(rec, stored, raw.size, unit, es, spe, norm0)
    assert np.array_equal(hdr.view(np.uint8), ref["headers"].view(np.uint8))
    assert np.array_equal(uoff, ref["unit_offsets"]) and data == ref["data"].tobytes()


def test_records_of_64k_units_are_small():
    # 64 KiB units of cfg3-like data: about 570 record bytes per unit, against
    # 4104 bytes of lane headers and offsets
    for tag, arr in ((dg.F32, dg.exp_avg_sq(1 << 18, 4)), (dg.BF16, dg.normal_bf16(1 << 19, 0.02, 5))):
        raw = np.ascontiguousarray(arr).view(np.uint8).reshape(-1)
        ref = oc.compress_tensor(raw, arr.size, tag, 65536, n_threads=4)
        rec, _ = cf.pack_tensor(ref["headers"], ref["unit_offsets"], ref["data"].tobytes(), raw.size, 65536,
                                oc.ES[tag], oc.SPE[tag], int(ref["table"]["norm_freq"][0]))
        assert len(rec) / oc.num_units(raw.size, 65536) < 620


def test_zero_lane_matches_an_all_zero_unit():
    # an all-zero I8 unit: every lane holds zeros, so every header is zero_lane's
    data = np.zeros(3000, np.uint8)
    table, _ = oc.normalize_histogram(np.bincount(np.r_[data, np.arange(256, dtype=np.uint8)], minlength=256), True)
    d, hdr, off = oc.encode(data, table, 0)
    norm0 = int(table["norm_freq"][0])
    for lane in range(256):
        K = (3000 - lane + 255) // 256
        st, zb = cf.zero_lane(norm0, K)
        assert (int(hdr[lane]["final_state"]), int(hdr[lane]["byte_count"])) == (st, len(zb))
        b0 = int(hdr[lane]["buf_offset"])
        assert d[b0: b0 + len(zb)].tobytes() == zb


# ---- reader checks on hand-built files

def _write(d, records, stored, n_elems=512, dtype=ck.I8, n_units=None, meta_size=None):
    os.makedirs(os.path.join(d, "tables"), exist_ok=True)
    nu = n_units if n_units is not None else (n_elems * ck.element_size(dtype) + UNIT - 1) // UNIT
    name = b"t0"
    entry = name.ljust(256, b"\0")
    entry += struct.pack("<BBB5x", dtype, 0, 1)
    entry += struct.pack("<QQQQ", n_elems * ck.element_size(dtype), n_elems, 0, len(stored))
    entry += b"".ljust(256, b"\0")
    entry += struct.pack("<QQQ", nu, 0, len(records) if meta_size is None else meta_size)
    assert len(entry) == 576
    data_base = 32 + 576
    with open(os.path.join(d, "rank_0_states.ansc"), "wb") as f:
        f.write(struct.pack("<IIIIQQ", 0x414E5343, 4, 0, 1, UNIT, data_base + len(stored)) + entry + bytes(stored)
                + bytes(records))
    norm = np.full(256, 16, np.uint32)
    cum = np.concatenate([[0], np.cumsum(norm)]).astype(np.uint32)
    with open(os.path.join(d, "tables", "rank_0_tables.dict"), "wb") as f:
        f.write(struct.pack("<IIII", 0x44494354, 1, 0, 1) + name.ljust(256, b"\0") + norm.tobytes() + cum.tobytes())


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


def _packed_unit(counts, states=None):
    """A kind-0 record for an I8 unit (one live plane, 256 live lanes)."""
    h = np.zeros(256, cf.HEADER)
    h["byte_count"] = counts
    h["final_state"] = L_ if states is None else states
    h["buf_offset"] = np.concatenate([[0], np.cumsum(counts)[:-1]])
    body = bytes(int(sum(counts)))
    return cf.pack_unit(h, body, UNIT, 1, 0, 16)


def _valid():
    r0, s0 = b"\x01", bytes(range(256))                 # a raw unit
    r1, s1 = _packed_unit(np.full(256, 1, np.int64) - (np.arange(256) % 2))   # 128 one-byte lanes
    return r0 + r1, s0 + s1


def test_valid_v4_records_pass_the_checks(tmp_path):
    rec, stored = _valid()
    assert rec[1] == 0
    _write(tmp_path, rec, stored)
    with pytest.raises(ck.CkrError) as e:
        _restore(str(tmp_path))
    assert e.value.code != ck.CKR_E_CORRUPT, str(e.value)


@pytest.mark.parametrize("case", ["unknown_kind", "records_short", "records_left_over", "stored_short",
                                  "stored_left_over", "width_above_32", "full_unit_past_length",
                                  "unit_count", "records_size_past_file"])
def test_corrupt_v4_records_are_rejected_on_the_host(tmp_path, case):
    rec, stored = _valid()
    kw = {}
    if case == "unknown_kind":
        rec = b"\x07" + rec[1:]
    elif case == "records_short":
        rec = rec[:-3]
    elif case == "records_left_over":
        rec = rec + b"\x01"
    elif case == "stored_short":
        stored = stored[:-1]
    elif case == "stored_left_over":
        stored = stored + b"\x00"
    elif case == "width_above_32":
        rec = rec[:1] + rec[1:6] + bytes([40]) + rec[7:]
    elif case == "full_unit_past_length":
        full = b"\x02" + b"".join(struct.pack("<II", L_, 2) for _ in range(256))   # 512 bytes in a 256-byte unit
        rec, stored = b"\x01" + full, bytes(256) + bytes(512)
    elif case == "unit_count":
        kw = dict(n_units=1 << 40)
    elif case == "records_size_past_file":
        kw = dict(meta_size=1 << 40)
    _write(tmp_path, rec, stored, **kw)
    with pytest.raises(ck.CkrError) as e:
        _restore(str(tmp_path))
    assert e.value.code == ck.CKR_E_CORRUPT, str(e.value)
