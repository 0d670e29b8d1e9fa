"""Rank checkpoint files: the writer against files assembled here, byte by
byte, from the on-disk layout (ANSCompressor.cpp:721-931) and the oracle's
compressed streams; the reader restores every tensor bit-exact."""
import os
import struct

import numpy as np
import pytest

import oracle as oc
from tests import datagen as dg

pytestmark = pytest.mark.gpu


def _ck():
    import checkers_amd as ck
    return ck


def _dev(arr, gpu):
    import torch
    b = np.ascontiguousarray(arr).view(np.uint8).reshape(-1)
    t = torch.empty(max(b.size, 16), dtype=torch.uint8, device=gpu)
    if b.size:
        t[: b.size].copy_(torch.from_numpy(b.copy()))
    return t[: b.size]


def _name(s):
    b = s.encode()[:255]
    return b + b"\0" * (256 - len(b))


def _records(seed=0):
    rng = np.random.default_rng(seed)
    bf = dg.normal_bf16(20000, 0.02, seed + 1)
    return [  # (name, raw array, dtype tag, cluster id)
        ("layers.0.w", bf, dg.BF16, 0),
        ("layers.1.w", dg.normal_bf16(15000, 0.02, seed + 2), dg.BF16, 0),
        ("master_weights::layers.0.w", (bf.astype(np.uint32) << 16).view(np.float32), dg.F32, -1),
        ("optimizer.exp_avg::layers.0.w", dg.normal_f32(30001, 1e-3, seed + 3), dg.F32, -1),
        ("empty", np.zeros(0, np.float32), dg.F32, -1),
        ("bytes", rng.integers(0, 256, 5000).astype(np.uint8).view(np.int8), dg.I8, -1),
        ("noise", rng.integers(0, 2**32, 7000, dtype=np.uint64).astype(np.uint32).view(np.float32), dg.F32, -1),
        ("layers.2.w", dg.normal_bf16(9000, 0.02, seed + 4), dg.BF16, 0),
        ("ints", rng.integers(-50, 50, 3000).astype(np.int32), dg.I32, 1),
        ("ints2", rng.integers(-50, 50, 2000).astype(np.int32), dg.I32, 1),
    ]


def _expected_files(recs, rank, repair):
    """.ansc v2, .mant, .dict bytes from the layout and the oracle's streams."""
    tables, anchors, ents = {}, {}, []
    for name, arr, tag, cid in recs:
        if cid >= 0 and cid not in anchors:
            anchors[cid] = name
    for name, arr, tag, cid in recs:
        n = arr.size
        if n == 0:
            continue
        raw = np.ascontiguousarray(arr).view(np.uint8).reshape(-1)
        masked, side = oc.extract_mantissa(raw, n, tag)
        owns = cid < 0 or cid not in tables
        if owns:
            table, tsum = oc.normalize_histogram(oc.byte_hist(masked), cid >= 0)
            if repair and tsum > 4096:
                return None
            if cid >= 0:
                tables[cid] = table
        else:
            table = tables[cid]
        data, hdr, off = oc.encode(masked, table, 0)
        ents.append(dict(name=name, tag=tag, owns=owns, anchor="" if owns else anchors[cid], n=n,
                         orig=raw.size, data=data.tobytes(), hdr=hdr.tobytes(), side=side.tobytes(),
                         spe=oc.SPE[tag], table=table,
                         raw=int(hdr[0]["byte_count"]) == raw.size and int(hdr["byte_count"][1:].sum()) == 0))
    ansc = struct.pack("<4I", 0x414E5343, 2, rank, len(ents))
    off = 0
    for e in ents:
        ansc += _name(e["name"]) + struct.pack("<3B5x4Q", e["tag"], e["raw"], e["owns"], e["orig"], e["n"], off,
                                               len(e["data"]))
        ansc += _name(e["anchor"]) + e["hdr"]
        off += len(e["data"])
    ansc += b"".join(e["data"] for e in ents)
    sides = [e for e in ents if e["spe"]]
    mant = struct.pack("<4I", 0x4D414E54, 2, rank, len(sides))
    off = 0
    for e in sides:
        mant += _name(e["name"]) + struct.pack("<2B6x3Q", e["tag"], e["spe"], e["n"], off, len(e["side"]))
        off += len(e["side"])
    mant += b"".join(e["side"] for e in sides)
    owners = [e for e in ents if e["owns"]]
    dct = struct.pack("<4I", 0x44494354, 1, rank, len(owners))
    for e in owners:
        dct += _name(e["name"]) + e["table"]["norm_freq"].astype("<u4").tobytes() + \
            e["table"]["cum_freq"].astype("<u4").tobytes()
    return ansc, mant, dct


def _write(ck, gpu, recs, tmp, rank, unit, repair=False):
    devs = [(name, _dev(arr, gpu) if arr.size else None, tag, cid) for name, arr, tag, cid in recs]
    return ck.write_checkpoint(str(tmp), rank, devs, unit_bytes=unit, repair_tables=repair)


def test_v2_files_match_layout_and_restore(gpu, tmp_path):
    ck = _ck()
    recs = _records()
    stats = _write(ck, gpu, recs, tmp_path, 3, 0)
    exp = _expected_files(recs, 3, False)
    got = [open(os.path.join(tmp_path, p), "rb").read() for p in
           ("rank_3_states.ansc", "mantissa/rank_3_mantissa.mant", "tables/rank_3_tables.dict")]
    for g, e, what in zip(got, exp, ("ansc", "mant", "dict")):
        assert g == e, what
    assert [s["record_index"] for s in stats] == [0, 1, 2, 3, 5, 6, 7, 8, 9]
    assert [s["owns_table"] for s in stats] == [1, 0, 1, 1, 1, 1, 0, 1, 0]
    # the bf16 cluster's full-alphabet table: the reference's one-pass
    # normalisation leaves it above 4096 (its H1 case), as the oracle shows
    masked, _ = oc.extract_mantissa(recs[0][1], recs[0][1].size, dg.BF16)
    assert stats[0]["table_sum"] == oc.normalize_histogram(oc.byte_hist(masked), True)[1] > 4096
    c = ck.Checkpoint(str(tmp_path), 3)
    assert len(c) == 9
    for i, (name, arr, tag, cid) in enumerate(r for r in recs if r[1].size):
        info = c.info(i)
        assert info["name"] == name and info["version"] == 2
        if stats[i]["table_sum"] != 4096:   # such streams cannot be decoded
            with pytest.raises(ck.CkrError):
                c.restore(i)
            continue
        out = c.restore(i).cpu().numpy()
        assert np.array_equal(out, np.ascontiguousarray(arr).view(np.uint8).reshape(-1)), name
    c.close()


@pytest.mark.parametrize("unit", [0, 65536, 4096])
def test_repaired_tables_restore_everything(gpu, tmp_path, unit):
    ck = _ck()
    recs = _records(5)
    stats = _write(ck, gpu, recs, tmp_path, 0, unit, repair=True)
    assert stats[0]["table_repaired"] == 1
    assert all(s["table_repaired"] == (s["owns_table"] and s["table_sum"] > 4096) for s in stats)
    c = ck.Checkpoint(str(tmp_path), 0)
    live = [r for r in recs if r[1].size]
    assert len(c) == len(live)
    for i, (name, arr, tag, cid) in enumerate(live):
        info = c.info(i)
        assert info["version"] == (4 if unit else 2) and info["num_elements"] == arr.size
        out = c.restore(i).cpu().numpy()
        assert np.array_equal(out, np.ascontiguousarray(arr).view(np.uint8).reshape(-1)), name


@pytest.mark.parametrize("unit", [65536, 4096])
def test_v4_records_and_stored_bytes_match_oracle_units(gpu, tmp_path, unit):
    """The v4 states file holds, per tensor, the unit records and stored bytes
    that the Python restatement of the format (tests/ckpt_format.py) makes of
    the oracle's chunked streams."""
    from tests import ckpt_format as cf
    ck = _ck()
    recs = [("a", dg.normal_f32(70000, 1e-3, 9), dg.F32, -1), ("b", dg.normal_bf16(50001, 0.02, 10), dg.BF16, -1),
            ("c", dg.exp_avg_sq(33333, 11), dg.F32, -1),
            ("d", np.random.default_rng(12).integers(0, 256, 360000).astype(np.uint8).view(np.int8), dg.I8, -1),
            # a cluster whose full-alphabet table sums to 4096; its member of
            # random bytes expands under that table, so its units pass through raw
            ("e", np.random.default_rng(13).integers(-100, 100, 50000).astype(np.int8), dg.I8, 0),
            ("f", np.random.default_rng(14).integers(0, 256, 100000).astype(np.uint8).view(np.int8), dg.I8, 0)]
    _write(ck, gpu, recs, tmp_path, 1, unit)
    blob = open(os.path.join(tmp_path, "rank_1_states.ansc"), "rb").read()
    magic, ver, rank, n, u, meta_base = struct.unpack_from("<4I2Q", blob, 0)
    assert (magic, ver, rank, n, u) == (0x414E5343, 4, 1, len(recs), unit)
    data_base = 32 + 576 * n
    total_stored, tables = 0, {}
    for k, (name, arr, tag, cid) in enumerate(recs):
        e = 32 + 576 * k
        doff, dsz = struct.unpack_from("<2Q", blob, e + 280)
        nu, moff, msz = struct.unpack_from("<3Q", blob, e + 552)
        raw = np.ascontiguousarray(arr).view(np.uint8).reshape(-1)
        masked, _ = oc.extract_mantissa(raw, arr.size, tag)
        if cid < 0 or cid not in tables:
            table, tsum = oc.normalize_histogram(oc.byte_hist(masked), cid >= 0)
            assert tsum == 4096
            tables.setdefault(cid, table)
        table = tables[cid] if cid >= 0 else table
        data, hdr, uoff = oc.encode(masked, table, unit)
        assert nu == oc.num_units(raw.size, unit)
        rec, stored = cf.pack_tensor(hdr, uoff, data.tobytes(), raw.size, unit, oc.ES[tag], oc.SPE[tag],
                                     int(table["norm_freq"][0]))
        assert blob[meta_base + moff: meta_base + moff + msz] == rec, name
        assert blob[data_base + doff: data_base + doff + dsz] == stored, name
        assert blob[e + 257] == (rec == b"\x01" * nu)     # raw: every unit passed through
        assert name != "f" or rec[:1] == b"\x01"      # the raw-unit path is exercised
        total_stored += dsz
    assert meta_base == data_base + total_stored
    c = ck.Checkpoint(str(tmp_path), 1)
    for i, (name, arr, tag, cid) in enumerate(recs):
        out = c.restore(i).cpu().numpy()
        assert np.array_equal(out, np.ascontiguousarray(arr).view(np.uint8).reshape(-1)), name
    c.close()
