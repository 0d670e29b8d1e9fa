"""The C ABI library on the CPU side: it loads, exports every declared symbol,
its host code matches the oracle, and argument errors come back as status
codes with a message (no GPU call is made in these tests)."""
import ctypes
import os
import re

import numpy as np
import pytest

import checkers_amd as ck
import oracle as oc
from tests import datagen as dg

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    text = open(os.path.join(ROOT, "include", "checkers_amd.h")).read()
    return sorted(set(re.findall(r"CKR_API\s+[\w\s\*]+?\b(ckr_\w+)\s*\(", text)))


def test_every_declared_symbol_is_exported():
    lib = ck.lib()
    names = declared_symbols()
    assert len(names) >= 19
    for n in names:
        assert hasattr(lib, n), n
    assert sorted(ck.EXPORTED) == names


def test_dtype_helpers():
    assert [ck.element_size(d) for d in (0, 1, 2, 3, 4, 255)] == [4, 2, 2, 1, 4, 0]
    assert [ck.sidecar_bytes_per_elem(d) for d in (0, 1, 2, 3, 4, 255)] == [2, 1, 1, 0, 0, 0]


@pytest.mark.parametrize("seed", range(12))
@pytest.mark.parametrize("full", [False, True])
def test_build_table_matches_oracle(seed, full):
    rng = np.random.default_rng(seed)
    h = np.zeros(256, np.uint32)
    k = int(rng.integers(1, 257))
    idx = rng.choice(256, k, replace=False)
    h[idx] = rng.integers(1, 10 ** int(rng.integers(1, 8)), k)
    t, s = ck.build_table(h, full)
    r, rs = oc.normalize_histogram(h, full)
    assert s == rs
    assert t.raw_bytes() == r.tobytes()[: 40000 - 60]


def test_build_table_on_config_histograms():
    for dt, raw in ((dg.F32, dg.normal_f32(1 << 18, 1e-3, 0)), (dg.BF16, dg.normal_bf16(1 << 18, 0.02, 1)),
                    (dg.F32, dg.exp_avg_sq(1 << 18, 2)), (dg.F32, dg.adversarial_f32(1 << 18, 3, (0, 1 << 16)))):
        m, _ = oc.extract_mantissa(raw, raw.size, dt)
        h = oc.byte_hist(m)
        for full in (False, True):
            t, s = ck.build_table(h, full)
            r, rs = oc.normalize_histogram(h, full)
            assert s == rs and t.raw_bytes() == r.tobytes()[: 40000 - 60]


def test_geometry_queries():
    n = 1_003_782_656
    assert ck.num_units(n, ck.F32, 65536) == (4 * n + 65535) // 65536
    assert ck.num_units(n, ck.BF16, 65536) == (2 * n + 65535) // 65536
    assert ck.num_units(1000, ck.F32, 0) == 1
    assert ck.num_units(0, ck.F32, 65536) == 0
    lib = ck.lib()
    assert lib.ckr_encode_max_output_bytes(n, ck.F32, 65536) == 4 * n
    assert lib.ckr_encode_workspace_bytes(n, ck.F32, 65536) < (3 << 30)
    assert lib.ckr_decode_workspace_bytes(n, ck.F32, 65536) < (1 << 24)


def test_argument_errors_are_status_codes():
    lib = ck.lib()
    t, _ = ck.build_table(np.ones(256, np.uint32) * 16)
    vp = ctypes.c_void_p
    fake = vp(0x10000)  # never dereferenced: validation fails first
    rc = lib.ckr_encode(fake, 10, 99, t.ptr, 0, fake, 100, fake, fake, None, fake, 1 << 20, None, None)
    assert rc == ck.CKR_E_INVALID and b"dtype" in lib.ckr_last_error()
    rc = lib.ckr_encode(fake, 100000, ck.F32, t.ptr, 1000, fake, 400000, fake, fake, None, fake, 1 << 30, None, None)
    assert rc == ck.CKR_E_INVALID and b"multiple of 256" in lib.ckr_last_error()
    rc = lib.ckr_encode(vp(0x10001), 100000, ck.F32, t.ptr, 65536, fake, 400000, fake, fake, None, fake, 1 << 30,
                        None, None)
    assert rc == ck.CKR_E_INVALID and b"aligned" in lib.ckr_last_error()
    rc = lib.ckr_encode(fake, 100000, ck.F32, t.ptr, 65536, fake, 10, fake, fake, None, fake, 1 << 30, None, None)
    assert rc == ck.CKR_E_CAPACITY
    rc = lib.ckr_encode(fake, 100000, ck.F32, t.ptr, 65536, fake, 400000, fake, fake, None, fake, 16, None, None)
    assert rc == ck.CKR_E_CAPACITY and b"workspace" in lib.ckr_last_error()
    # single-unit layout is limited by the u32 header fields
    rc = lib.ckr_encode(fake, 1 << 31, ck.F32, t.ptr, 0, fake, 1 << 33, fake, fake, None, fake, 1 << 40, None, None)
    assert rc == ck.CKR_E_INVALID and b"2^32" in lib.ckr_last_error()
    # a table that does not sum to 4096 cannot be decoded
    h = np.ones(256, np.uint32)
    h[0] = 1_000_000
    bad_t, s = ck.build_table(h)
    assert s == 4348
    ws = lib.ckr_decode_workspace_bytes(1000, ck.I8, 256)
    rc = lib.ckr_decode(fake, fake, fake, bad_t.ptr, 1000, ck.I8, 256, None, fake, fake, ws, None, None)
    assert rc == ck.CKR_E_TABLE and b"4096" in lib.ckr_last_error()
    # masked dtypes need their sidecar
    rc = lib.ckr_decode(fake, fake, fake, t.ptr, 1000, ck.F32, 256, None, fake, fake, 1 << 20, None, None)
    assert rc == ck.CKR_E_INVALID and b"sidecar" in lib.ckr_last_error()


def test_fast_path_switch_round_trips():
    prev = ck.set_fast_paths(0)
    assert ck.set_fast_paths(2) == 0
    assert ck.set_fast_paths(3) == 2
    assert ck.set_fast_paths(prev) == 3
    assert ck.set_fast_paths(4) == prev   # out of range: back to 1
    assert ck.set_fast_paths(prev) == 1


def test_repair_host_helpers():
    """Bucket counts of the tie-break order come from libstdc++'s own policy:
    they must equal std::unordered_map::reserve(n).bucket_count()."""
    import random
    import oracle as oc
    rnd = random.Random(7)
    ns = list(range(0, 300)) + [rnd.randrange(2, 5_000_000) for _ in range(200)]
    assert all(ck.repair_bucket_count(n) == oc.repair_bucket_count(n) for n in ns)
    assert ck.repair_masked_bits(ck.F32) == 23 and ck.repair_masked_bits(ck.BF16) == 7
    assert ck.repair_masked_bits(ck.F16) == 10 and ck.repair_masked_bits(ck.F16, 3) == 3
    assert ck.repair_masked_bits(ck.BF16, 40) == 7 and ck.repair_masked_bits(ck.F32, 0) == 0
    with pytest.raises(ck.CkrError):
        ck.repair_masked_bits(ck.I32)
    assert ck.lib().ckr_repair_workspace_bytes(1 << 31, ck.F32, -1, 50) == 0


def test_encoder_job_record_follows_its_buffers():
    """compress_many copies each encoder's job record from a template: replacing
    one of the encoder's buffers (as a caller may, to point two jobs at
    overlapping ranges) must show in the record it passes."""
    import torch
    e = ck.Encoder(100_000, ck.F32, 65536, device="cpu")
    assert e._job.d_headers == e.headers.data_ptr()
    e.headers = torch.empty(e.headers.numel() + 16, dtype=torch.int32)
    e.out = torch.empty(e.out_cap, dtype=torch.uint8)
    assert e._job.d_headers == e.headers.data_ptr()
    assert e._job.d_out == e.out.data_ptr()
    assert e._job.d_workspace == e.ws.data_ptr() and e._job.workspace_bytes == e.ws_bytes
