"""GPU parity: the HIP library (through its C ABI) against the CPU oracle.

Bar: bit-exact histograms and tables, byte-identical encoded data, headers,
unit offsets and sidecars at the same unit size, and decode back to the input
bits.  Moments are the only floating-point outputs; their tolerance is stated
in test_analyzer_parity.
"""
import numpy as np
import pytest

import oracle as oc
from tests import datagen as dg

pytestmark = pytest.mark.gpu


def _ck():
    import checkers_amd as ck
    return ck


def _to_dev(arr, gpu):
    import torch
    b = dg.raw_bytes(arr)
    t = torch.empty(max(b.size, 16), dtype=torch.uint8, device=gpu)
    if b.size:
        t[: b.size].copy_(torch.from_numpy(b.copy()))
    return t


CASES = [
    # (name, dtype, n, unit, generator)
    ("f32_normal_64k", dg.F32, 16384 * 5 + 1000, 65536, lambda n: dg.normal_f32(n, 1e-3, 0)),
    ("f32_normal_whole", dg.F32, 40000, 0, lambda n: dg.normal_f32(n, 1e-3, 1)),
    ("f32_normal_768", dg.F32, 20011, 768, lambda n: dg.normal_f32(n, 1e-3, 2)),
    ("f32_expavgsq_64k", dg.F32, 16384 * 3, 65536, lambda n: dg.exp_avg_sq(n, 3)),
    ("f32_upcast_bf16", dg.F32, 50000, 65536,
     lambda n: (dg.normal_bf16(n, 0.02, 4).astype(np.uint32) << 16).view(np.float32)),
    ("bf16_normal_64k", dg.BF16, 32768 * 3 + 1, 65536, lambda n: dg.normal_bf16(n, 0.02, 5)),
    ("bf16_normal_whole", dg.BF16, 30001, 0, lambda n: dg.normal_bf16(n, 0.02, 6)),
    ("bf16_normal_4k", dg.BF16, 70000, 4096, lambda n: dg.normal_bf16(n, 0.02, 7)),
    ("bf16_rmsnorm_ones", dg.BF16, 4096, 65536, lambda n: dg.f32_to_bf16_bits(np.ones(n, np.float32))),
    ("f16_normal", dg.F16, 10001, 1024, lambda n: (np.random.default_rng(8).standard_normal(n) * 0.02).astype(np.float16)),
    ("i8_random", dg.I8, 100000, 2048, lambda n: np.random.default_rng(9).integers(-128, 128, n).astype(np.int8)),
    ("i8_const", dg.I8, 3000, 512, lambda n: np.full(n, 7, np.int8)),
    ("i32_small", dg.I32, 50000, 65536, lambda n: np.random.default_rng(10).integers(-3, 4, n).astype(np.int32)),
    ("adversarial_f32", dg.F32, 300000, 65536, lambda n: dg.adversarial_f32(n, 11, (100000, 150000))),
    ("random_bits_f32", dg.F32, 16384 * 4, 65536,  # live lanes ~9 bits/symbol: decode staging overflows
     lambda n: np.random.default_rng(13).integers(0, 2**32, n, dtype=np.uint64).astype(np.uint32).view(np.float32)),
    ("random_bits_bf16", dg.BF16, 32768 * 2 + 6, 65536,
     lambda n: np.random.default_rng(14).integers(0, 2**16, n).astype(np.uint16)),
    ("f32_1mib_units", dg.F32, 262144 * 2 + 4097, 1 << 20, lambda n: dg.normal_f32(n, 1e-3, 15)),
    ("f32_expavgsq_128k_units", dg.F32, 32832 * 4 + 100, 131328, lambda n: dg.exp_avg_sq(n, 17)),
    ("bf16_1mib_units", dg.BF16, 524288 * 2 + 1111, 1 << 20, lambda n: dg.normal_bf16(n, 0.02, 18)),
    ("bf16_256k_one_unit", dg.BF16, 131072, 262144, lambda n: dg.normal_bf16(n, 0.02, 19)),
    # 1 MiB units of random bits (passthrough units) and an adversarial mix at
    # 256 KiB units, whole units and a partial last one
    ("random_bits_f32_1mib", dg.F32, 262144 * 2 + 333, 1 << 20,
     lambda n: np.random.default_rng(20).integers(0, 2**32, n, dtype=np.uint64).astype(np.uint32).view(np.float32)),
    ("adversarial_f32_256k", dg.F32, 65536 * 3 + 999, 262144, lambda n: dg.adversarial_f32(n, 21, (70000, 140000))),
    # units above 1 MiB (one chain per lane, then the 1024-row segments side by
    # side): the one-stream layout of a tensor with a partial top row, one that
    # ends on a segment boundary, and 4 MiB units with a partial last one
    ("f32_whole_long", dg.F32, 600001, 0, lambda n: dg.normal_f32(n, 1e-3, 24)),
    ("bf16_whole_long", dg.BF16, 1300001, 0, lambda n: dg.normal_bf16(n, 0.02, 25)),
    ("f32_whole_long_segments", dg.F32, 256 * 1024 * 5 // 4, 0, lambda n: dg.exp_avg_sq(n, 26)),
    ("f16_whole_long", dg.F16, 700003, 0, lambda n: (np.random.default_rng(27).standard_normal(n) * 0.02).astype(np.float16)),
    ("f32_4mib_units", dg.F32, (1 << 20) * 2 + 12345, 4 << 20, lambda n: dg.adversarial_f32(n, 28, (300000, 400000))),
    ("bf16_partial_units", dg.BF16, 3 * 512 + 1, 1024, lambda n: dg.normal_bf16(n, 0.02, 16)),
    ("tiny_f32_1", dg.F32, 1, 65536, lambda n: np.array([1.5], np.float32)),
    ("tiny_bf16_3", dg.BF16, 3, 0, lambda n: dg.normal_bf16(n, 0.02, 12)),
    ("tiny_i8_255", dg.I8, 255, 0, lambda n: np.arange(n, dtype=np.uint8).view(np.int8)),
    ("tiny_i8_256", dg.I8, 256, 256, lambda n: np.arange(n, dtype=np.uint8).view(np.int8)),
    ("tiny_i8_257", dg.I8, 257, 256, lambda n: np.arange(n, dtype=np.uint8).view(np.int8)),
    ("empty_f32", dg.F32, 0, 65536, lambda n: np.zeros(0, np.float32)),
]


@pytest.fixture(params=[1, 0, 2, 3], ids=["fast", "general", "overflow", "overflow_fast_redo"])
def paths(request):
    ck = _ck()
    prev = ck.set_fast_paths(request.param)
    yield request.param
    ck.set_fast_paths(prev)


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_compress_parity_and_roundtrip(case, paths, gpu):
    import torch
    ck = _ck()
    name, dt, n, unit, gen = case
    print(f"[case] {name} dtype={dt} n={n} unit={unit} fast={paths}", flush=True)
    raw = gen(n)
    ref = oc.compress_tensor(raw, n, dt, unit)
    src = _to_dev(raw, gpu)
    enc = ck.compress(src, dt, unit, n_elems=n)
    torch.cuda.synchronize()
    # table
    assert np.array_equal(enc.table.norm, ref["table"]["norm_freq"])
    assert np.array_equal(enc.table.cum, ref["table"]["cum_freq"])
    # packed data, headers, unit offsets
    assert enc.total == ref["data"].size
    nu = ref["unit_offsets"].size - 1
    assert np.array_equal(enc.unit_offsets[: nu + 1].cpu().numpy().view(np.uint64), ref["unit_offsets"])
    if nu:
        assert np.array_equal(enc.headers_np()[: nu * 256], ref["headers"])
    assert np.array_equal(enc.data_np(), ref["data"])
    # sidecar
    spe = oc.SPE[dt]
    if spe and n:
        assert np.array_equal(enc.sidecar[: n * spe].cpu().numpy(), ref["sidecar"])
    # decode → original bits
    dst, bad = ck.decode(enc)
    torch.cuda.synchronize()
    assert bad == 0
    assert np.array_equal(dst.cpu().numpy(), dg.raw_bytes(raw))


@pytest.mark.parametrize("mode", [1, 3, 2])
def test_overflowing_units_take_the_redo_route(mode, gpu):
    """Units of uniform random bits inside lognormal data outgrow the LDS slots
    sized from the whole tensor: by default (mode 1) they, and in mode 3 (minimal
    slots) every unit, are coded again by the fast encoder with slots that hold
    any lane, with no general-kernel launch; mode 2 sends them through the
    general kernels.  Bytes equal the oracle's."""
    import torch
    ck = _ck()
    n = 65536 // 4 * 40 + 77
    raw = dg.adversarial_f32(n, 31, (16384 * 7, 16384 * 12))
    ref = oc.compress_tensor(raw, n, dg.F32, 65536)
    src = _to_dev(raw, gpu)
    prev = ck.set_fast_paths(mode)
    try:
        ck.compress(src, dg.F32, 65536, n_elems=n)   # warm-up
        torch.cuda.synchronize()
        ck.profile_begin()
        enc = ck.compress(src, dg.F32, 65536, n_elems=n)
        torch.cuda.synchronize()
        prof = ck.profile_end()
    finally:
        ck.set_fast_paths(prev)
    print(f"[case] redo route mode={mode}: {sorted(prof)}", flush=True)
    if mode == 2:
        assert "encode_kernel" in prof and "encode_fast_redo_kernel" not in prof
    else:
        assert "encode_kernel" not in prof and "compact_kernel" not in prof
        assert mode == 1 or "encode_fast_redo_kernel" in prof
    assert enc.total == ref["data"].size
    assert np.array_equal(enc.headers_np()[: 41 * 256], ref["headers"])
    assert np.array_equal(enc.data_np(), ref["data"])
    dst, bad = ck.decode(enc)
    torch.cuda.synchronize()
    assert bad == 0 and np.array_equal(dst.cpu().numpy(), dg.raw_bytes(raw))


@pytest.mark.parametrize("dt,gen", [
    (dg.F32, lambda n: dg.normal_f32(n, 1e-3, 20)),
    (dg.BF16, lambda n: dg.normal_bf16(n, 0.02, 21)),
    (dg.F16, lambda n: (np.random.default_rng(22).standard_normal(n)).astype(np.float16)),
    (dg.I8, lambda n: np.random.default_rng(23).integers(-128, 128, n).astype(np.int8)),
])
@pytest.mark.parametrize("n", [1, 7, 4099, 1 << 20])
def test_histogram_and_split_parity(dt, gen, n, gpu):
    import torch
    ck = _ck()
    print(f"[case] hist dtype={dt} n={n}", flush=True)
    raw = gen(n)
    masked, side = oc.extract_mantissa(raw, n, dt)
    src = _to_dev(raw, gpu)
    h = ck.byte_histogram(src, dt, n_elems=n)
    torch.cuda.synchronize()
    assert np.array_equal(h.cpu().numpy().view(np.uint32), oc.byte_hist(masked))
    if oc.SPE[dt]:
        m, s = ck.extract_mantissa(src, dt, n_elems=n)
        torch.cuda.synchronize()
        assert np.array_equal(m.cpu().numpy(), masked)
        assert np.array_equal(s.cpu().numpy(), side)


def test_passthrough_unit_with_mismatched_table(gpu):
    """A table that prices the data badly makes units expand → stored raw (ANSCompressor.cpp:694-713)."""
    import torch
    ck = _ck()
    n, unit = 20000, 1024
    rng = np.random.default_rng(30)
    raw = rng.integers(-128, 128, n).astype(np.int8)
    raw[:3000] = 0  # first units compress, the rest expand
    h = np.full(256, 100, np.uint32)
    h[0] = 100_000  # rare symbols get 3-4 slots: ~10 bits each, so random bytes expand
    t_ck, s_ck = ck.build_table(h)
    t_oc, s_oc = oc.normalize_histogram(h)
    assert s_ck == s_oc == 4096
    data, hdr, off = oc.encode(dg.raw_bytes(raw), t_oc, unit)
    src = _to_dev(raw, gpu)
    enc = ck.encode(src, dg.I8, t_ck, unit, n_elems=n)
    torch.cuda.synchronize()
    sizes = np.diff(off.astype(np.int64))
    assert (sizes == unit).any() and (sizes < unit).any()  # both kinds of unit present
    assert enc.total == data.size
    assert np.array_equal(enc.data_np(), data)
    assert np.array_equal(enc.headers_np()[: hdr.size], hdr)
    dst, bad = ck.decode(enc)
    assert bad == 0 and np.array_equal(dst.cpu().numpy(), dg.raw_bytes(raw))


@pytest.mark.parametrize("dt,unit,n", [
    (dg.F32, 1 << 20, (1 << 18) * 3 + 5000),
    (dg.F32, 131328, 32832 * 4 + 17),
    (dg.BF16, 1 << 18, (1 << 17) * 2 + 333),
    (dg.F32, 2 << 20, (1 << 19) * 3 + 4321),
    (dg.BF16, 3 << 20, (3 << 19) * 2 + 77),
])
def test_large_units_with_foreign_table(dt, unit, n, paths, gpu):
    """Units above 64 KiB under a table that does not fit the data: alternate
    units expand (stored raw, ANSCompressor.cpp:694-713) and contain symbols
    with f == 0 (raw-byte escape, :185-192)."""
    import torch
    ck = _ck()
    es = 4 if dt == dg.F32 else 2
    print(f"[case] large units foreign table dtype={dt} unit={unit} n={n} fast={paths}", flush=True)
    rng = np.random.default_rng(50)
    b = rng.integers(0, 256, (n, es), dtype=np.uint8)
    cheap = (np.arange(n) // (unit // es)) % 2 == 0
    for c in ([2, 3] if es == 4 else [1]):  # live bytes of the cheap units: symbols 1..8
        b[cheap, c] = rng.integers(1, 9, int(cheap.sum()))
    raw = b.reshape(-1).view(np.uint32 if es == 4 else np.uint16)
    h = np.full(256, 16, np.uint32)
    h[1:9] = 1000
    h[200:] = 0
    t_ck, s_ck = ck.build_table(h)
    t_oc, s_oc = oc.normalize_histogram(h)
    assert s_ck == s_oc == 4096
    masked, side = oc.extract_mantissa(raw, n, dt)
    data, hdr, off = oc.encode(masked, t_oc, unit)
    sizes = np.diff(off.astype(np.int64))
    lens = np.minimum(unit, n * es - unit * np.arange(sizes.size))
    assert (sizes == lens).any() and (sizes < lens).any()  # both kinds of unit present
    enc = ck.encode(_to_dev(raw, gpu), dt, t_ck, unit, n_elems=n)
    torch.cuda.synchronize()
    assert enc.total == data.size
    assert np.array_equal(enc.unit_offsets[: off.size].cpu().numpy().view(np.uint64), off)
    assert np.array_equal(enc.headers_np()[: hdr.size], hdr)
    assert np.array_equal(enc.data_np(), data)
    assert np.array_equal(enc.sidecar[: side.size].cpu().numpy(), side)
    dst, bad = ck.decode(enc)
    torch.cuda.synchronize()
    assert bad == 0 and np.array_equal(dst.cpu().numpy(), dg.raw_bytes(raw))


@pytest.mark.parametrize("dt", [dg.F32, dg.BF16])
def test_one_stream_tensor_stored_raw(dt, paths, gpu):
    """The one-stream layout (unit_bytes 0) of a tensor above 1 MiB under a table
    that prices its live bytes badly: the whole tensor expands and is stored raw
    (ANSCompressor.cpp:694-713), with escapes for the symbols the table lacks
    (:185-192); bytes equal the oracle's and the decode copies it back."""
    import torch
    ck = _ck()
    es = 4 if dt == dg.F32 else 2
    n = (3 << 20) // es + 37
    print(f"[case] one-stream raw dtype={dt} n={n} fast={paths}", flush=True)
    raw = np.random.default_rng(52).integers(0, 256, n * es, dtype=np.uint8).view(np.uint32 if es == 4 else np.uint16)
    h = np.full(256, 1, np.uint32)
    h[1] = 3000  # every other symbol, zero included, gets one slot (12 bits); the table sums to 4096
    h[240:] = 0
    t_ck, s_ck = ck.build_table(h)
    t_oc, s_oc = oc.normalize_histogram(h)
    assert s_ck == s_oc == 4096
    masked, side = oc.extract_mantissa(raw, n, dt)
    data, hdr, off = oc.encode(masked, t_oc, 0)
    assert off[1] == n * es  # stored raw
    enc = ck.encode(_to_dev(raw, gpu), dt, t_ck, 0, n_elems=n)
    torch.cuda.synchronize()
    assert enc.total == data.size
    assert np.array_equal(enc.headers_np()[: hdr.size], hdr)
    assert np.array_equal(enc.data_np(), data)
    assert np.array_equal(enc.sidecar[: side.size].cpu().numpy(), side)
    dst, bad = ck.decode(enc)
    torch.cuda.synchronize()
    assert bad == 0 and np.array_equal(dst.cpu().numpy(), dg.raw_bytes(raw))


def test_escape_symbols_match_reference_bytes(gpu):
    """Symbols with f == 0 take the reference's raw-byte escape (ANSCompressor.cpp:185-192)."""
    import torch
    ck = _ck()
    n, unit = 8192, 4096
    raw = np.random.default_rng(31).integers(0, 16, n).astype(np.int8)
    h = np.zeros(256, np.uint32)
    h[:10] = 100  # symbols 10..15 absent from the table
    t_ck, _ = ck.build_table(h)
    t_oc, _ = oc.normalize_histogram(h)
    data, hdr, off = oc.encode(dg.raw_bytes(raw), t_oc, unit)
    enc = ck.encode(_to_dev(raw, gpu), dg.I8, t_ck, unit, n_elems=n)
    torch.cuda.synchronize()
    assert enc.total == data.size
    assert np.array_equal(enc.data_np(), data)
    assert np.array_equal(enc.headers_np()[: hdr.size], hdr)


@pytest.mark.parametrize("dt,n,bins,gen", [
    (dg.F32, 100000, 256, lambda n: dg.normal_f32(n, 1e-3, 40)),
    (dg.F32, 4097, 16, lambda n: dg.exp_avg_sq(n, 41)),
    (dg.BF16, 70001, 4096, lambda n: dg.normal_bf16(n, 0.02, 42)),
    (dg.F16, 5000, 256, lambda n: (np.random.default_rng(43).standard_normal(n)).astype(np.float16)),
    (dg.I8, 3001, 256, lambda n: np.random.default_rng(44).integers(-128, 128, n).astype(np.int8)),
    (dg.I32, 3001, 100, lambda n: np.random.default_rng(45).integers(-10**6, 10**6, n).astype(np.int32)),
    (dg.F32, 1000, 256, lambda n: np.full(n, 0.25, np.float32)),           # range 0 → bin 0
    (dg.F32, 20000, 256, lambda n: dg.adversarial_f32(n, 46)),             # NaN / inf / denormals
])
def test_analyzer_parity(dt, n, bins, gen, gpu):
    ck = _ck()
    import torch
    print(f"[case] analyze dtype={dt} n={n} bins={bins}", flush=True)
    raw = gen(n)
    ref = oc.tensor_stats(raw, n, dt, bins)
    got = ck.analyze([_to_dev(raw, gpu)[: n * oc.ES[dt]]], [dt], bins=bins)[0]
    torch.cuda.synchronize()
    # min/max are order-independent: exact (== treats ±0 alike)
    assert np.array_equal(got["minmax"], ref["minmax"]) or (got["minmax"] == ref["minmax"]).all()
    # histogram: bit-exact given exact min/max and IEEE fp32 sub/mul
    assert np.array_equal(got["histogram"], ref["histogram"])
    # moments: the GPU sums in fp64, the reference in fp32; compare both with the
    # fp64 closed form: mean to 1e-6 of the spread, var/skew/kurt to 1e-4 relative.
    m64 = ref["moments64"]
    if np.all(np.isfinite(m64)):
        spread = max(abs(float(ref["minmax"][1]) - float(ref["minmax"][0])), 1e-30)
        assert abs(got["moments"][0] - m64[0]) <= 1e-6 * spread + 1e-30
        assert abs(got["moments"][1] - m64[1]) <= 1e-4 * abs(m64[1]) + 1e-30
        if m64[1] > 1e-9 * (1 + 1e-4):  # skew/kurt only above the reference's var > 1e-9 gate
            for k in (2, 3):
                assert abs(got["moments"][k] - m64[k]) <= 1e-4 * max(abs(m64[k]), 1.0), (k, got["moments"], m64)
        elif m64[1] < 1e-9 * (1 - 1e-4):
            assert got["moments"][2] == 0 and got["moments"][3] == 0
    fp = got["fingerprint"]
    assert np.array_equal(fp[:4], got["moments"], equal_nan=True)
    assert np.array_equal(fp[4:], np.float32(got["minmax"][1] - got["minmax"][0]).reshape(1), equal_nan=True)


@pytest.mark.parametrize("dt,n,unit,gen", [
    (dg.F32, 16384 * 3 + 77, 65536, lambda n: dg.normal_f32(n, 1e-3, 21)),
    (dg.BF16, 32768 + 4099, 4096, lambda n: dg.normal_bf16(n, 0.02, 22)),
    (dg.F32, 300, 1024, lambda n: dg.exp_avg_sq(n, 23)),
])
@pytest.mark.parametrize("shift", [0, 5, 61])
def test_decode_from_relocated_stream(dt, n, unit, gen, shift, gpu):
    """The packed bytes moved to a buffer that ends right after them and starts
    `shift` bytes past a 64-byte boundary: chunks around both ends of the buffer
    are read only inside it, and decoding stays bit-exact."""
    import torch
    ck = _ck()
    print(f"[case] relocated dtype={dt} n={n} unit={unit} shift={shift}", flush=True)
    raw = gen(n)
    src = _to_dev(raw, gpu)
    enc = ck.compress(src, dt, unit, n_elems=n)
    torch.cuda.synchronize()
    base = torch.zeros(enc.total + 64, dtype=torch.uint8, device=gpu)
    moved = base[shift: shift + enc.total]
    moved.copy_(enc.data[: enc.total])
    dst = torch.empty(n * ck.element_size(dt), dtype=torch.uint8, device=gpu)
    d = ck.Decoder(n, dt, unit, device=gpu)
    bad = d.decode(moved, enc.headers, enc.unit_offsets, enc.table, enc.sidecar, dst)
    torch.cuda.synchronize()
    assert bad == 0
    assert np.array_equal(dst.cpu().numpy(), dg.raw_bytes(raw))


def test_histogram_counts_wrap_like_reference(gpu):
    """Counts are uint32 and wrap modulo 2^32 past 4 Gi occurrences of one byte
    value, as the reference's g_hist does (src/ANSCompressor.cpp:109-126,
    uint32_t atomicAdd); the table is then normalised from the wrapped counts
    (src/ANSCompressor.cpp:416-451).  6.4 GB bf16: a seeded prefix, zeros after."""
    import torch
    ck = _ck()
    n, m = (1 << 31) + (1 << 30) + 12345, 1 << 20
    print(f"[case] hist wrap bf16 n={n}", flush=True)
    pat = dg.normal_bf16(m, 0.02, 5)
    masked, _ = oc.extract_mantissa(pat, m, dg.BF16)
    want = oc.byte_hist(masked).astype(np.uint64)
    want[0] += 2 * (n - m)
    want = (want % (1 << 32)).astype(np.uint32)
    assert int(want[0]) != 2 * (n - m) + int(oc.byte_hist(masked)[0])  # the case does wrap
    t = torch.zeros(n, dtype=torch.int16, device=gpu)
    t[:m].copy_(torch.from_numpy(pat.view(np.int16).copy()))
    h = ck.byte_histogram(t, dg.BF16, n_elems=n)
    torch.cuda.synchronize()
    del t
    got = h.cpu().numpy().view(np.uint32)
    assert np.array_equal(got, want)
    tab, tsum = ck.build_table(got)
    ref, rsum = oc.normalize_histogram(want)
    assert np.array_equal(tab.norm, ref["norm_freq"]) and np.array_equal(tab.cum, ref["cum_freq"])
    assert tsum == rsum  # 4115 here: the reference's over-full table for a dominant symbol


@pytest.mark.parametrize("unit", [65536, 1 << 20, 4 << 20])
@pytest.mark.parametrize("where", ["live", "zero", "state", "zero_last", "zero_header"])
def test_decode_counts_corrupted_lanes(unit, where, gpu):
    """A flipped byte in a live lane's stream or a zero-plane lane's stream, or a
    wrong final state, is reported as a bad lane (the decoder's postconditions:
    final state L, every byte consumed, canonical zero-plane streams).  A
    zero-plane lane's bytes are compared step by step during the decode (units
    up to 1 MiB) or decoded (above: they must give zeros): a flip in its first
    or last byte, in the second unit, or in its header counts that one lane.
    Those bytes do not enter the output, and a decode that does not read the
    count gives the original bytes without comparing them."""
    import torch
    ck = _ck()
    n = (unit // 4) * 2 + 777
    print(f"[case] corruption {where} unit={unit}", flush=True)
    raw = dg.normal_f32(n, 1e-3, 60)
    enc = ck.compress(_to_dev(raw, gpu), dg.F32, unit, n_elems=n)
    torch.cuda.synchronize()
    dst, bad = ck.decode(enc)
    assert bad == 0 and np.array_equal(dst.cpu().numpy(), dg.raw_bytes(raw))
    hdr = enc.headers_np()
    lane = {"live": 3, "zero": 0, "state": 2, "zero_last": 256 + 1, "zero_header": 256 + 4}[where]
    h = hdr[lane]  # fp32 columns: bytes 0, 1 masked, 2, 3 live; lanes 256.. are unit 1's
    assert h["byte_count"] > 8
    uo = int(enc.unit_offsets[lane // 256].cpu())
    if where == "state":
        enc.headers.view(-1)[4 * lane] ^= 0x40  # final_state of unit 0, lane 2
    elif where == "zero_header":
        enc.headers.view(-1)[4 * lane] ^= 0x40  # final_state of unit 1, lane 4 (zero-plane)
    elif where == "zero_last":
        enc.data[uo + int(h["buf_offset"]) + int(h["byte_count"]) - 1] ^= 0x01
    else:
        enc.data[uo + int(h["buf_offset"]) + 5] ^= 0x10
    torch.cuda.synchronize()
    _, bad = ck.decode(enc)
    torch.cuda.synchronize()
    if where.startswith("zero"):
        assert bad == 1
    else:
        assert bad >= 1
    if where in ("zero", "zero_last"):
        # a zero-plane lane's bytes do not enter the output: a decode that does
        # not read the count (and so does not compare them) still gives the
        # original bytes, alone and in ckr_decode_many
        d = ck.Decoder(n, dg.F32, unit, device=gpu)
        out = torch.empty(n * 4, dtype=torch.uint8, device=gpu)
        assert d.decode(enc.data, enc.headers, enc.unit_offsets, enc.table, enc.sidecar, out, check=False) is None
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy(), dg.raw_bytes(raw))
        out.zero_()
        assert ck.decode_many([d], [enc], [out], check=False) is None
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy(), dg.raw_bytes(raw))


@pytest.mark.parametrize("tag,unit", [(dg.F32, 1 << 20), (dg.BF16, 1 << 20), (dg.F32, 65536)])
def test_encode_planes_matches_encode(tag, unit, paths, gpu):
    """ckr_byte_histogram_planes: the masked histogram and the two live planes'
    (checked against numpy); ckr_encode_planes gives ckr_encode's bytes, and a
    slice of whole units under the whole tensor's table gives the whole
    encode's first units (units are independent given the table)."""
    import torch
    ck = _ck()
    es = 4 if tag == dg.F32 else 2
    n = (unit // es) * 3 + 771
    print(f"[case] encode_planes tag={tag} unit={unit}", flush=True)
    raw = dg.normal_f32(n, 1e-3, 40) if tag == dg.F32 else dg.normal_bf16(n, 0.02, 41)
    t = _to_dev(raw, gpu)
    hh = ck.byte_histogram(t, tag, n_elems=n, planes=True).cpu().numpy().view(np.uint32)
    masked, _ = oc.extract_mantissa(raw, n, tag)
    mb = np.frombuffer(masked.tobytes(), np.uint8)
    fl = 2 if tag == dg.F32 else 1
    assert np.array_equal(hh[:256], oc.byte_hist(masked))
    assert np.array_equal(hh[256:512], np.bincount(mb[fl::4], minlength=256))
    assert np.array_equal(hh[512:], np.bincount(mb[3::4], minlength=256))
    assert np.array_equal(hh[:256], ck.byte_histogram(t, tag, n_elems=n).cpu().numpy().view(np.uint32))
    table, _ = ck.build_table(hh[:256])
    e1 = ck.Encoder(n, tag, unit, device=gpu).encode(t, table)
    e2 = ck.Encoder(n, tag, unit, device=gpu).encode(t, table, planes=hh[256:])
    torch.cuda.synchronize()
    assert e1.total == e2.total
    assert torch.equal(e1.data[: e1.total], e2.data[: e2.total])
    assert torch.equal(e1.headers, e2.headers) and torch.equal(e1.unit_offsets, e2.unit_offsets)
    assert torch.equal(e1.sidecar, e2.sidecar)
    # plane histograms that say nothing true about the data (empty, one hot bin)
    # only size the slots: the bytes stay ckr_encode's
    for bogus in (np.zeros(512, np.uint32), np.eye(1, 512, 7, dtype=np.uint32).reshape(-1) * 1000):
        e4 = ck.Encoder(n, tag, unit, device=gpu).encode(t, table, planes=bogus)
        torch.cuda.synchronize()
        assert e4.total == e1.total and torch.equal(e4.data[: e4.total], e1.data[: e1.total])
        assert torch.equal(e4.headers, e1.headers) and torch.equal(e4.unit_offsets, e1.unit_offsets)
    m = 2 * unit // es
    e3 = ck.Encoder(m, tag, unit, device=gpu).encode(t[: m * es], table, planes=hh[256:])
    torch.cuda.synchronize()
    off = e1.unit_offsets.cpu().numpy()
    assert e3.total == int(off[2])
    assert torch.equal(e3.data[: e3.total], e1.data[: e3.total])
    assert torch.equal(e3.headers.reshape(-1), e1.headers.reshape(-1)[: e3.headers.numel()])
    assert np.array_equal(e3.unit_offsets.cpu().numpy(), off[:3])
    spe = oc.SPE[tag]
    assert torch.equal(e3.sidecar[: m * spe], e1.sidecar[: m * spe])


@pytest.mark.parametrize("unit", [65536, 1 << 20, 0])
def test_compress_many_matches_single_calls(unit, paths, gpu):
    """ckr_compress_many (jobs this small: every histogram first, then the
    encodes back to back) gives each job exactly what ckr_compress gives it, and
    the oracle's bytes; with unit 0 (one stream per tensor) the 1.2 MB fp32
    tensor takes the long-unit kernels, the bf16 one the two-pass encoder."""
    import torch
    ck = _ck()
    specs = [(dg.F32, 300001, lambda n: dg.normal_f32(n, 1e-3, 70)),
             (dg.BF16, 400003, lambda n: dg.normal_bf16(n, 0.02, 71)),
             (dg.F32, 0, lambda n: np.zeros(0, np.float32)),
             (dg.F32, 50000, lambda n: dg.exp_avg_sq(n, 72)),
             (dg.I8, 70001, lambda n: np.random.default_rng(73).integers(-4, 4, n).astype(np.int8))]
    print(f"[case] compress_many unit={unit} fast={paths}", flush=True)
    raws = [gen(n) for _, n, gen in specs]
    srcs = [_to_dev(r, gpu) for r in raws]
    encs = [ck.Encoder(n, dt, unit, device=gpu) for dt, n, _ in specs]
    many = ck.compress_many(encs, srcs)
    torch.cuda.synchronize()
    for (dt, n, _), raw, src, m in zip(specs, raws, srcs, many):
        ref = oc.compress_tensor(raw, n, dt, unit)
        assert np.array_equal(m.table.norm, ref["table"]["norm_freq"])
        assert m.total == ref["data"].size
        assert np.array_equal(m.data_np(), ref["data"])
        nu = ref["unit_offsets"].size - 1
        assert np.array_equal(m.unit_offsets[: nu + 1].cpu().numpy().view(np.uint64), ref["unit_offsets"])
        assert np.array_equal(m.headers_np()[: nu * 256], ref["headers"])
        if oc.SPE[dt]:
            assert np.array_equal(m.sidecar[: n * oc.SPE[dt]].cpu().numpy(), ref["sidecar"])
        dst, bad = ck.decode(m)
        torch.cuda.synchronize()
        assert bad == 0 and np.array_equal(dst.cpu().numpy(), dg.raw_bytes(raw))
    with pytest.raises(ck.CkrError):  # one Encoder twice would share its buffers
        ck.compress_many([encs[0], encs[0]], [srcs[0], srcs[0]])


@pytest.mark.parametrize("batched", [True, False])
def test_decode_many_matches_single_decodes(batched, gpu):
    """ckr_decode_many (tensors this small decoded together: in one set-up and
    one decode launch per dtype class when the fast decoder takes every job,
    else side by side on four streams, here forced by an int8 job) restores
    every job bit-exact and reports each job's bad lanes as ckr_decode does: a
    job whose stream bytes were corrupted counts its own bad lanes and no other
    job counts any; check=False queues the same work without a
    synchronisation; one Decoder twice is refused."""
    import torch
    ck = _ck()
    g = torch.Generator(device=gpu).manual_seed(81)
    ts = [(torch.randn(n, device=gpu, generator=g) * sc).to(dt) for n, sc, dt in
          ((300_001, 0.02, torch.bfloat16), (1 << 20, 1e-3, torch.float32), (5, 1e-3, torch.float32),
           (2_000_003, 0.02, torch.bfloat16), (0, 1.0, torch.float32), (700_000, 1e-3, torch.float32))]
    if not batched:
        ts.append(torch.randint(-128, 128, (100_003,), dtype=torch.int8, device=gpu, generator=g))
    tags = [ck.torch_tag(t.dtype) for t in ts]
    srcs = [t.view(torch.uint8) for t in ts]
    print("[case] decode_many", flush=True)
    encs = ck.compress_many([ck.Encoder(t.numel(), tag, 65536, device=gpu) for t, tag in zip(ts, tags)], srcs)
    decs = [ck.Decoder(t.numel(), tag, 65536, device=gpu) for t, tag in zip(ts, tags)]
    dsts = [torch.empty(max(s.numel(), 1), dtype=torch.uint8, device=gpu) for s in srcs]
    bads = ck.decode_many(decs, encs, dsts)
    assert bads == [0] * len(ts)
    for s, d in zip(srcs, dsts):
        assert torch.equal(d[: s.numel()], s)
    for d in dsts:
        d.zero_()
    assert ck.decode_many(decs, encs, dsts, check=False) is None
    torch.cuda.synchronize()
    for s, d in zip(srcs, dsts):
        assert torch.equal(d[: s.numel()], s)
    # corrupt job 3's stream bytes in the middle of its data
    e3 = encs[3]
    mid = e3.total // 2
    e3.data[mid: mid + 64] ^= 0x5A
    one = decs[3].decode(e3.data, e3.headers, e3.unit_offsets, e3.table, e3.sidecar,
                         torch.empty_like(dsts[3]))
    assert one > 0
    bads = ck.decode_many(decs, encs, dsts)
    assert bads[3] == one and all(b == 0 for k, b in enumerate(bads) if k != 3)
    with pytest.raises(ck.CkrError):
        ck.decode_many([decs[0], decs[0]], encs[:2], dsts[:2])


def test_decode_many_large_jobs_alternate_streams(gpu):
    """Jobs above 256 MiB (decoded alternately on two streams, each starting as
    the previous one drains): every job bit-exact with no bad lanes, with and
    without the synchronising check."""
    import torch
    ck = _ck()
    g = torch.Generator(device=gpu).manual_seed(82)
    ts = [torch.randn(70_000_003, device=gpu, generator=g) * 1e-3,
          (torch.randn(3_000_001, device=gpu, generator=g) * 0.02).to(torch.bfloat16),
          torch.randn(68_000_000, device=gpu, generator=g) * 1e-3]
    tags = [ck.torch_tag(t.dtype) for t in ts]
    srcs = [t.view(torch.uint8) for t in ts]
    print("[case] decode_many large jobs", flush=True)
    encs = ck.compress_many([ck.Encoder(t.numel(), tag, 65536, device=gpu) for t, tag in zip(ts, tags)], srcs)
    decs = [ck.Decoder(t.numel(), tag, 65536, device=gpu) for t, tag in zip(ts, tags)]
    dsts = [torch.empty_like(s) for s in srcs]
    assert ck.decode_many(decs, encs, dsts) == [0, 0, 0]
    for s, d in zip(srcs, dsts):
        assert torch.equal(d, s)
    for d in dsts:
        d.zero_()
    ck.decode_many(decs, encs, dsts, check=False)
    torch.cuda.synchronize()
    for s, d in zip(srcs, dsts):
        assert torch.equal(d, s)


def test_compress_many_repeated_byte_identical(gpu):
    """Regression for a race between the fast encoder's packer waves (one of them
    wrote the lane records over the exchange words before the others had read
    them, so a late packer could pack with wrong lane sizes while the headers
    stayed right): many compress_many calls, each tensor byte-identical to one
    ckr_compress of it every time."""
    import torch
    ck = _ck()
    g = torch.Generator(device=gpu)
    g.manual_seed(80)
    ts = [(torch.randn(n, device=gpu, generator=g) * s).to(dt) for n, s, dt in
          ((16 << 20, 0.02, torch.bfloat16), (4 << 20, 0.02, torch.bfloat16), (8 << 20, 1e-3, torch.float32),
           (6 << 20, 0.02, torch.bfloat16), (2 << 20, 1e-3, torch.float32))]
    tags = [ck.torch_tag(t.dtype) for t in ts]
    srcs = [t.view(torch.uint8) for t in ts]
    refs = []
    for t, tag, s in zip(ts, tags, srcs):
        e = ck.Encoder(t.numel(), tag, 65536, device=gpu).compress(s)
        torch.cuda.synchronize()
        refs.append(e.data[: e.total].clone())
    encs = [ck.Encoder(t.numel(), tag, 65536, device=gpu) for t, tag in zip(ts, tags)]
    for it in range(25):
        print(f"[case] compress_many repeat {it}", flush=True)
        res = ck.compress_many(encs, srcs)
        torch.cuda.synchronize()
        for k, (r, ref) in enumerate(zip(res, refs)):
            assert r.total == ref.numel() and torch.equal(r.data[: r.total], ref), (it, k)


def test_compress_many_one_launch_for_many_jobs(gpu):
    """A shard of more small tensors than one encode launch takes (22 bf16 of
    sizes from 1 element to 3 MiB, 4 fp32): the encodes of each kind go in
    launches of at most 16 jobs, workgroups shared in proportion to the jobs'
    units; every tensor's bytes, headers and offsets equal one ckr_compress of
    it, twice in a row."""
    import torch
    ck = _ck()
    g = torch.Generator(device=gpu).manual_seed(83)
    sizes = [1, 7, 4096, 32768, 32769, 100_000, 1 << 20, 1_500_001] + [(k * 97_531) % 1_600_000 + 1 for k in range(14)]
    ts = [(torch.randn(n, device=gpu, generator=g) * 0.02).to(torch.bfloat16) for n in sizes]
    ts += [torch.randn(n, device=gpu, generator=g) * 1e-3 for n in (3, 65536, 700_001, 250_000)]
    tags = [ck.torch_tag(t.dtype) for t in ts]
    srcs = [t.view(torch.uint8) for t in ts]
    refs = []
    for t, tag, s in zip(ts, tags, srcs):
        e = ck.Encoder(t.numel(), tag, 65536, device=gpu).compress(s)
        torch.cuda.synchronize()
        refs.append((e.total, e.data[: e.total].clone(), e.headers.clone(), e.unit_offsets.clone(), e.table.norm.copy()))
    encs = [ck.Encoder(t.numel(), tag, 65536, device=gpu) for t, tag in zip(ts, tags)]
    for it in range(2):
        print(f"[case] compress_many {len(ts)} jobs, call {it}", flush=True)
        res = ck.compress_many(encs, srcs)
        torch.cuda.synchronize()
        for k, (r, (tot, data, hdr, off, norm)) in enumerate(zip(res, refs)):
            assert r.total == tot and torch.equal(r.data[: r.total], data), (it, k)
            assert torch.equal(r.headers, hdr) and torch.equal(r.unit_offsets, off), (it, k)
            assert np.array_equal(r.table.norm, norm), (it, k)


def test_compress_many_large_overlapped_histogram(gpu):
    """A tensor above the 256 MiB bound under which compress_many counts every
    histogram first, so that its histogram runs beside the previous encode (8
    KiB of LDS, one workgroup per CU) and covers it in several strides per
    thread: compress_many still gives exactly what ckr_compress gives."""
    import torch
    ck = _ck()
    unit = 65536
    g = torch.Generator(device=gpu).manual_seed(80)
    a = (torch.randn(3_000_001, device=gpu, generator=g) * 0.02).to(torch.bfloat16)
    b = torch.randn(70_000_000 + 7, device=gpu, generator=g) * 1e-3
    c = (torch.randn(5_000_011, device=gpu, generator=g) * 0.02).to(torch.bfloat16)
    srcs = [a.view(torch.uint8), b.view(torch.uint8), c.view(torch.uint8)]
    specs = [(dg.BF16, a.numel()), (dg.F32, b.numel()), (dg.BF16, c.numel())]
    print("[case] compress_many large overlapped histogram", flush=True)
    many = ck.compress_many([ck.Encoder(n, dt, unit, device=gpu) for dt, n in specs], srcs)
    one = [ck.Encoder(n, dt, unit, device=gpu).compress(t) for (dt, n), t in zip(specs, srcs)]
    torch.cuda.synchronize()
    for m, o in zip(many, one):
        assert np.array_equal(m.table.norm, o.table.norm)
        assert m.total == o.total
        assert np.array_equal(m.data_np(), o.data_np())
        assert np.array_equal(m.headers_np(), o.headers_np())
        assert torch.equal(m.unit_offsets, o.unit_offsets)
        assert torch.equal(m.sidecar, o.sidecar)


def test_cfg3_size_tensors_through_compress_many(gpu):
    """One bf16 and one fp32 tensor of cfg3's shape (1,003,782,656 elements,
    the Llama-3-8B ZeRO-3 rank-0-of-8 share; 6 GB) through ckr_compress_many,
    at a size the oracle cannot code in seconds.  Checked by what holds at any
    size: the table equals the oracle's normalize_histogram of a histogram
    torch counts independently (the zero planes counted in closed form), the
    sidecar equals the input's low bytes, unit offsets are monotone and end at
    the total, and the decode is bit-exact with every lane's postconditions met."""
    import torch
    ck = _ck()
    n, unit = 1_003_782_656, 65536
    g = torch.Generator(device=gpu).manual_seed(90)
    tensors = [(dg.BF16, (torch.randn(n, device=gpu, generator=g) * 0.02).to(torch.bfloat16)),
               (dg.F32, torch.randn(n, device=gpu, generator=g) * 1e-3)]
    print("[case] cfg3-size bf16 + fp32 through compress_many", flush=True)
    encs = [ck.Encoder(n, dt, unit, device=gpu) for dt, _ in tensors]
    res = ck.compress_many(encs, [t.view(torch.uint8) for _, t in tensors])
    torch.cuda.synchronize()
    for (dt, t), r in zip(tensors, res):
        es, spe = oc.ES[dt], oc.SPE[dt]
        by = t.view(torch.uint8).view(n, es)
        hist = torch.bincount(by[:, spe:].reshape(-1), minlength=256).cpu().numpy().astype(np.uint64)
        hist[0] += n * spe
        assert int(hist.max()) < (1 << 32)  # no u32 wrap at this size
        want, tsum = oc.normalize_histogram(hist.astype(np.uint32))
        assert tsum == 4096 and np.array_equal(r.table.norm, want["norm_freq"])
        assert torch.equal(r.sidecar[: n * spe].view(n, spe), by[:, :spe])
        uo = r.unit_offsets
        assert int(uo[0]) == 0 and int(uo[-1]) == r.total and bool((uo[1:] >= uo[:-1]).all())
        dst, bad = ck.decode(r)
        torch.cuda.synchronize()
        assert bad == 0 and torch.equal(dst, t.view(torch.uint8))
        del dst


@pytest.mark.parametrize("dt,shift", [(dg.F32, 4), (dg.F32, 12), (dg.BF16, 2), (dg.BF16, 6), (dg.BF16, 8),
                                      (dg.F16, 14), (dg.I8, 1), (dg.I8, 3)])
@pytest.mark.parametrize("unit", [65536, 1 << 20])
def test_element_aligned_sources_and_destinations(dt, shift, unit, paths, gpu):
    """A tensor that starts `shift` bytes into its allocation (a slice of a flat
    buffer at an element offset that is not a multiple of 16 bytes): histogram,
    compress, compress_many and decode into an equally shifted destination give
    the oracle's bytes and the original bits."""
    import torch
    ck = _ck()
    n = 300_007
    gen = {dg.F32: lambda: dg.normal_f32(n, 1e-3, 90), dg.BF16: lambda: dg.normal_bf16(n, 0.02, 91),
           dg.F16: lambda: (np.random.default_rng(92).standard_normal(n) * 0.02).astype(np.float16),
           dg.I8: lambda: np.random.default_rng(93).integers(-5, 5, n).astype(np.int8)}[dt]
    raw = gen()
    b = dg.raw_bytes(raw)
    print(f"[case] element-aligned dt={dt} shift={shift} unit={unit} fast={paths}", flush=True)
    buf = torch.zeros(b.size + 64, dtype=torch.uint8, device=gpu)
    buf[shift:shift + b.size].copy_(torch.from_numpy(b.copy()))
    src = buf[shift:shift + b.size]
    assert src.data_ptr() % 16 == shift % 16
    ref = oc.compress_tensor(raw, n, dt, unit)
    h = ck.byte_histogram(src, dt, n_elems=n)
    assert np.array_equal(h.cpu().numpy().view(np.uint32), oc.byte_hist(ref["masked"]))
    one = ck.compress(src, dt, unit, n_elems=n)
    many = ck.compress_many([ck.Encoder(n, dt, unit, device=gpu), ck.Encoder(n, dt, unit, device=gpu)], [src, src])
    torch.cuda.synchronize()
    for e in [one] + many:
        assert np.array_equal(e.table.norm, ref["table"]["norm_freq"])
        assert e.total == ref["data"].size and np.array_equal(e.data_np(), ref["data"])
        nu = ref["unit_offsets"].size - 1
        assert np.array_equal(e.headers_np()[: nu * 256], ref["headers"])
        if oc.SPE[dt]:
            assert np.array_equal(e.sidecar[: n * oc.SPE[dt]].cpu().numpy(), ref["sidecar"])
    out = torch.full((b.size + 64,), 0xA5, dtype=torch.uint8, device=gpu)
    dst, bad = ck.decode(one, dst=out[shift:shift + b.size])
    torch.cuda.synchronize()
    assert bad == 0 and np.array_equal(dst.cpu().numpy(), b)
    o = out.cpu().numpy()
    assert (o[:shift] == 0xA5).all() and (o[shift + b.size:] == 0xA5).all()  # nothing written outside



def test_invalid_device_pointers_are_errors(gpu):
    """Host memory, freed device memory and ranges that run past their
    allocation are rejected on the host before any launch (the reference checks
    each pointer with hipPointerGetAttributes, src/ANSCompressor.cpp:567-585):
    hipPointerGetAttributes reports unregistered memory for the first two, and
    hipMemGetAddressRange bounds the third."""
    import ctypes
    import torch
    ck = _ck()
    hip = ctypes.CDLL("libamdhip64.so")
    n = 4096
    enc = ck.Encoder(n, ck.F32, 65536, device=gpu)
    hist = torch.zeros(256, dtype=torch.int32, device=gpu)

    def compress_from(p, nbytes_elems=n):
        return ck.lib().ckr_compress(ctypes.c_void_p(p), nbytes_elems, ck.F32, 65536, 0, enc.out.data_ptr(),
                                     enc.out_cap, enc.headers.data_ptr(), enc.unit_offsets.data_ptr(),
                                     enc.sidecar.data_ptr(), enc.ws.data_ptr(), enc.ws_bytes, None, None, None)

    host = np.zeros(n, np.float32)
    assert compress_from(host.ctypes.data) == ck.CKR_E_INVALID
    assert b"device-accessible" in ck.lib().ckr_last_error()
    d = ctypes.c_void_p()
    assert hip.hipMalloc(ctypes.byref(d), ctypes.c_size_t(1 << 20)) == 0
    try:
        # the last 4 KiB of a 1 MiB allocation, read as 16 KiB
        assert compress_from(d.value + (1 << 20) - 4096) == ck.CKR_E_INVALID
        assert b"past its allocation" in ck.lib().ckr_last_error()
        assert ck.lib().ckr_byte_histogram(ctypes.c_void_p(d.value + 4096), 1 << 20, ck.I8, hist.data_ptr(),
                                           None) == ck.CKR_E_INVALID
    finally:
        assert hip.hipFree(d) == 0
    assert compress_from(d.value) == ck.CKR_E_INVALID  # freed
    assert ck.lib().ckr_byte_histogram(d, 4096, ck.I8, hist.data_ptr(), None) == ck.CKR_E_INVALID
    # a valid call afterwards still works (no error left behind by the queries)
    t = torch.randn(n, device=gpu) * 1e-3
    e = enc.compress(t.view(torch.uint8))
    dst, bad = ck.decode(e)
    torch.cuda.synchronize()
    assert bad == 0 and torch.equal(dst, t.view(torch.uint8))


def test_batched_calls_refuse_overlapping_outputs(gpu):
    """ckr_compress_many and ckr_decode_many run jobs on several streams at
    once: an output range of one job that overlaps another output (headers
    inside another job's headers, a destination inside another's) is refused
    before anything is queued."""
    import torch
    ck = _ck()
    a = torch.randn(200_000, device=gpu) * 1e-3
    b = torch.randn(50_000, device=gpu) * 1e-3
    ea, eb = ck.Encoder(a.numel(), ck.F32, 65536, device=gpu), ck.Encoder(b.numel(), ck.F32, 65536, device=gpu)
    eb.headers = ea.headers[1024:]          # job 1's headers start at job 0's unit 1
    with pytest.raises(ck.CkrError) as e:
        ck.compress_many([ea, eb], [a.view(torch.uint8), b.view(torch.uint8)])
    assert e.value.code == ck.CKR_E_INVALID and "overlaps" in str(e.value)
    eb = ck.Encoder(b.numel(), ck.F32, 65536, device=gpu)
    ra, rb = ck.compress_many([ea, eb], [a.view(torch.uint8), b.view(torch.uint8)])
    da, db = ck.Decoder(a.numel(), ck.F32, 65536, device=gpu), ck.Decoder(b.numel(), ck.F32, 65536, device=gpu)
    dst = torch.zeros(a.numel() * 4, dtype=torch.uint8, device=gpu)
    with pytest.raises(ck.CkrError) as e:
        ck.decode_many([da, db], [ra, rb], [dst, dst[4096:4096 + b.numel() * 4]])
    assert e.value.code == ck.CKR_E_INVALID and "overlaps" in str(e.value)
    db2 = torch.zeros(b.numel() * 4, dtype=torch.uint8, device=gpu)
    assert ck.decode_many([da, db], [ra, rb], [dst, db2]) == [0, 0]
    torch.cuda.synchronize()
    assert torch.equal(dst, a.view(torch.uint8)) and torch.equal(db2, b.view(torch.uint8))
