"""Pins for the CPU oracle (oracle/ckr_oracle.cpp) — CPU only.

The reference has no tests, fixtures or golden vectors for this path, so each
oracle function is pinned by what the mathematics fixes: closed forms and
hand-derived known answers, brute force with independent numpy arithmetic,
and invariants chosen so a plausible slip (wrong threshold, sign, index or
rounding direction) fails one of them.
"""
import numpy as np
import pytest

import oracle as oc
from tests import datagen as dg

M = 4096
L = 1 << 23


# ---------------------------------------------------------------- byte-plane split
@pytest.mark.parametrize("n", [1, 2, 3, 17, 1000])
def test_extract_mantissa_closed_form(n):
    # fp32: masked keeps the top 16 bits, sidecar holds the low 16 bits in element order
    x = dg.normal_f32(n, 1e-3, n)
    m, s = oc.extract_mantissa(x, n, dg.F32)
    u = x.view(np.uint32)
    assert np.array_equal(m.view(np.uint32), u & np.uint32(0xFFFF0000))
    assert np.array_equal(s.view(np.uint16), (u & 0xFFFF).astype(np.uint16))
    # bf16 / fp16: low byte to the sidecar
    for dt in (dg.BF16, dg.F16):
        b = dg.normal_bf16(n, 0.02, n + 1)
        m, s = oc.extract_mantissa(b, n, dt)
        assert np.array_equal(m.view(np.uint16), b & np.uint16(0xFF00))
        assert np.array_equal(s, (b & 0xFF).astype(np.uint8))
        assert np.array_equal(oc.merge_sidecar(m, s, n, dt).view(np.uint16), b)
    # no sidecar for int dtypes: the masked stream is the raw bytes
    i8 = np.arange(n, dtype=np.int64).astype(np.int8)
    m, s = oc.extract_mantissa(i8, n, dg.I8)
    assert s.size == 0 and np.array_equal(m, i8.view(np.uint8))


def test_byte_hist_brute_force():
    d = np.random.default_rng(1).integers(0, 256, 100_003).astype(np.uint8)
    assert np.array_equal(oc.byte_hist(d), np.bincount(d, minlength=256).astype(np.uint32))


# ---------------------------------------------------------------- table
def test_table_single_symbol():
    h = np.zeros(256, np.uint32)
    h[77] = 12345
    t, s = oc.normalize_histogram(h)
    assert s == M and t["norm_freq"][77] == M and t["norm_freq"].sum() == M
    assert t["cum_freq"][77] == 0 and t["cum_freq"][78] == M
    assert t["x_max"][77] == (1 << 19) * M
    assert (t["decode_sym"] == 77).all()


def test_table_two_equal_symbols():
    h = np.zeros(256, np.uint32)
    h[0] = h[1] = 5
    t, s = oc.normalize_histogram(h)
    assert s == M and t["norm_freq"][0] == 2048 and t["norm_freq"][1] == 2048
    assert t["cum_freq"][1] == 2048 and t["cum_freq"][2] == M


def test_table_empty_histogram():
    t, s = oc.normalize_histogram(np.zeros(256, np.uint32))
    assert s == M and t["norm_freq"][0] == M and (t["cum_freq"][1:] == M).all()
    assert t["x_max"][0] == (1 << 19) * M and (t["decode_freq"] == M).all()


def _py_table(h, full):
    """The normalisation steps with Python's stable sort — identical to the
    reference whenever no two fractional parts are equal (no ties to break)."""
    total = int(h.sum())
    norm = np.zeros(256, np.int64)
    for i in range(256):
        if not full and h[i] == 0:
            continue
        norm[i] = max(1, max(int(h[i]), 1) * M // total)
    fr = [(i, max(int(h[i]), 1) * M / total) for i in range(256) if norm[i]]
    fr = [(i, e - int(e)) for i, e in fr]
    fracs = [f for _, f in fr]
    fr.sort(key=lambda t: -t[1])
    a = int(norm.sum())
    if a < M:
        for k in range(min(M - a, len(fr))):
            norm[fr[k][0]] += 1
    elif a > M:
        rem = a - M
        for k in range(len(fr) - 1, -1, -1):
            if rem and norm[fr[k][0]] > 1:
                norm[fr[k][0]] -= 1
                rem -= 1
    return norm, len(set(fracs)) == len(fracs)


@pytest.mark.parametrize("seed", range(20))
def test_table_matches_untied_restatement_and_bounds(seed):
    rng = np.random.default_rng(seed)
    h = np.zeros(256, np.uint32)
    k = int(rng.integers(2, 200))
    idx = rng.choice(256, k, replace=False)
    h[idx] = rng.integers(1000, 10**7, k)
    t, s = oc.normalize_histogram(h)
    norm = t["norm_freq"].astype(np.int64)
    assert s == M == norm.sum()
    exact = h.astype(np.float64) * M / h.sum()
    present = h > 0
    assert (norm[~present] == 0).all() and (norm[present] >= 1).all()
    assert (np.abs(norm[present] - np.maximum(exact[present], 1)) < 2).all()
    if exact[present].min() >= 1:  # no slot was rounded up to the minimum: only +1 corrections
        fl = np.floor(exact[present])
        assert ((norm[present] == fl) | (norm[present] == fl + 1)).all()
    ref, untied = _py_table(h, False)
    if untied:
        assert np.array_equal(norm, ref)
    # derived arrays
    assert np.array_equal(t["cum_freq"], np.concatenate([[0], np.cumsum(norm)]).astype(np.uint32))
    assert np.array_equal(t["x_max"], (norm << 19).astype(np.uint32))
    slots = np.repeat(np.arange(256), norm)
    assert np.array_equal(t["decode_sym"], slots.astype(np.uint8))


def test_table_one_pass_decrement_defect():
    # 255 symbols seen once and one seen 10^6 times: step 1 assigns 255 + 4094
    # slots; the single decrement pass can only take one slot (from the only
    # symbol above 1), so the table sums to 4348, as the reference's code does.
    h = np.ones(256, np.uint32)
    h[0] = 1_000_000
    t, s = oc.normalize_histogram(h)
    assert s == 255 + 4094 - 1 == 4348
    # full-alphabet mode on masked bf16 N(0,0.02): sum 4316 (the survey's scratch number)
    x = dg.normal_bf16(1 << 20, 0.02, 0)
    m, _ = oc.extract_mantissa(x, x.size, dg.BF16)
    t, s = oc.normalize_histogram(oc.byte_hist(m), ensure_full_alphabet=True)
    assert s > M


# ---------------------------------------------------------------- rANS
def _two_symbol_table():
    h = np.zeros(256, np.uint32)
    h[0] = h[1] = 1
    t, _ = oc.normalize_histogram(h)
    return t


def test_rans_all_zero_known_answer():
    # one symbol, f = 4096: the state never changes and nothing is emitted
    z = np.zeros(4096 * 4, np.uint8)
    t, _ = oc.normalize_histogram(oc.byte_hist(z))
    data, hdr, off = oc.encode(z, t, 0)
    assert data.size == 0 and (hdr["final_state"] == L).all() and (hdr["byte_count"] == 0).all()


def test_rans_hand_derived_renorm():
    # f(0) = 2048: coding a 0 maps x -> 2x - x % 2048; from 2^23 seven zeros give
    # 2^30 = x_max(0) = 2^19 * 2048, so the eighth emits the low byte (0x00) and
    # continues from 2^22 -> 2^23.  A unit of 8 rows of zeros: every lane emits
    # exactly one 0x00 byte and ends in 2^23.
    t = _two_symbol_table()
    data, hdr, off = oc.encode(np.zeros(8 * 256, np.uint8), t, 0)
    assert data.size == 256 and (data == 0).all()
    assert (hdr["final_state"] == L).all() and (hdr["byte_count"] == 1).all()
    assert np.array_equal(hdr["buf_offset"], np.arange(256, dtype=np.uint32))
    # one more zero per lane (9 rows): after the eighth the state is 2^23, the
    # ninth doubles it
    data, hdr, _ = oc.encode(np.zeros(9 * 256, np.uint8), t, 0)
    assert data.size == 256 and (hdr["final_state"] == 2 * L).all()
    # a single symbol 1 (cum 2048) per lane: x = 2*2^23 - 0 + 2048
    d1 = np.ones(256, np.uint8)
    _, hdr, _ = oc.encode(d1, t, 0)
    assert (hdr["final_state"] == 2 * L + 2048).all()


def _encode_decode(masked, table, unit):
    data, hdr, off = oc.encode(masked, table, unit)
    back, bad = oc.decode(data, hdr, off, table, masked.size, unit)
    return data, hdr, off, back, bad


@pytest.mark.parametrize("unit", [0, 256, 1024, 65536])
def test_rans_roundtrip_and_entropy(unit):
    x = dg.normal_f32(50_000, 1e-3, 3)
    m, _ = oc.extract_mantissa(x, x.size, dg.F32)
    h = oc.byte_hist(m)
    t, _ = oc.normalize_histogram(h)
    data, hdr, off, back, bad = _encode_decode(m, t, unit)
    assert bad == 0 and np.array_equal(back, m)
    assert off[-1] == data.size and (np.diff(off.astype(np.int64)) >= 0).all()
    # coded size vs the table's cost of the data: rANS is within the final
    # states (4 bytes per lane, carried in headers) of sum(-log2(f/M)) / 8
    f = t["norm_freq"].astype(np.float64)
    cost = float((h * np.log2(M / np.where(f > 0, f, 1))).sum() / 8)
    nu = oc.num_units(m.size, unit)
    assert cost - 4 * 256 * nu - 64 <= data.size <= cost + 256 * nu + 64


def test_rans_units_are_independent_encodes():
    # unit-chunked coding == each chunk coded alone (same table), concatenated
    x = dg.normal_bf16(3 * 32768 + 5, 0.02, 4)
    m, _ = oc.extract_mantissa(x, x.size, dg.BF16)
    t, _ = oc.normalize_histogram(oc.byte_hist(m))
    U = 65536
    data, hdr, off = oc.encode(m, t, U)
    for u in range(off.size - 1):
        d_u, h_u, o_u = oc.encode(m[u * U:(u + 1) * U], t, 0)
        assert np.array_equal(data[off[u]:off[u + 1]], d_u)
        assert np.array_equal(hdr[u * 256:(u + 1) * 256], h_u)


def test_rans_passthrough_unit():
    # a table that gives the data's symbols 3-4 slots makes random units expand
    rng = np.random.default_rng(5)
    d = rng.integers(0, 256, 8192).astype(np.uint8)
    d[:2048] = 0
    h = np.full(256, 100, np.uint32)
    h[0] = 100_000
    t, s = oc.normalize_histogram(h)
    assert s == M
    data, hdr, off, back, bad = _encode_decode(d, t, 1024)
    sizes = np.diff(off.astype(np.int64))
    raw = sizes == 1024
    assert raw.any() and (~raw).any()
    for u in np.nonzero(raw)[0]:
        hu = hdr[u * 256:(u + 1) * 256]
        assert hu["byte_count"][0] == 1024 and (hu["byte_count"][1:] == 0).all()
        assert np.array_equal(data[off[u]:off[u + 1]], d[u * 1024:(u + 1) * 1024])
    assert bad == 0 and np.array_equal(back, d)


def test_rans_escape_emits_raw_byte():
    # f(5) == 0: the reference writes the raw symbol and leaves the state alone
    h = np.zeros(256, np.uint32)
    h[0] = 1
    t, _ = oc.normalize_histogram(h)  # only symbol 0, f = 4096
    d = np.zeros(256, np.uint8)
    d[3] = 5
    data, hdr, _ = oc.encode(d, t, 0)
    assert data.tolist() == [5] and hdr["byte_count"][3] == 1 and (hdr["final_state"] == L).all()


# ---------------------------------------------------------------- analyzer
def _np_hist(x, bins):
    b = min(bins, 256)
    f = x.astype(np.float32)
    lo = np.float32(min(np.float32(1e37), np.nanmin(f)))
    hi = np.float32(max(np.float32(-1e37), np.nanmax(f)))
    rng_ = np.float32(hi - lo)
    h = np.zeros(b, np.uint32)
    if rng_ > np.float32(1e-9):
        scale = np.float32(np.float32(b) - np.float32(1.0)) / rng_
        t = (f - lo) * scale  # float32 ops, correctly rounded
        idx = np.where(np.isnan(t), 0, np.clip(t, -2**31, 2**31 - 1)).astype(np.int64)
        idx = np.clip(idx, 0, b - 1)
        np.add.at(h, idx, 1)
    else:
        h[0] = f.size
    return h, lo, hi


@pytest.mark.parametrize("dt,n,bins", [(dg.F32, 100_001, 256), (dg.F32, 5000, 16), (dg.BF16, 30_000, 4096),
                                       (dg.F16, 3001, 100), (dg.I8, 4000, 256), (dg.I32, 777, 7)])
def test_stats_histogram_minmax_moments(dt, n, bins):
    rng = np.random.default_rng(n)
    if dt == dg.F32:
        raw = dg.normal_f32(n, 1e-3, n)
        vals = raw.astype(np.float64)
    elif dt == dg.BF16:
        raw = dg.normal_bf16(n, 0.02, n)
        vals = (raw.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    elif dt == dg.F16:
        raw = rng.standard_normal(n).astype(np.float16)
        vals = raw.astype(np.float64)
    elif dt == dg.I8:
        raw = rng.integers(-128, 128, n).astype(np.int8)
        vals = raw.astype(np.float64)
    else:
        raw = rng.integers(-10**6, 10**6, n).astype(np.int32)
        vals = raw.astype(np.float32).astype(np.float64)
    r = oc.tensor_stats(raw, n, dt, bins)
    h, lo, hi = _np_hist(vals.astype(np.float32), bins)
    assert r["minmax"][0] == lo and r["minmax"][1] == hi
    assert np.array_equal(r["histogram"], h)
    mu = vals.mean()
    c = vals - mu
    var = (c ** 2).mean()
    m64 = r["moments64"]
    assert np.isclose(m64[0], mu, rtol=1e-12, atol=1e-15)
    assert np.isclose(m64[1], var, rtol=1e-10)
    assert np.isclose(m64[2], (c ** 3).mean() / var ** 1.5, rtol=1e-8, atol=1e-10)
    assert np.isclose(m64[3], (c ** 4).mean() / var ** 2, rtol=1e-8)
    # the fp32 reference-order values track the fp64 ones
    assert abs(r["moments"][0] - mu) <= 1e-5 * (hi - lo) + 1e-12
    assert np.isclose(r["moments"][1], var, rtol=1e-3)


def test_stats_normal_sanity_and_constant():
    x = dg.normal_f32(1 << 18, 0.5, 9)
    r = oc.tensor_stats(x, x.size, dg.F32, 256)
    mean, var, skew, kurt = r["moments"]
    assert abs(mean) < 0.01 and abs(var - 0.25) < 0.005 and abs(skew) < 0.02 and abs(kurt - 3) < 0.05
    c = np.full(100, 3.0, np.float32)
    r = oc.tensor_stats(c, 100, dg.F32, 256)
    assert r["histogram"][0] == 100 and r["histogram"][1:].sum() == 0
    assert r["moments"][1] == 0 and r["moments"][2] == 0 and r["moments"][3] == 0


def test_stats_initial_bounds_quirk():
    # min starts at 1e37 and max at -1e37 (TensorAnalyzer.cpp:86-87): a tensor of
    # +inf reports min 1e37
    x = np.full(10, np.inf, np.float32)
    r = oc.tensor_stats(x, 10, dg.F32, 256)
    assert r["minmax"][0] == np.float32(1e37) and np.isinf(r["minmax"][1])


def test_threaded_split_and_histogram_equal_single_thread():
    """The CPU baseline's threaded split and histogram give the single-thread
    functions' bytes and counts (fp32, bf16, int8; a length that splits unevenly)."""
    for dt, gen in ((dg.F32, lambda n: dg.normal_f32(n, 1e-3, 5)), (dg.BF16, lambda n: dg.normal_bf16(n, 0.02, 6)),
                    (dg.I8, lambda n: np.random.default_rng(7).integers(-128, 128, n).astype(np.int8))):
        n = 300_007
        raw = gen(n)
        m1, s1 = oc.extract_mantissa(raw, n, dt)
        m8, s8 = oc.extract_mantissa(raw, n, dt, n_threads=8)
        assert np.array_equal(m1, m8) and np.array_equal(s1, s8)
        assert np.array_equal(oc.byte_hist(m1), oc.byte_hist(m1, n_threads=8))
