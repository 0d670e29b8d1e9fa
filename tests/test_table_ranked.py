"""The table by ranks (ckr_build_table_ranked, the device table's arithmetic
run on the host) against ckr_build_table, which sorts with libstdc++'s
std::sort as the reference's normalize_histogram does
(src/ANSCompressor.cpp:416-503): on 10^5 histograms, random and tie-heavy,
with and without the full alphabet, every table not marked ambiguous equals
the sorted one bit for bit, and the ambiguous ones are exactly those whose
correction boundary cuts a group of equal fractional parts."""
import numpy as np
import pytest

import checkers_amd as ck

M = 4096


def histograms(seed, n):
    """n histograms of 256 words from seven families (seeded)."""
    rng = np.random.default_rng(seed)
    out = np.zeros((n, 256), np.uint32)
    for i in range(n):
        k = i % 7
        if k == 0:    # random counts, some symbols absent
            h = rng.integers(0, 1000, 256)
            h[rng.random(256) < 0.3] = 0
        elif k == 1:  # tie-heavy: counts from a small set
            h = rng.choice([0, 1, 2, 3, 5, 8, 13], 256)
        elif k == 2:  # a sampled peaked distribution (like an exponent byte)
            p = np.exp(-0.5 * ((np.arange(256) - rng.integers(0, 256)) / rng.uniform(1, 20)) ** 2)
            h = rng.multinomial(int(rng.integers(1, 10 ** 6)), p / p.sum())
        elif k == 3:  # a few symbols
            h = np.zeros(256, np.int64)
            h[rng.choice(256, int(rng.integers(1, 6)), replace=False)] = rng.integers(1, 5000, 1)[0]
        elif k == 4:  # large counts
            h = rng.integers(0, 2 ** 24, 256)
        elif k == 5:  # every symbol equal
            h = np.full(256, int(rng.integers(0, 100)))
        else:         # equal counts in groups of 2 to 5
            vals = rng.integers(1, 3000, 64)
            h = np.repeat(vals, 4)[:256]
            rng.shuffle(h)
            h[rng.random(256) < 0.2] = 0
        out[i] = h
    return out


def boundary_tie(h, ensure):
    """Whether the correction's boundary cuts a group of equal fractional
    parts (a direct statement of the ambiguity, for the check)."""
    h = np.asarray(h, np.uint64)
    total = int(h.sum())
    inc = np.ones(256, bool) if ensure else h > 0
    if not inc.any():
        return False
    hm = np.maximum(h, 1).astype(np.float64)
    norm = np.where(inc, np.maximum((np.maximum(h, 1) * M // total) if total else 0, 1), 0).astype(np.int64)
    exact = hm * M / float(total) if total else np.ones(256)
    frac = exact - np.trunc(exact)
    assigned = int(norm.sum())
    if assigned == M:
        return False
    if assigned < M:
        rem = M - assigned
        f = np.sort(frac[inc])[::-1]
    else:
        rem = assigned - M
        el = inc & (norm > 1)
        f = np.sort(frac[el])  # from the end of the descending order
    if rem <= 0 or rem >= f.size:
        return False
    return f[rem - 1] == f[rem]


@pytest.mark.parametrize("ensure", [False, True])
def test_ranked_tables_equal_sorted_tables(ensure):
    hs = histograms(7 + int(ensure), 50_000)
    n_amb = np.zeros(7, int)
    for i, h in enumerate(hs):
        ref, _ = ck.build_table(h, ensure)
        got, amb = ck.build_table_ranked(h, ensure)
        assert amb == boundary_tie(h, ensure), h
        if amb:
            n_amb[i % 7] += 1
            continue
        assert np.array_equal(got.norm, ref.norm), h
        assert got.raw_bytes() == ref.raw_bytes()
    # the tie-heavy families reach the ambiguous case; sampled distributions
    # (the tensors' kind) rarely do, large counts never here
    per = len(hs) // 7
    assert n_amb[1] > per // 2 and n_amb[6] > per // 4, n_amb
    assert n_amb[2] < per // 20 and n_amb[4] == 0, n_amb


def test_ranked_table_special_cases():
    # no symbol: every slot for symbol 0
    got, amb = ck.build_table_ranked(np.zeros(256, np.uint32), False)
    ref, _ = ck.build_table(np.zeros(256, np.uint32), False)
    assert not amb and np.array_equal(got.norm, ref.norm) and got.norm[0] == M
    # three equal counts, two of which must get the last two slots: ambiguous
    h = np.zeros(256, np.uint32)
    h[0], h[0x3F], h[0x40], h[0xBF] = 3000, 1000, 1000, 1000
    _, amb = ck.build_table_ranked(h, False)
    assert amb
