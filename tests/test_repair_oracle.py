"""Pins the oracle's prefix-mask repair (Re-Pair over masked words).

The reference's CLI, compiled from its own sources (oracle/_ref), wrote the
golden reports under tests/golden/repair/; the oracle must reproduce every
count in them.  The tie-break model the GPU path uses (pair with the largest
count; among equal counts the one std::unordered_map visits first: buckets in
reverse order of their first insertion, within a bucket the latest inserted
first) is checked against the oracle's real std::unordered_map on sequences
built to have many ties, and against hand-worked cases.
"""
import numpy as np
import pytest

import oracle as oc
from tests import repair_fixtures as rf

MB = 1024.0 * 1024.0


@pytest.mark.parametrize("name", rf.cases())
def test_oracle_matches_reference_reports(name):
    case = rf.load_case(name)
    build = lambda raw, n, es, k, mr: oc.repair_build(raw, n, es, k, mr)
    apply_ = lambda raw, n, es, k, rules: oc.repair_apply(raw, n, es, k, rules)
    got_t, got_g = rf.evaluate(case, build, apply_)
    hdr, rows = case["tensor_rows"]
    assert len(rows) == len(got_t)
    col = {h: i for i, h in enumerate(hdr)}
    for r, g in zip(rows, got_t):
        assert int(r[col["layer"]]) == g["layer"]
        assert int(r[col["compressed_token_count"]]) == g["tokens"]
        assert int(r[col["rule_count"]]) == g["rules"]
        assert int(r[col["masked_mantissa_bits"]]) == g["masked_bits"]
        for c, v in (("cfg_payload_size_mb", g["payload"]), ("grammar_size_mb_charged", g["grammar"]),
                     ("residual_raw_size_mb", g["residual"]), ("masked_only_size_mb", g["masked_only"]),
                     ("original_size_mb", g["original"]),
                     ("lossy_compressed_size_mb", g["payload"] + g["grammar"])):
            assert float(r[col[c]]) == pytest.approx(v / MB, rel=1e-5, abs=0), (c, r)
    ghdr, grows = case["group_rows"]
    gcol = {h: i for i, h in enumerate(ghdr)}
    assert len(grows) == len(got_g)
    for r, g in zip(grows, got_g):
        assert int(r[gcol["rule_count"]]) == g["rules"]
        assert int(r[gcol["max_pair_frequency"]]) == g["max_pair"]
        assert float(r[gcol["grammar_size_mb"]]) == pytest.approx(g["grammar"] / MB, rel=1e-5, abs=0)


def pair_hash(l, r):
    m = (1 << 64) - 1
    return (l ^ ((r + 0x9E3779B97F4A7C15 + ((l << 6) & m) + (l >> 2)) & m)) & m


def model_build(words, max_rules):
    """Re-Pair with the tie-break written out as the GPU path computes it."""
    t = [int(w) for w in words]
    rules, maxf, nxt = [], 0, 1 << 63
    for _ in range(max_rules):
        if len(t) < 2:
            break
        P = oc.repair_bucket_count(len(t))
        cnt, first = {}, {}
        for i in range(len(t) - 1):
            k = (t[i], t[i + 1])
            cnt[k] = cnt.get(k, 0) + 1
            first.setdefault(k, i)
        bfirst = {}
        for k, f in first.items():
            b = pair_hash(*k) % P
            bfirst[b] = min(bfirst.get(b, f), f)
        best = max(cnt.values())
        maxf = max(maxf, best)
        if best < 2:
            break
        cands = [k for k in cnt if cnt[k] == best]
        k = max(cands, key=lambda k: (bfirst[pair_hash(*k) % P], first[k]))
        out, i = [], 0
        while i < len(t):
            if i + 1 < len(t) and (t[i], t[i + 1]) == k:
                out.append(nxt)
                i += 2
            else:
                out.append(t[i])
                i += 1
        rules.append((nxt, k[0], k[1], best))
        nxt += 1
        t = out
    return rules, len(t), maxf


@pytest.mark.parametrize("seed", range(40))
def test_tie_order_model_matches_unordered_map(seed):
    rng = np.random.default_rng(seed)
    n = int(rng.integers(2, 400))
    alpha = int(rng.integers(1, 9))
    vals = rng.integers(0, 1 << 16, alpha).astype(np.uint16)
    if seed % 3 == 0:   # periodic: every pair of the period ties
        per = vals[rng.integers(0, alpha, int(rng.integers(2, 7)))]
        w = np.tile(per, n // per.size + 1)[:n]
    else:
        w = vals[rng.integers(0, alpha, n)]
    ref = oc.repair_build(w, n, 2, 0, 50)
    rules, out_len, maxf = model_build(w, 50)
    assert ref["rules"] == rules and ref["out_len"] == out_len and ref["max_pair"] == maxf


def test_bucket_collision_decides_tie():
    # two pairs with equal counts whose buckets coincide: the one whose bucket
    # was created first is visited last, unless another pair created it earlier
    n = 64
    P = oc.repair_bucket_count(n)
    base = [0x1111, 0x2222]
    found = None
    for a in range(1, 4000):
        for b in (0x5555, 0x6666):
            if pair_hash(a << 4, b) % P == pair_hash(0x7770, 0x8880) % P and (a << 4, b) != (0x7770, 0x8880):
                found = (a << 4, b)
                break
        if found:
            break
    assert found
    seq = [0x7770, 0x8880, 0x9990, found[0], found[1], 0x9990] * 2
    seq += [0x9990 + 16 * i for i in range(1, n - len(seq) + 1)]
    w = np.array(seq, np.uint16)
    ref = oc.repair_build(w, w.size, 2, 0, 1)
    rules, _, _ = model_build(w, 1)
    assert ref["rules"] == rules


def test_hand_worked_runs_and_stop():
    # "aaaa" -> counts (a,a)=3 -> greedy left to right gives [X, X]; then (X,X)=1 stops
    w = np.array([5, 5, 5, 5], np.uint16)
    r = oc.repair_build(w, 4, 2, 0, 50)
    assert r["rules"] == [(1 << 63, 5, 5, 3)] and r["out_len"] == 2 and r["max_pair"] == 3
    # odd run: "aaa" -> [X, a]
    r = oc.repair_build(np.array([5, 5, 5], np.uint16), 3, 2, 0, 50)
    assert r["out_len"] == 2 and len(r["rules"]) == 1
    # all pairs distinct: no rule, max pair frequency 1
    r = oc.repair_build(np.array([1, 2, 3, 4], np.uint16), 4, 2, 0, 50)
    assert r["rules"] == [] and r["out_len"] == 4 and r["max_pair"] == 1
    # one element: no pair counted at all
    r = oc.repair_build(np.array([1], np.uint16), 1, 2, 0, 50)
    assert r["rules"] == [] and r["out_len"] == 1 and r["max_pair"] == 0
    # masking: 0x3C01 and 0x3C02 become equal with 2 masked bits
    r = oc.repair_build(np.array([0x3C01, 0x3C02, 0x3C01, 0x3C02], np.uint16), 4, 2, 2, 50)
    assert r["rules"][0][1:3] == (0x3C00, 0x3C00)
    # (1,2)x4 -> X; (X,X)x3 -> Y giving [Y, Y]; (Y,Y)x1 stops.  Rules apply in
    # order to another sequence, the second one nesting the first
    r = oc.repair_build(np.array([1, 2, 1, 2, 1, 2, 1, 2], np.uint16), 8, 2, 0, 50)
    X, Y = 1 << 63, (1 << 63) + 1
    assert r["rules"] == [(X, 1, 2, 4), (Y, X, X, 3)] and r["out_len"] == 2 and r["max_pair"] == 4
    assert oc.repair_apply(np.array([1, 2, 1, 2, 9], np.uint16), 5, 2, 0, r["rules"]) == 2
