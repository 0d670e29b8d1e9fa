"""GPU parity of the prefix-mask repair (Re-Pair over masked words).

The HIP path (ckr_repair_build / ckr_repair_apply through the C ABI) must
reproduce the reference CLI's golden reports and, on every case, the oracle's
rules, compressed length, largest pair count and the compressed sequence
itself, symbol for symbol.  All integer: bit-exact.
"""
import numpy as np
import pytest

import oracle as oc
from tests import datagen as dg
from tests import repair_fixtures as rf

pytestmark = pytest.mark.gpu

TAG = {"float32": 0, "bfloat16": 1, "bf16": 1, "float16": 2, "fp16": 2}
ES = {0: 4, 1: 2, 2: 2}


def _ck():
    import checkers_amd as ck
    return ck


def _dev(raw, gpu):
    import torch
    raw = np.ascontiguousarray(raw).view(np.uint8).reshape(-1)
    t = torch.empty(max(raw.size, 16), dtype=torch.uint8, device=gpu)
    if raw.size:
        t[: raw.size].copy_(torch.from_numpy(raw.copy()))
    return t[: raw.size]


def _check_case(gpu, raw, dtype, masked, max_rules=50, other=None):
    """GPU build (and apply to `other`) against the oracle, sequences included."""
    ck = _ck()
    es = ES[dtype]
    raw = np.ascontiguousarray(raw).view(np.uint8).reshape(-1)
    if other is not None:
        other = np.ascontiguousarray(other).view(np.uint8).reshape(-1)
    n = raw.size // es
    k = ck.repair_masked_bits(dtype, masked)
    rp = ck.Repairer(max(n, 1) if other is None else max(n, other.size // es, 1), dtype, masked, max_rules)
    got = rp.build(_dev(raw, gpu), want_seq=True)
    ref = oc.repair_build(raw, n, es, k, max_rules, want_seq=True)
    assert got["rules"] == ref["rules"]
    assert got["out_len"] == ref["out_len"] and got["max_pair"] == ref["max_pair"]
    assert np.array_equal(got["seq"], ref["seq"])
    if other is not None:
        m = other.size // es
        g_len, g_seq = rp.apply(_dev(other, gpu), got["rules"], want_seq=True)
        r_len, r_seq = oc.repair_apply(other, m, es, k, ref["rules"], want_seq=True)
        assert g_len == r_len and np.array_equal(g_seq, r_seq)
    return got


@pytest.mark.parametrize("name", rf.cases())
def test_golden_reports(gpu, name):
    """Counts of the reference CLI's reports, computed through the GPU path."""
    ck = _ck()
    case = rf.load_case(name)
    got_t, got_g = [], []
    for g in case["groups"]:
        dt = TAG[case["manifest"][(g["state_type"], g["category"], g["rep"])]["dtype"]]

        def build(raw, n, es, k, mr, dt=dt):
            return ck.Repairer(max(n, 1), dt, k, mr).build(_dev(raw, gpu))

        def apply_(raw, n, es, k, rules, dt=dt):
            return ck.Repairer(max(n, 1), dt, k, max(len(rules), 1)).apply(_dev(raw, gpu), rules)

        t, gg = rf.evaluate(dict(case, groups=[g]), build, apply_)
        got_t += t
        got_g += gg
    hdr, rows = case["tensor_rows"]
    col = {h: i for i, h in enumerate(hdr)}
    assert len(rows) == len(got_t)
    for r, g in zip(rows, got_t):
        assert int(r[col["compressed_token_count"]]) == g["tokens"], (name, r)
        assert int(r[col["rule_count"]]) == g["rules"]
    ghdr, grows = case["group_rows"]
    gcol = {h: i for i, h in enumerate(ghdr)}
    assert len(grows) == len(got_g)
    for r, g in zip(grows, got_g):
        assert int(r[gcol["rule_count"]]) == g["rules"]
        assert int(r[gcol["max_pair_frequency"]]) == g["max_pair"]


@pytest.mark.parametrize("name", rf.cases())
def test_golden_inputs_match_oracle(gpu, name):
    case = rf.load_case(name)
    for g in case["groups"]:
        rep = case["manifest"][(g["state_type"], g["category"], g["rep"])]
        dt = TAG[rep["dtype"]]
        others = [case["manifest"][(g["state_type"], g["category"], l)]["raw"] for l in g["layers"]]
        for o in others:
            _check_case(gpu, rep["raw"], dt, case["opts"]["masked"], case["opts"]["max_rules"], other=o)


def _bf16(n, s, seed):
    return dg.normal_bf16(n, s, seed)


def _long_runs(seed):
    """Runs of one word, 5,000 to 40,000 long, between stretches of normal
    bf16: long spans next to short ones on both sides."""
    rng = np.random.default_rng(seed)
    parts = []
    for i in range(12):
        parts.append(_bf16(int(rng.integers(1, 300)), 0.02, seed + i))
        parts.append(np.full(int(rng.integers(5_000, 40_000)), [0x3F80, 0xBC00, 0x3F80][i % 3], np.uint16))
    return np.concatenate(parts)


SYNTH = [
    # (name, dtype, masked request, max_rules, generator)
    ("bf16_normal_300k", 1, None, 50, lambda: _bf16(300_000, 0.02, 11)),
    ("bf16_partial_3", 1, 3, 30, lambda: _bf16(50_000, 0.02, 12)),
    ("f32_expavg_200k", 0, None, 50, lambda: dg.normal_f32(200_000, 1e-3, 13).view(np.uint32)),
    ("f32_partial_12_hash", 0, 12, 20, lambda: dg.normal_f32(60_000, 1e-3, 14).view(np.uint32)),
    ("f32_nomask_hash", 0, 0, 20,
     lambda: np.random.default_rng(15).integers(0, 40, 30_000).astype(np.uint32) * 0x01010101),
    ("f16_runs", 2, 0, 50, lambda: np.repeat(np.array([0x3C00, 0x4000, 0x3C00], np.uint16), [999, 1, 3001])),
    ("f16_periodic", 2, 0, 50, lambda: np.tile(np.array([1, 2, 3, 1, 2], np.uint16), 3000)),
    ("f16_const_odd", 2, 0, 50, lambda: np.full(40_001, 7, np.uint16)),
    ("f16_two", 2, 0, 50, lambda: np.array([5, 5], np.uint16)),
    ("f16_three", 2, 0, 50, lambda: np.array([5, 5, 5], np.uint16)),
    ("f16_one", 2, 0, 50, lambda: np.array([5], np.uint16)),
    ("f16_empty", 2, 0, 50, lambda: np.array([], np.uint16)),
    ("f16_random_ties", 2, 0, 50, lambda: np.random.default_rng(16).integers(0, 6, 777).astype(np.uint16)),
    ("adversarial_f32", 0, None, 50, lambda: dg.adversarial_f32(100_000, 17).view(np.uint32)),
    # spans longer than a tombstone's length field holds (4095 positions with
    # 16-bit ids, 65535 with 32-bit): their lengths go through len / back
    ("bf16_const_long_spans", 1, None, 50, lambda: np.full(200_003, 0x3F80, np.uint16)),
    ("f32_const_long_spans_hash", 0, 12, 50, lambda: np.full(150_001, 0x3F800000, np.uint32)),
    ("bf16_long_runs_mixed", 1, None, 50, lambda: _long_runs(17)),
]


@pytest.fixture(params=[1, 0], ids=["kept_counts", "recount"])
def counting(request):
    # mode 0 of ckr_set_fast_paths: the build recounts every pair each round
    import checkers_amd as ck
    prev = ck.set_fast_paths(request.param)
    yield request.param
    ck.set_fast_paths(prev)


@pytest.mark.parametrize("name,dtype,masked,max_rules,gen", SYNTH, ids=[c[0] for c in SYNTH])
def test_repair_parity(gpu, name, dtype, masked, max_rules, gen, counting):
    raw = gen()
    print(f"[repair] {name} n={raw.size} counting={counting}", flush=True)
    other = np.roll(raw, 7)[: max(raw.size - 5, 0)] if raw.size else raw
    _check_case(gpu, raw, dtype, masked, max_rules, other=other)


def test_repair_many_blocks(gpu, counting):
    # more replace blocks than the single-workgroup scan has threads (4096 tokens each)
    raw = _bf16(4_500_000, 0.02, 21)
    print(f"[repair] many_blocks n=4.5M counting={counting}", flush=True)
    _check_case(gpu, raw, 1, None, 3)


def test_apply_with_foreign_rules(gpu):
    # rules naming symbols absent from the tensor, and rules that never match
    ck = _ck()
    a = np.tile(np.array([0x3C00, 0x4000], np.uint16), 500)
    b = np.tile(np.array([0x3C00, 0x4400, 0x4000], np.uint16), 300)
    ref = oc.repair_build(a, a.size, 2, 0, 50)
    rp = ck.Repairer(a.size, 2, 0, 50)
    g_len, g_seq = rp.apply(_dev(b, gpu), ref["rules"], want_seq=True)
    r_len, r_seq = oc.repair_apply(b, b.size, 2, 0, ref["rules"], want_seq=True)
    assert g_len == r_len and np.array_equal(g_seq, r_seq)


def test_repair_errors(gpu):
    ck = _ck()
    with pytest.raises(ck.CkrError):
        ck.Repairer(100, ck.I8)
    rp = ck.Repairer(100, ck.F16, None, 4)
    import torch
    x = torch.zeros(400, dtype=torch.uint8, device=gpu)
    with pytest.raises(ck.CkrError):
        rp.build(x)           # 200 words > workspace of 100
    with pytest.raises(ck.CkrError):
        rp.apply(x[:100], [(5, 1, 2, 3)])   # replacement must be 2^63 + index


def test_repeated_builds_and_applies_on_one_workspace(gpu):
    """The rounds of a build or apply on a workspace already used for the same
    shape replay a captured graph: four builds and applies of different data on
    one Repairer, with other device work between them, each against the oracle."""
    import torch
    ck = _ck()
    n = 300_000
    rp = ck.Repairer(n, 1, None, 50)
    k = ck.repair_masked_bits(1, None)
    for rep in range(4):
        raw = _bf16(n, 0.02 * (1 + rep), 40 + rep).view(np.uint8)
        got = rp.build(_dev(raw, gpu), want_seq=True)
        torch.ones(1 << 20, device=gpu).mul_(3.0).sum().item()   # eager work between the replays
        ref = oc.repair_build(raw, n, 2, k, 50, want_seq=True)
        assert got["rules"] == ref["rules"], rep
        assert got["out_len"] == ref["out_len"] and got["max_pair"] == ref["max_pair"]
        assert np.array_equal(got["seq"], ref["seq"]), rep
        other = _bf16(n, 0.03, 50 + rep).view(np.uint8)
        g_len, g_seq = rp.apply(_dev(other, gpu), got["rules"], want_seq=True)
        r_len, r_seq = oc.repair_apply(other, n, 2, k, ref["rules"], want_seq=True)
        assert g_len == r_len and np.array_equal(g_seq, r_seq), rep
