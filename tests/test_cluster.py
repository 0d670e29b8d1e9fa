"""Fingerprint weights and clusters (host code of the library) against the
oracle, which is pinned here by hand-worked cases."""
import math

import numpy as np
import pytest

import checkers_amd as ck
import oracle as oc


def test_oracle_hand_worked_clusters():
    # five model-state tensors differing in the mean only: pairwise distances in
    # units of the (population) std of that dimension are 1,1,9,10,10,11,19,20,29,30;
    # the threshold is element 10//4 = 2 of the sorted list, 9; strictly closer
    # pairs merge: {A,B}, {C,D}; E alone
    fps = [[m, 0, 0, 0, 0] for m in (0, 1, 10, 11, 30)]
    ids, thr = oc.cluster(["a", "b", "c", "d", "e"], fps)
    sd = math.sqrt(np.var([0, 1, 10, 11, 30]))
    assert ids == [0, 0, 1, 1, -1]
    assert thr == [pytest.approx(9 / sd, rel=1e-12)]
    # four equally spaced: threshold = 2nd smallest distance = the smallest, none strictly below
    ids, _ = oc.cluster(list("abcd"), [[m, 0, 0, 0, 0] for m in (0, 1, 10, 11)])
    assert ids == [-1, -1, -1, -1]
    # categories in name order (exp_avg < exp_avg_sq < master_weights < model_state), ids run on
    names = ["w1", "optimizer.exp_avg::x", "w2", "optimizer.exp_avg::y", "w3", "optimizer.exp_avg::z",
             "master_weights::m", "w4", "optimizer.exp_avg::q", "w5"]
    fps = [[0, 0, 0, 0, 0], [5, 0, 0, 0, 0], [1, 0, 0, 0, 0], [5.1, 0, 0, 0, 0], [10, 0, 0, 0, 0],
           [50, 0, 0, 0, 0], [1, 1, 1, 1, 1], [11, 0, 0, 0, 0], [60, 0, 0, 0, 0], [30, 0, 0, 0, 0]]
    ids, thr = oc.cluster(names, fps)
    # exp_avg {5, 5.1, 50, 60}: distances .1,10,44.9,45,54.9,55 -> threshold 10 -> {x,y} merge -> id 0
    # model_state as the first case -> ids 1 and 2
    assert ids == [1, 0, 1, 0, 2, -1, -1, 2, -1, -1]
    assert len(thr) == 3


def test_oracle_hand_worked_weights():
    w = oc.fingerprint_weights([[1, 0, 0, 0, 0], [3, 0, 0, 0, 0]])
    assert w[0] == pytest.approx(1 / (1 + 5e-8), rel=1e-12) and all(abs(x) < 1e-7 for x in w[1:])


@pytest.mark.parametrize("seed", range(30))
def test_cluster_matches_oracle(seed):
    rng = np.random.default_rng(seed)
    n = int(rng.integers(1, 40))
    pre = ["", "optimizer.exp_avg::", "optimizer.exp_avg_sq::", "master_weights::"]
    names = [pre[int(rng.integers(0, 4))] + f"t{i}" for i in range(n)]
    base = rng.standard_normal((4, 5)) * 10
    fps = (base[rng.integers(0, 4, n)] + rng.standard_normal((n, 5)) * rng.choice([0.01, 1.0])).astype(np.float32)
    if seed % 5 == 0:
        fps[:, 2] = 0.0   # a constant dimension (std -> 1)
    ids, thr = ck.cluster(names, fps)
    rids, rthr = oc.cluster(names, fps)
    assert ids == rids
    assert thr == pytest.approx(rthr, rel=1e-12, abs=0)
    assert ck.fingerprint_weights(fps) == pytest.approx(oc.fingerprint_weights(fps), rel=1e-9, abs=1e-15)
