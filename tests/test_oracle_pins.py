"""The CPU oracle is pinned before anything is compared against it.

Runs every check in pins.py against the oracle, then against builds of the
oracle with one planted mistake each (-DORACLE_MUTATION=k) and requires that
each planted mistake is caught by at least one check.
"""
import json
import os

import numpy as np
import pytest

import oracle
import pins

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.parametrize("check", pins.ALL_CHECKS, ids=lambda c: c.__name__)
def test_oracle_passes(check):
    fails = check(0)
    assert not fails, "\n".join(fails)


MUTATIONS = {
    1: "eps dropped",
    2: "mean over D-1",
    3: "sign of projection term flipped",
    4: "dot uses dy instead of dy*gamma",
    5: "dgamma uses x instead of xhat",
    6: "gamma index reversed",
    7: "r*r replaced by r",
    8: "dgamma drops last row",
}


@pytest.mark.parametrize("mutation", sorted(MUTATIONS), ids=lambda m: MUTATIONS[m])
def test_planted_mistake_is_caught(mutation):
    assert oracle.load(mutation).oracle_mutation() == mutation
    fails = pins.run_all(mutation)
    assert fails, f"mutation {mutation} ({MUTATIONS[mutation]}) passed every pinning check"


def test_bf16_rounding_matches_torch():
    with open(os.path.join(HERE, "golden", "bf16_golden.json")) as fh:
        g = json.load(fh)
    f = np.array(g["f32_bits"], dtype=np.uint32).view(np.float32)
    want = np.array(g["bf16_bits"], dtype=np.uint16)
    got = oracle.bf16_encode(f)
    nan = np.array(g["is_nan"])
    assert np.array_equal(got[~nan], want[~nan])
    back = oracle.bf16_decode(got)
    assert np.all(np.isnan(back[nan]))
    # decode is exact: bf16 -> f32 -> bf16 round trip
    assert np.array_equal(oracle.bf16_encode(oracle.bf16_decode(want[~nan])), want[~nan])


def test_oracle_threads_agree():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((64, 96)).astype(np.float32)
    g = rng.uniform(0.5, 1.5, 96).astype(np.float32)
    dy = rng.standard_normal((64, 96)).astype(np.float32)
    oracle.set_threads(1)
    y1, i1 = oracle.fwd(x, g, 1e-6)
    dx1, dg1 = oracle.bwd(x, g, i1, dy)
    oracle.set_threads(4)
    try:
        y4, i4 = oracle.fwd(x, g, 1e-6)
        dx4, dg4 = oracle.bwd(x, g, i4, dy)
    finally:
        oracle.set_threads(1)
    assert np.array_equal(y1, y4) and np.array_equal(dx1, dx4) and np.array_equal(dg1, dg4)


def test_oracle_empty_inputs():
    x = np.zeros((0, 16), dtype=np.float32)
    y, inv = oracle.fwd(x, None, 1e-6)
    assert y.shape == (0, 16) and inv.shape == (0,)
    dx, dg = oracle.bwd(x, None, inv, x, dgamma=np.ones(16, np.float32))
    assert np.all(dg == 0.0)
