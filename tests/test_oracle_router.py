"""Pin the oracle router against an argsort-stable restatement (tests/test_fast_router.py:14-45)."""
import numpy as np
import pytest


def _expected(host, bias):
    with np.errstate(over="ignore"):
        small = 1 / (1 + np.exp(np.abs(host)))
    original = np.where(host < 0, small, 1 - small).astype(np.float32)
    chosen = np.argsort(-(original + bias), axis=-1, kind="stable")[..., :8]
    weights = np.take_along_axis(original, chosen, axis=-1)
    weights = weights / (weights.sum(axis=-1, keepdims=True) + 1e-20) * 2.5
    return chosen, weights


def router_case(case, rows, seed=28):
    rng = np.random.default_rng(seed)
    host = rng.normal(size=(rows, 256)).astype(np.float32)
    bias = rng.normal(0, .2, 256).astype(np.float32)
    if case == "bias":
        bias[:8] = 4
    elif case == "ties":
        host[:] = .5
        bias[:] = 0
    elif case == "saturated":
        host *= 100
    elif case == "zero":
        host[:] = -1000
    return host, bias


@pytest.mark.parametrize("rows", [1, 2, 3, 4, 8])
@pytest.mark.parametrize("case", ["random", "bias", "ties", "saturated", "zero"])
def test_oracle_route_matches_stable_argsort(orc, rows, case):
    host, bias = router_case(case, rows)
    ids, scores = orc.route(host, bias)
    chosen, weights = _expected(host, bias)
    np.testing.assert_array_equal(ids[:, :8], chosen)
    np.testing.assert_array_equal(ids[:, 8], 256)
    np.testing.assert_allclose(scores, weights, rtol=1e-6, atol=1e-7)
    assert np.isfinite(scores).all()
    if case == "bias":
        np.testing.assert_array_equal(np.sort(ids[:, :8], axis=1), np.tile(np.arange(8), (rows, 1)))
    if case == "ties":
        np.testing.assert_array_equal(ids[:, :8], np.tile(np.arange(8), (rows, 1)))


def test_bias_changes_selection_not_probability(orc):
    # exlr8 tests/test_model.py:391-398: bias selects, the sigmoid score weights
    host, bias = router_case("random", 1)
    ids0, s0 = orc.route(host, np.zeros(256, np.float32))
    forced = np.zeros(256, np.float32)
    forced[ids0[0, 7]] = 0  # unchanged top
    big = np.zeros(256, np.float32)
    big[200:208] = 10
    ids1, s1 = orc.route(host, big)
    np.testing.assert_array_equal(np.sort(ids1[0, :8]), np.arange(200, 208))
    sig = 1 / (1 + np.exp(-host[0, 200:208].astype(np.float64)))
    np.testing.assert_allclose(np.sort(s1[0]), np.sort(sig / sig.sum() * 2.5), rtol=1e-5)


def test_router_logits_float64_textbook(orc):
    rng = np.random.default_rng(1)
    x = rng.normal(size=(3, 1024)).astype(np.float32)
    xb = (x.view(np.uint32) >> 16).astype(np.uint16)
    w = rng.normal(0, .02, (256, 1024)).astype(np.float32)
    got = orc.router_logits(xb, w)
    want = ((xb.astype(np.uint32) << 16).view(np.float32).astype(np.float64) @ w.T.astype(np.float64))
    np.testing.assert_allclose(got, want, rtol=1e-6, atol=1e-7)


def test_segment_table_brute_force(orc):
    rng = np.random.default_rng(4)
    ids = rng.integers(0, 10, 57).astype(np.uint32)
    order, counts, starts, table = orc.segment_table(ids, 10, 8)
    np.testing.assert_array_equal(order, np.argsort(ids, kind="stable"))
    np.testing.assert_array_equal(counts, np.bincount(ids, minlength=10))
    # every slot appears once; blocks are contiguous, sorted, at most 8 rows, one expert each
    covered = np.concatenate([np.arange(f, f + l) for _, f, l in table.T])
    np.testing.assert_array_equal(covered, np.arange(ids.size))
    for e, f, l in table.T:
        assert 1 <= l <= 8 and (ids[order[f:f + l]] == e).all()
