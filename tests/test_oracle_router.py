"""Pin the oracle router against a greedy selection restatement.

The router (exlr8/fast_router.py:7-25) scores every expert with sigmoid(logit), adds the
selection bias, keeps the 8 best corrected scores (lower expert id first on equal scores) and
weights them by their uncorrected sigmoid, normalised to sum to 2.5 with 1e-20 added to the
denominator (exlr8/metal/fast_router.metal:34-39); slot 8 names the shared expert 256.  The restatement below picks experts one at a time in float64.
"""
import numpy as np
import pytest


def greedy_route(logits, bias):
    """(ids [rows, 8], weights [rows, 8]) by repeated arg-max; the first maximum wins a tie."""
    logits = np.asarray(logits, np.float64)
    sig = np.exp(-np.logaddexp(0.0, -logits))          # sigmoid without overflow
    ids = np.zeros((logits.shape[0], 8), np.int64)
    weights = np.zeros((logits.shape[0], 8))
    for r in range(logits.shape[0]):
        corrected = (sig[r].astype(np.float32) + np.asarray(bias, np.float32)).astype(np.float64)
        for slot in range(8):
            best = int(np.argmax(corrected))                # first index among equal maxima
            ids[r, slot], weights[r, slot] = best, sig[r, best]
            corrected[best] = -np.inf
        weights[r] *= 2.5 / (1e-20 + weights[r].sum())
    return ids, weights


def router_case(case, rows, seed=28):
    """Logits [rows, 256] and bias [256] for one named situation of the selection."""
    rng = np.random.default_rng(seed + rows)
    logits = rng.standard_normal((rows, 256)).astype(np.float32) * 1.5
    bias = rng.uniform(-0.3, 0.3, 256).astype(np.float32)
    if case == "bias":          # a bias block outranks every sigmoid difference
        bias[:] = 0
        bias[40:48] = 3.0
    elif case == "ties":        # all corrected scores equal: the eight lowest ids win
        logits[:] = 0.25
        bias[:] = 0
    elif case == "saturated":   # |logits| far past the sigmoid's saturation
        logits *= 80
    elif case == "zero":        # every sigmoid is ~0: the weights are still finite
        logits[:] = -900
    return logits, bias


@pytest.mark.parametrize("rows", [1, 2, 3, 4, 8])
@pytest.mark.parametrize("case", ["random", "bias", "ties", "saturated", "zero"])
def test_oracle_route_matches_greedy_selection(orc, rows, case):
    logits, bias = router_case(case, rows)
    ids, scores = orc.route(logits, bias)
    chosen, weights = greedy_route(logits, bias)
    np.testing.assert_array_equal(ids[:, :8], chosen)
    np.testing.assert_array_equal(ids[:, 8], 256)
    np.testing.assert_allclose(scores, weights, rtol=2e-6, atol=1e-7)
    assert np.isfinite(scores).all()
    if case == "bias":
        np.testing.assert_array_equal(np.sort(ids[:, :8], axis=1), np.tile(np.arange(40, 48), (rows, 1)))
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
