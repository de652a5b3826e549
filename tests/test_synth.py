"""The synthetic workloads' routing statistics (no GPU): the speculative-verify batch must repeat
about 30% of its routed experts across its 8 tokens (40-52 distinct experts of 72 slots, the
shared expert included), as the 8-token verify workload specifies; independent tokens repeat far
fewer.  Routing runs through the oracle on the host-generated router weights and activations."""
import numpy as np
import pytest
import torch

from conftest import bf16_bits

BENCH_SEED = 2026  # bench.py's default seed; the verify batches use seeds BENCH_SEED + 2000 + t


def _distinct(orc, x, w, bias):
    ids, _ = orc.route(orc.router_logits(bf16_bits(x), w.numpy()), bias.numpy())
    return len(np.unique(ids))


@pytest.mark.parametrize("t", range(4))
def test_verify_batch_repeats_about_30_percent(orc, t):
    from mlxlr8_amd import synth
    w, bias = synth.router("cpu", BENCH_SEED)
    x, _ = synth.activations("cpu", BENCH_SEED + 2000 + t, 8, correlated=True)
    u = _distinct(orc, x, w, bias)
    assert 40 <= u <= 52, u


def test_independent_tokens_repeat_less(orc):
    from mlxlr8_amd import synth
    w, bias = synth.router("cpu", BENCH_SEED)
    x, _ = synth.activations("cpu", BENCH_SEED + 2000, 8)
    assert _distinct(orc, x, w, bias) > 52


def test_router_and_activations_are_device_independent():
    from mlxlr8_amd import synth
    w1, b1 = synth.router("cpu", 5)
    w2, b2 = synth.router("cpu", 5)
    assert torch.equal(w1, w2) and torch.equal(b1, b2)
    assert abs(float(w1.std()) - 0.02) < 1e-3
