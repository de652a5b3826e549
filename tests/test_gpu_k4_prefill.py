"""Grouped K4 expert MLP for prefill rows (moe_k4_grouped_mlp) on the MI355X against the oracle's
per-slot K4 MLP (exlr8/fast_prefill.py:188-211 grouped_expert_mlp semantics)."""
import sys

import numpy as np
import pytest
import torch

from conftest import bf16_bits, bits_to_f32, f16_bits, rel_l2

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _layer(cuda, seed, h, m, experts):
    from mlxlr8_amd import synth
    layer = synth.k4_layer(cuda, seed, hidden=h, intermediate=m, experts=experts)
    host = {p: layer["packed"][p].cpu().numpy() for p in ("gate", "up", "down")}
    sc = {p: tuple(f16_bits(v) for v in layer["scales"][p]) for p in ("gate", "up", "down")}
    return layer, host, sc


def _oracle_values(orc, x, ids, host, sc, h, m):
    rows = ids.shape[0]
    res = np.zeros((rows, h), np.uint16)
    _, want = orc.k4_moe(bf16_bits(x), ids, np.zeros((rows, 8), np.float32), res, h, m,
                         host["gate"], host["up"], host["down"], sc["gate"][0], sc["gate"][1], sc["up"][0],
                         sc["up"][1], sc["down"][0], sc["down"][1], want_values=True)
    return bits_to_f32(want).reshape(rows, 9, h)


def test_grouped_all_item_classes_small(cuda, orc):
    """Segments of 70 (64 + 6), 40, 33, 20, 12 and 5 rows: every M-tile class and a split expert."""
    from mlxlr8_amd.fast_prefill import grouped_expert_mlp
    h, m, E = 256, 256, 6
    say(f"case: grouped small h={h} m={m} experts={E}")
    layer, host, sc = _layer(cuda, 303, h, m, E)
    counts = {0: 70, 1: 40, 2: 20, 3: 12, 4: 5, 5: 33}  # 180 slots = 20 rows x 9
    flat = np.concatenate([np.full(c, e, np.int32) for e, c in counts.items()])
    rng = np.random.default_rng(7)
    rng.shuffle(flat)
    ids_np = flat.reshape(-1, 9)
    rows = ids_np.shape[0]
    x = torch.from_numpy(rng.normal(size=(rows, h)).astype(np.float32)).to(cuda).to(torch.bfloat16)
    ids = torch.from_numpy(ids_np).to(cuda)
    values = grouped_expert_mlp(x, ids, layer["packed"], layer["scales"], 4, h, m)
    torch.cuda.synchronize()
    assert values.shape == (rows, 9, h) and values.dtype == torch.bfloat16
    got = bits_to_f32(bf16_bits(values)).reshape(rows, 9, h)
    want = _oracle_values(orc, x, ids_np.astype(np.uint32), host, sc, h, m)
    err = rel_l2(got, want)
    worst = max(rel_l2(got[r, s], want[r, s]) for r in range(rows) for s in range(9))
    say(f"  rel_l2={err:.3e} worst slot {worst:.3e}")
    assert err <= 1e-3
    assert worst <= 4e-3  # bf16 output rounding of one 256-wide slot


def test_grouped_glm_shapes(cuda, orc):
    from mlxlr8_amd.fast_prefill import grouped_expert_mlp
    h, m, E, rows = 6144, 2048, 5, 24
    say(f"case: grouped GLM h={h} m={m} experts={E} rows={rows}")
    layer, host, sc = _layer(cuda, 404, h, m, E)
    rng = np.random.default_rng(8)
    ids_np = rng.integers(0, E, (rows, 9)).astype(np.int32)
    g = torch.Generator(device=cuda)
    g.manual_seed(10)
    x = torch.randn((rows, h), generator=g, device=cuda).to(torch.bfloat16)
    values = grouped_expert_mlp(x, torch.from_numpy(ids_np).to(cuda), layer["packed"], layer["scales"], 4, h, m)
    torch.cuda.synchronize()
    got = bits_to_f32(bf16_bits(values)).reshape(rows, 9, h)
    want = _oracle_values(orc, x, ids_np.astype(np.uint32), host, sc, h, m)
    err = rel_l2(got, want)
    say(f"  rel_l2={err:.3e}")
    assert err <= 1e-3


def test_grouped_matches_decode_path(cuda):
    """The grouped prefill and the decode MLP (moe_k4_mlp) compute the same values."""
    from mlxlr8_amd.fast_decode import fast_expert_mlp
    from mlxlr8_amd.fast_prefill import grouped_expert_mlp
    h, m, E, rows = 6144, 2048, 4, 6
    say("case: grouped vs decode path")
    layer, _, _ = _layer(cuda, 505, h, m, E)
    rng = np.random.default_rng(9)
    ids = torch.from_numpy(rng.integers(0, E, (rows, 9)).astype(np.int32)).to(cuda)
    x = torch.from_numpy(rng.normal(size=(rows, h)).astype(np.float32)).to(cuda).to(torch.bfloat16)
    a = grouped_expert_mlp(x, ids, layer["packed"], layer["scales"], 4, h, m)
    b = fast_expert_mlp(x, ids, layer["packed"], layer["scales"], 4, h, m)
    torch.cuda.synchronize()
    err = rel_l2(bits_to_f32(bf16_bits(a)), bits_to_f32(bf16_bits(b)))
    say(f"  rel_l2={err:.3e}")
    assert err <= 1e-3
    # deterministic across calls
    c = grouped_expert_mlp(x, ids, layer["packed"], layer["scales"], 4, h, m)
    torch.cuda.synchronize()
    assert torch.equal(a, c)
