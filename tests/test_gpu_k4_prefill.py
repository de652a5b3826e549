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


def _layer_k(cuda, seed, h, m, experts, k):
    from mlxlr8_amd import synth
    layer = synth.k4_layer(cuda, seed, hidden=h, intermediate=m, experts=experts, k=k)
    host = {p: layer["packed"][p].cpu().numpy() for p in ("gate", "up", "down")}
    sc = {p: tuple(f16_bits(v) for v in layer["scales"][p]) for p in ("gate", "up", "down")}
    return layer, host, sc


@pytest.mark.parametrize("k", [3, 2])
def test_grouped_k3_k2_small(cuda, orc, k):
    """K3/K2 experts through the generic-window grouped kernel: every M-tile class, a split expert."""
    from mlxlr8_amd.fast_prefill import grouped_expert_mlp
    h, m, E = 256, 384, 6
    say(f"case: grouped K{k} small h={h} m={m} experts={E}")
    layer, host, sc = _layer_k(cuda, 600 + k, h, m, E, k)
    counts = {0: 70, 1: 40, 2: 20, 3: 12, 4: 5, 5: 33}
    flat = np.concatenate([np.full(c, e, np.int32) for e, c in counts.items()])
    rng = np.random.default_rng(11 + k)
    rng.shuffle(flat)
    ids_np = flat.reshape(-1, 9)
    rows = ids_np.shape[0]
    x = torch.from_numpy(rng.normal(size=(rows, h)).astype(np.float32)).to(cuda).to(torch.bfloat16)
    values = grouped_expert_mlp(x, torch.from_numpy(ids_np).to(cuda), layer["packed"], layer["scales"], k, h, m)
    torch.cuda.synchronize()
    got = bits_to_f32(bf16_bits(values)).reshape(rows, 9, h)
    res = np.zeros((rows, h), np.uint16)
    _, want = orc.k4_moe(bf16_bits(x), ids_np.astype(np.uint32), np.zeros((rows, 8), np.float32), res, h, m,
                         host["gate"], host["up"], host["down"], sc["gate"][0], sc["gate"][1], sc["up"][0],
                         sc["up"][1], sc["down"][0], sc["down"][1], want_values=True, k=k)
    err = rel_l2(got, bits_to_f32(want).reshape(rows, 9, h))
    say(f"  rel_l2={err:.3e}")
    assert err <= 1e-3


def test_k3_expert_layer_glm_shapes(cuda, orc):
    """A K3 layer (the multi-token-prediction layer's width) at 6144 x 2048: decode rows through
    ExpertLayer and the combined finish, against the oracle's K3 MoE layer."""
    from mlxlr8_amd.experts import ExpertLayer
    from mlxlr8_amd.fast_decode import compiled_expert_mlp_finish
    h, m, E, rows = 6144, 2048, 5, 2
    say(f"case: K3 ExpertLayer GLM shapes experts={E} rows={rows}")
    layer, host, sc = _layer_k(cuda, 707, h, m, E, 3)
    expert = ExpertLayer(layer["packed"], layer["scales"], h, m, k=3, number=78)
    rng = np.random.default_rng(12)
    ids_np = rng.integers(0, E, (rows, 9)).astype(np.int32)
    x = torch.from_numpy(rng.normal(size=(rows, h)).astype(np.float32)).to(cuda).to(torch.bfloat16)
    residual = torch.from_numpy(rng.normal(size=(rows, h)).astype(np.float32)).to(cuda).to(torch.bfloat16)
    scores = torch.from_numpy(rng.uniform(.05, .3, (rows, 8)).astype(np.float32)).to(cuda)
    ids = torch.from_numpy(ids_np).to(cuda)
    values = expert(x, ids)
    out = compiled_expert_mlp_finish(expert)(x, ids, scores, residual)
    torch.cuda.synchronize()
    want_out, want = orc.k4_moe(bf16_bits(x), ids_np.astype(np.uint32), scores.cpu().numpy(), bf16_bits(residual), h, m,
                                host["gate"], host["up"], host["down"], sc["gate"][0], sc["gate"][1], sc["up"][0],
                                sc["up"][1], sc["down"][0], sc["down"][1], want_values=True, k=3)
    err = rel_l2(bits_to_f32(bf16_bits(values)).reshape(rows, 9, h), bits_to_f32(want).reshape(rows, 9, h))
    err_out = rel_l2(bits_to_f32(bf16_bits(out)), bits_to_f32(want_out))
    say(f"  values rel_l2={err:.3e} out rel_l2={err_out:.3e}")
    assert err <= 1e-3 and err_out <= 1e-3


@pytest.mark.parametrize("k,side,per_slot", [(3, 1, False), (3, 2, True), (2, 1, True)])
def test_k3_expert_linear(cuda, orc, k, side, per_slot):
    """expert_linear for K3/K2 experts (one projection, either storage side, token or slot rows)."""
    from mlxlr8_amd.trellis import expert_linear
    in_f, out_f, E, rows, slots = (256, 384, 4, 3, 5) if side == 1 else (384, 256, 4, 3, 5)
    say(f"case: K{k} expert_linear side={side} per_slot={per_slot}")
    rng = np.random.default_rng(30 + k + side)
    packed = torch.from_numpy(rng.integers(0, 256, E * in_f * out_f * k // 8, dtype=np.uint8)).to(cuda)
    ins = rng.uniform(-.5, .5, (E, in_f)).astype(np.float16)
    outs = rng.uniform(-.5, .5, (E, out_f)).astype(np.float16)
    ids_np = rng.integers(0, E, (rows, slots)).astype(np.int32)
    shape = (rows, slots, in_f) if per_slot else (rows, in_f)
    x = torch.from_numpy(rng.normal(size=shape).astype(np.float32)).to(cuda).to(torch.bfloat16)
    y = expert_linear(x, torch.from_numpy(ids_np).to(cuda), packed, torch.from_numpy(ins).to(cuda),
                      torch.from_numpy(outs).to(cuda), k, in_f, out_f, side)
    torch.cuda.synchronize()
    assert y.shape == (rows, slots, out_f)
    xf = bits_to_f32(bf16_bits(x))
    xs = xf.reshape(rows * slots, in_f) if per_slot else np.repeat(xf.reshape(rows, in_f), slots, axis=0)
    want = orc.k4_linear(xs, ids_np.ravel(), packed.cpu().numpy(), in_f, out_f, side, ins.view(np.uint16),
                         outs.view(np.uint16), k=k)
    # the reference's expert_linear returns T(y): compare with the oracle's float output cast to bf16
    want_t = torch.from_numpy(want).to(torch.bfloat16).float().numpy()
    got = bits_to_f32(bf16_bits(y)).reshape(-1, out_f)
    err = rel_l2(got, want_t)
    say(f"  rel_l2={err:.3e}")
    assert err <= 1e-3
    np.testing.assert_allclose(got, want, rtol=2 ** -7, atol=1e-6)  # within one bf16 ulp
