"""Load-time K4 -> joined-MXFP4 encode on the MI355X against the CPU oracle (bit-exact codes and
scales), at the reference test's fixture shapes and at the GLM-5.3 expert shape."""
import sys

import numpy as np
import pytest
import torch

from conftest import f16_bits

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _expert_layer(cuda, h, m, count, seed):
    from mlxlr8_amd.experts import ExpertLayer
    rng = np.random.default_rng(seed)
    signs = rng.choice([-1, 1], h).astype(np.float16)
    packed, scales = {}, {}
    for projection in ("gate", "up", "down"):
        incoming, outgoing = (m, h) if projection == "down" else (h, m)
        packed[projection] = rng.integers(0, 256, count * h * m // 2, np.uint8)
        incoming_scale = rng.uniform(.01, .04, (count, incoming)).astype(np.float16)
        if projection != "down":
            block = rng.uniform(.01, .04, (count, h // 128)).astype(np.float16)
            block *= rng.choice([-1, 1], block.shape).astype(np.float16)
            incoming_scale = np.repeat(block, 128, axis=-1) * signs
        scales[projection] = (incoming_scale, rng.uniform(-.5, .5, (count, outgoing)).astype(np.float16))
    layer = ExpertLayer({p: torch.from_numpy(a).to(cuda) for p, a in packed.items()},
                        {p: tuple(torch.from_numpy(v).to(cuda) for v in pair) for p, pair in scales.items()}, h, m)
    return layer, packed, scales


def _oracle_encode(orc, packed, scales, h, m, count):
    unit = np.sign(scales["gate"][0][0]).astype(np.float16)
    gu = (np.zeros((count, 2 * m, h // 2), np.uint8), np.zeros((count, 2 * m, h // 32), np.uint8))
    dn = (np.zeros((count, h, m // 2), np.uint8), np.zeros((count, h, m // 32), np.uint8))
    orc.k4_to_mxfp4(packed["gate"], h, m, 1, count, scales["gate"][0].view(np.uint16), unit.view(np.uint16), *gu, 0)
    orc.k4_to_mxfp4(packed["up"], h, m, 1, count, scales["up"][0].view(np.uint16), unit.view(np.uint16), *gu, m)
    orc.k4_to_mxfp4(packed["down"], m, h, 2, count, None, None, *dn, 0)
    return unit, gu, dn


@pytest.mark.parametrize("h,m,count", [(256, 128, 257), (6144, 2048, 2)])
def test_encode_bit_exact(cuda, orc, h, m, count):
    from mlxlr8_amd.joined_mxfp4 import encode
    say(f"encode h={h} m={m} experts={count}")
    layer, packed, scales = _expert_layer(cuda, h, m, count, 817 + h)
    unit, weights = encode(layer)
    torch.cuda.synchronize()
    ounit, gu, dn = _oracle_encode(orc, packed, scales, h, m, count)
    np.testing.assert_array_equal(f16_bits(unit).reshape(-1), ounit.view(np.uint16))
    for name, got, want in (("gate_up", weights["gate_up"], gu), ("down", weights["down"], dn)):
        assert got[2] is None
        for i in range(2):
            g = got[i].cpu().numpy()
            assert g.shape == want[i].shape, (name, i, g.shape, want[i].shape)
            bad = np.argwhere(g != want[i])
            assert bad.size == 0, f"{name}[{i}]: {len(bad)} mismatches, first at {bad[:3].tolist()}"


def test_joined_from_expert_layer(cuda, orc):
    """JoinedMXFP4(expert) (reference constructor) encodes, then decodes a routed block that matches
    the oracle's MXFP4 layer on the encoded weights."""
    from conftest import bf16_bits, bits_to_f32, rel_l2
    from mlxlr8_amd.joined_mxfp4 import JoinedMXFP4
    h, m, count = 6144, 2048, 3
    say("JoinedMXFP4(expert) at 6144 x 2048, 3 experts")
    layer, _, scales = _expert_layer(cuda, h, m, count, 2024)
    joined = JoinedMXFP4(layer)
    torch.manual_seed(3)
    x = torch.randn(2, h, device=cuda).to(torch.bfloat16)
    ids = torch.tensor([[0, 1, 2, 0, 1, 2, 0, 1, 2], [2, 2, 1, 1, 0, 0, 2, 1, 0]], dtype=torch.int32, device=cuda)
    values = joined.slots(x, ids)
    torch.cuda.synchronize()
    (gc, gs), (dc, ds) = joined.weights["gate_up"], joined.weights["down"]
    scores = np.full((2, 8), 0.125, np.float32)
    residual = np.zeros((2, h), np.uint16)
    _, want = orc.mxfp4_moe(bf16_bits(x), ids.cpu().numpy().astype(np.uint32), scores, residual, h, m,
                            gc.cpu().numpy(), gs.cpu().numpy(), dc.cpu().numpy(), ds.cpu().numpy(),
                            f16_bits(joined.unit), scales["gate"][1].view(np.uint16), scales["up"][1].view(np.uint16),
                            scales["down"][0].view(np.uint16), scales["down"][1].view(np.uint16), want_values=True)
    got = bits_to_f32(bf16_bits(values)).reshape(want.shape)
    err = rel_l2(got, bits_to_f32(want))
    say(f"rel L2 {err:.2e}")
    assert err <= 1e-3
