"""The fused finishes equal their unfused composition bit for bit (MI355X, through the C ABI).

The reference requires ``JoinedMXFP4.finish(x, ids, scores, residual)`` to equal the per-slot
values of ``slots`` combined by the caller (tests/test_joined_mxfp4.py:89-107), and the K4
``compiled_expert_mlp_finish`` to equal ``fast_expert_mlp`` plus the model combine
(tests/test_fast_decode.py:459-476, exlr8/model.py:415-418).  Here the fused entry points
(moe_mxfp4_mlp_finish, moe_k4_mlp_finish, and the one-call decode blocks) are checked against
moe_mxfp4_mlp / moe_k4_mlp followed by moe_combine_values.
"""
import sys

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

H, M = 6144, 2048


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _same(a, b):
    return torch.equal(a.contiguous().view(torch.int16), b.contiguous().view(torch.int16))


@pytest.fixture(scope="module")
def joined(cuda):
    from mlxlr8_amd import synth
    from mlxlr8_amd.joined_mxfp4 import JoinedMXFP4
    say("building 9-expert MXFP4 layer")
    L = synth.mxfp4_layer(cuda, 303, experts=9)
    side = L["side"]
    return JoinedMXFP4(L["weights"], L["unit"], {"gate": (None, side["out_gate"]), "up": (None, side["out_up"]),
                                                 "down": (side["in_down"], side["out_down"])}, H, M)


@pytest.fixture(scope="module")
def k4(cuda):
    from mlxlr8_amd import synth
    from mlxlr8_amd.experts import ExpertLayer
    say("building 9-expert K4 layer")
    return ExpertLayer(**synth.k4_layer(cuda, 404, experts=9), hidden=H, intermediate=M)


def _case(cuda, rows, seed, experts=9):
    g = torch.Generator(device="cpu").manual_seed(seed)
    ids = torch.randint(0, experts - 1, (rows, 9), generator=g, dtype=torch.int32)
    ids[:, 8] = experts - 1
    scores = torch.rand((rows, 8), generator=g) * 0.3 + 0.02
    x = torch.randn((rows, H), generator=g).to(torch.bfloat16)
    res = torch.randn((rows, H), generator=g).to(torch.bfloat16)
    return x.to(cuda), ids.to(cuda), scores.to(cuda), res.to(cuda)


@pytest.mark.parametrize("rows", [1, 2, 3, 4, 8])
def test_mxfp4_finish_equals_slots_plus_combine(cuda, joined, rows):
    from mlxlr8_amd.fast_decode import combine_values
    say(f"case: mxfp4 finish == combine(slots) rows={rows}")
    x, ids, scores, res = _case(cuda, rows, 700 + rows)
    fused = joined.finish(x, ids, scores, res)
    values = joined.slots(x, ids)
    composed = combine_values(values, scores, res)
    torch.cuda.synchronize()
    assert _same(fused, composed)


@pytest.mark.parametrize("rows", [1, 2, 3, 4, 8])
def test_k4_finish_equals_values_plus_combine(cuda, k4, rows):
    from mlxlr8_amd.fast_decode import combine_values, compiled_expert_mlp_finish, fast_expert_mlp
    say(f"case: k4 finish == combine(values) rows={rows}")
    x, ids, scores, res = _case(cuda, rows, 800 + rows)
    fused = compiled_expert_mlp_finish(k4)(x, ids, scores, res)
    values = fast_expert_mlp(x, ids, k4.packed, k4.scales, 4, H, M)
    composed = combine_values(values, scores, res)
    torch.cuda.synchronize()
    assert _same(fused, composed)
