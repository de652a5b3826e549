"""Every entry that takes caller ids clamps an id outside [0, experts) to the nearest valid expert:
the decode path (<= 8 MXFP4 rows, <= 16 K4 rows) and the grouped path (more rows) give a slot with
an out-of-range id exactly the values of the clamped id, so a batch gives the same result on
either side of the path switch."""
import pytest
import torch

from gpu_helpers import say

pytestmark = pytest.mark.gpu


def _bits(t):
    return t.contiguous().view(torch.int16)


def _ids(cuda, rows, experts, seed):
    g = torch.Generator(device="cpu").manual_seed(seed)
    ids = torch.stack([torch.randperm(experts - 1, generator=g)[:8] for _ in range(rows)])
    ids = torch.cat([ids, torch.full((rows, 1), experts - 1)], dim=1)
    return ids.to(torch.int32).to(cuda)


def _check(call, ids, experts, label):
    bad = ids.clone()
    bad[0, 3] = experts + 40          # beyond the last expert -> clamped to experts - 1
    bad[-1, 5] = -7                    # negative -> clamped to 0
    want_ids = bad.clone()
    want_ids[0, 3] = experts - 1
    want_ids[-1, 5] = 0
    got = call(bad)
    want = call(want_ids)
    torch.cuda.synchronize()
    assert torch.isfinite(got.float()).all(), f"{label}: non-finite values"
    assert torch.equal(_bits(got), _bits(want)), f"{label}: out-of-range ids not clamped"


def test_mxfp4_slots_clamp_on_both_paths(cuda):
    from mlxlr8_amd import synth
    from mlxlr8_amd.joined_mxfp4 import JoinedMXFP4
    L = synth.mxfp4_layer(cuda, 53, experts=8)
    side = L["side"]
    joined = JoinedMXFP4(L["weights"], L["unit"], {"gate": (None, side["out_gate"]), "up": (None, side["out_up"]),
                                                   "down": (side["in_down"], side["out_down"])}, 6144, 2048)
    assert joined.grouped_exact
    for rows in (8, 9):
        say(f"case: MXFP4 slots, 8 experts, rows {rows} ({'decode' if rows <= 8 else 'grouped'} path)")
        x, _ = synth.activations(cuda, 54 + rows, rows)
        ids = _ids(cuda, rows, 8, rows)
        _check(lambda i: joined.slots(x, i), ids, 8, f"mxfp4 rows {rows}")


def test_k4_values_clamp_on_both_paths(cuda):
    from mlxlr8_amd import synth
    from mlxlr8_amd.experts import ExpertLayer
    h, m = 1024, 256
    layer = synth.k4_layer(cuda, 57, hidden=h, intermediate=m, experts=12)
    experts = ExpertLayer(layer["packed"], layer["scales"], h, m)
    for rows in (16, 17):
        say(f"case: K4 values, 12 experts, rows {rows} ({'decode' if rows <= 16 else 'grouped'} path)")
        x, _ = synth.activations(cuda, 58 + rows, rows, hidden=h)
        ids = _ids(cuda, rows, 12, 100 + rows)
        _check(lambda i: experts(x, i), ids, 12, f"k4 rows {rows}")
