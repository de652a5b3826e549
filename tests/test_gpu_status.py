"""Stalled-launch reporting of the fused decode blocks (moe_decode_status): with the cross-wave
wait bound set to one poll from the host, waits give up early -- every kernel still exits normally,
its outputs are then unreliable -- and the launches are counted in the workspace; with the default
bound restored the count stays zero and the outputs equal a launch made before.  Nothing here makes
a kernel fault: an exhausted wait only lets the wave go on with the words it has (indices clamped)."""
import pytest
import torch

from gpu_helpers import say

pytestmark = pytest.mark.gpu


def _bits(t):
    return t.contiguous().view(torch.uint8)


def _forced_stall_then_recovery(run, label):
    from mlxlr8_amd._lib import set_wait_bound, stalled_launches
    torch.cuda.synchronize()
    assert stalled_launches() == 0
    good = run().clone()
    torch.cuda.synchronize()
    assert stalled_launches() == 0, f"{label}: a launch stalled with the default wait bound"
    stalled = 0
    try:
        set_wait_bound(1)
        for _ in range(4):
            run()
            torch.cuda.synchronize()
            stalled += stalled_launches()
            if stalled:
                break
    finally:
        set_wait_bound(0)
    say(f"{label}: launches reported stalled under a one-poll bound: {stalled}")
    assert stalled >= 1, f"{label}: no launch was reported although every wait was bounded to one poll"
    again = run()
    torch.cuda.synchronize()
    assert stalled_launches() == 0, f"{label}: the count did not reset"
    assert torch.equal(_bits(again), _bits(good)), f"{label}: outputs after recovery differ"


def test_k4_block_reports_stalled_waits(cuda):
    from mlxlr8_amd import synth
    from mlxlr8_amd.experts import ExpertLayer
    say("case: fused K4 block, h 1024 m 256, one row, wait bound 1 poll")
    h, m = 1024, 256
    layer = synth.k4_layer(cuda, 31, hidden=h, intermediate=m)
    w, bias = synth.router(cuda, 31, hidden=h)
    x, residual = synth.activations(cuda, 31, 1, hidden=h)
    experts = ExpertLayer(layer["packed"], layer["scales"], h, m)
    _forced_stall_then_recovery(lambda: experts.decode_block_routes(x, residual, w, bias)[0], "k4")


def test_mxfp4_block_reports_stalled_waits(cuda):
    from mlxlr8_amd import synth
    from mlxlr8_amd.joined_mxfp4 import JoinedMXFP4
    say("case: fused joined-MXFP4 block, GLM shape, one row, wait bound 1 poll")
    L = synth.mxfp4_layer(cuda, 37)
    w, bias = synth.router(cuda, 37)
    x, residual = synth.activations(cuda, 37, 1)
    side = L["side"]
    joined = JoinedMXFP4(L["weights"], L["unit"], {"gate": (None, side["out_gate"]), "up": (None, side["out_up"]),
                                                   "down": (side["in_down"], side["out_down"])}, 6144, 2048)
    _forced_stall_then_recovery(lambda: joined.decode_block(x, residual, w, bias)[0], "mxfp4")
