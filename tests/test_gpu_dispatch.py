"""The drop-in entry points dispatch prefill-sized batches as the reference does (MI355X).

* ``MoEBlock`` (exlr8/model.py:385-418) on joined-MXFP4 experts with a 512-token chunk runs the
  one-call grouped prefill (router, sorted grouped MX-MFMA GEMMs, combine); every one of the 512
  rows is checked against the oracle.
* ``MoEBlock`` on K4 experts with 40 rows routes, runs the grouped trellis MLP
  (exlr8/experts.py:170-175: more than 16 rows) and combines; every row is checked.
* ``JoinedMXFP4.slots`` beyond 8 rows takes the grouped GEMM (exlr8/joined_mxfp4.py:98-113).
* Resident decode never synchronises with the host (exlr8 tests/test_experts.py:121-136).
"""
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from conftest import bf16_bits, bits_to_f32, f16_bits, rel_l2
from gpu_helpers import check_routing, oracle_k4, say

pytestmark = pytest.mark.gpu

H, M = 6144, 2048


def _mx(cuda, seed, experts=257):
    from mlxlr8_amd import synth
    from mlxlr8_amd.joined_mxfp4 import JoinedMXFP4
    L = synth.mxfp4_layer(cuda, seed, experts=experts)
    side = L["side"]
    joined = JoinedMXFP4(L["weights"], L["unit"], {"gate": (None, side["out_gate"]), "up": (None, side["out_up"]),
                                                   "down": (side["in_down"], side["out_down"])}, H, M)
    return joined, L


def _mx_host(L):
    (gc, gs), (dc, ds) = L["weights"]["gate_up"], L["weights"]["down"]
    side = L["side"]
    return dict(gc=gc.cpu().numpy(), gs=gs.cpu().numpy(), dc=dc.cpu().numpy(), ds=ds.cpu().numpy(),
                unit=f16_bits(L["unit"]), og=f16_bits(side["out_gate"]), ou=f16_bits(side["out_up"]),
                idn=f16_bits(side["in_down"]), od=f16_bits(side["out_down"]))


def _mx_oracle(orc, host, x_bits, ids, scores, res_bits, want_values=False):
    return orc.mxfp4_moe(x_bits, ids, scores, res_bits, H, M, host["gc"], host["gs"], host["dc"], host["ds"],
                         host["unit"], host["og"], host["ou"], host["idn"], host["od"], want_values=want_values)


def test_moe_block_prefill_mxfp4_every_row(cuda, orc):
    """The 512-token prefill workload (Zipf-skewed routing) through MoEBlock: all rows vs the oracle."""
    from mlxlr8_amd import synth
    from mlxlr8_amd.fast_router import route, router_logits
    from mlxlr8_amd.model import MoEArgs, MoEBlock
    say("case: MoEBlock 512-row prefill, joined MXFP4, every row")
    joined, L = _mx(cuda, 21)
    w, bias = synth.router(cuda, 22, zipf=True)
    x, res = synth.activations(cuda, 23, 512)
    block = MoEBlock(MoEArgs(), w, bias, SimpleNamespace(affine=joined, k=4, hidden=H, intermediate=M))
    out = block(x, res)
    again = block(x, res)
    ids, scores = route(router_logits(x, w), bias)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), again.view(torch.int16))
    ids = ids.cpu().numpy().astype(np.uint32)
    mism = check_routing(orc, x, w, bias, ids, "prefill")
    counts = np.bincount(ids.ravel(), minlength=257)
    want = _mx_oracle(orc, _mx_host(L), bf16_bits(x), ids, scores.cpu().numpy(), bf16_bits(res))
    got, wantf, r = bits_to_f32(bf16_bits(out)), bits_to_f32(want), bits_to_f32(bf16_bits(res))
    err, err_moe = rel_l2(got, wantf), rel_l2(got - r, wantf - r)
    row_err = np.linalg.norm(got - wantf, axis=1) / np.linalg.norm(wantf, axis=1)
    say(f"  experts used={int((counts > 0).sum())} max tokens/expert={counts[:256].max()} rel_l2={err:.3e} "
        f"moe-part={err_moe:.3e} worst row={row_err.max():.3e} routing mismatches={int(mism.sum())}")
    assert err <= 1e-3 and err_moe <= 1e-3
    assert row_err.max() <= 2e-3


def test_joined_slots_grouped_beyond_decode_rows(cuda, orc):
    from mlxlr8_amd import synth
    say("case: JoinedMXFP4.slots rows=40 (grouped GEMM)")
    joined, L = _mx(cuda, 31, experts=17)
    g = torch.Generator(device="cpu").manual_seed(32)
    ids = torch.randint(0, 17, (40, 9), generator=g, dtype=torch.int32)
    x, _ = synth.activations(cuda, 33, 40)
    values = joined.slots(x, ids.to(cuda))
    torch.cuda.synchronize()
    _, want = _mx_oracle(orc, _mx_host(L), bf16_bits(x), ids.numpy().astype(np.uint32),
                         np.zeros((40, 8), np.float32), np.zeros((40, H), np.uint16), want_values=True)
    err = rel_l2(bits_to_f32(bf16_bits(values)), bits_to_f32(want))
    say(f"  rel_l2={err:.3e}")
    assert values.shape == (40, 9, H) and err <= 1e-3


def test_moe_block_k4_grouped_rows(cuda, orc):
    """40 rows of the K4 layer through MoEBlock: route, grouped trellis MLP, combine (every row)."""
    from mlxlr8_amd import synth
    from mlxlr8_amd.experts import ExpertLayer
    from mlxlr8_amd.fast_router import route, router_logits
    from mlxlr8_amd.model import MoEArgs, MoEBlock
    say("case: MoEBlock 40 rows, K4 grouped")
    spec = synth.k4_layer(cuda, 1234)
    experts = ExpertLayer(**spec, hidden=H, intermediate=M)
    w, bias = synth.router(cuda, 41, zipf=True)
    x, res = synth.activations(cuda, 42, 40)
    out = MoEBlock(MoEArgs(), w, bias, experts)(x, res)
    ids, scores = route(router_logits(x, w), bias)
    torch.cuda.synchronize()
    ids = ids.cpu().numpy().astype(np.uint32)
    check_routing(orc, x, w, bias, ids, "k4 grouped")
    want = oracle_k4(orc, bf16_bits(x), ids, scores.cpu().numpy(), bf16_bits(res), spec["packed"], spec["scales"],
                     H, M)
    got, wantf, r = bits_to_f32(bf16_bits(out)), bits_to_f32(want), bits_to_f32(bf16_bits(res))
    err, err_moe = rel_l2(got, wantf), rel_l2(got - r, wantf - r)
    say(f"  rel_l2={err:.3e} moe-part={err_moe:.3e}")
    assert err <= 1e-3 and err_moe <= 1e-3


def test_resident_decode_never_synchronises(cuda):
    """The decode entry points enqueue work only: no torch operation in them synchronises
    (exlr8 tests/test_experts.py:121-136 checks the same for its resident path)."""
    from mlxlr8_amd import synth
    from mlxlr8_amd.experts import ExpertLayer
    from mlxlr8_amd.fast_decode import fast_expert_mlp
    from mlxlr8_amd.model import MoEArgs, MoEBlock
    say("case: no host synchronisation in decode")
    experts = ExpertLayer(**synth.k4_layer(cuda, 77, experts=257), hidden=H, intermediate=M)
    joined, _ = _mx(cuda, 78)
    w, bias = synth.router(cuda, 79)
    xs = [synth.activations(cuda, 80 + r, r) for r in (1, 8)]
    ids = torch.randint(0, 257, (3, 9), device=cuda, dtype=torch.int32)
    k4_block = MoEBlock(MoEArgs(), w, bias, experts)
    mx_block = MoEBlock(MoEArgs(), w, bias, SimpleNamespace(affine=joined, k=4, hidden=H, intermediate=M))
    # first calls allocate workspaces and load the library
    for x, r in xs:
        k4_block(x, r)
        mx_block(x, r)
    fast_expert_mlp(xs[0][0].expand(3, H).contiguous(), ids, experts.packed, experts.scales, 4, H, M)
    torch.cuda.synchronize()
    torch.cuda.set_sync_debug_mode("error")
    try:
        for x, r in xs:
            k4_block(x, r)
            mx_block(x, r)
            experts.decode_block(x, r, w, bias)
        fast_expert_mlp(xs[0][0].expand(3, H).contiguous(), ids, experts.packed, experts.scales, 4, H, M)
        joined.slots(xs[1][0][:3], ids)
    finally:
        torch.cuda.set_sync_debug_mode("default")
    torch.cuda.synchronize()
