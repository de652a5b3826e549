"""Joined-MXFP4 expert path on the MI355X against the CPU oracle (config-1 shapes)."""
import sys

import numpy as np
import pytest
import torch

from conftest import bf16_bits, bits_to_f32, f16_bits, rel_l2

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _layer(cuda, experts, seed, edit_scales=None):
    from mlxlr8_amd import synth
    from mlxlr8_amd.joined_mxfp4 import JoinedMXFP4
    L = synth.mxfp4_layer(cuda, seed, experts=experts)
    (gc, gs), (dc, ds) = L["weights"]["gate_up"], L["weights"]["down"]
    if edit_scales is not None:
        edit_scales(gs, ds)
    side = L["side"]
    joined = JoinedMXFP4(L["weights"], L["unit"],
                         {"gate": (None, side["out_gate"]), "up": (None, side["out_up"]),
                          "down": (side["in_down"], side["out_down"])}, 6144, 2048)
    host = dict(gc=gc.cpu().numpy(), gs=gs.cpu().numpy(), dc=dc.cpu().numpy(), ds=ds.cpu().numpy(),
                unit=f16_bits(L["unit"]), og=f16_bits(side["out_gate"]), ou=f16_bits(side["out_up"]),
                idn=f16_bits(side["in_down"]), od=f16_bits(side["out_down"]))
    return joined, host


def _oracle(orc, host, x, ids, scores, residual):
    return orc.mxfp4_moe(bf16_bits(x), ids, scores, residual, 6144, 2048, host["gc"], host["gs"], host["dc"],
                         host["ds"], host["unit"], host["og"], host["ou"], host["idn"], host["od"], want_values=True)


@pytest.fixture(scope="module")
def small(cuda):
    say("building 5-expert MXFP4 layer")
    return _layer(cuda, 5, 77)


@pytest.mark.parametrize("rows", [1, 3])
def test_mxfp4_slots_values(cuda, orc, small, rows):
    say(f"case: mxfp4 slots rows={rows}")
    joined, host = small
    rng = np.random.default_rng(rows)
    ids = torch.from_numpy(rng.integers(0, 5, (rows, 9)).astype(np.int32)).to(cuda)
    x = torch.from_numpy(rng.normal(size=(rows, 6144)).astype(np.float32)).to(cuda).to(torch.bfloat16)
    values = joined.slots(x, ids)
    _, want = _oracle(orc, host, x, ids.cpu().numpy(), np.zeros((rows, 8), np.float32),
                      np.zeros((rows, 6144), np.uint16))
    err = rel_l2(bits_to_f32(bf16_bits(values)), bits_to_f32(want))
    say(f"  rel_l2={err:.3e}")
    assert values.shape == (rows, 9, 6144)
    assert err <= 1e-3


@pytest.mark.parametrize("rows", [1, 2, 8])
def test_mxfp4_finish(cuda, orc, small, rows):
    say(f"case: mxfp4 finish rows={rows}")
    joined, host = small
    rng = np.random.default_rng(100 + rows)
    ids = rng.integers(0, 4, (rows, 9)).astype(np.int32)
    ids[:, 8] = 4
    scores = rng.uniform(.03, .4, (rows, 8)).astype(np.float32)
    x = torch.from_numpy(rng.normal(size=(rows, 6144)).astype(np.float32)).to(cuda).to(torch.bfloat16)
    res = torch.from_numpy(rng.normal(size=(rows, 6144)).astype(np.float32)).to(cuda).to(torch.bfloat16)
    out = joined.finish(x, torch.from_numpy(ids).to(cuda), torch.from_numpy(scores).to(cuda), res)
    want, _ = _oracle(orc, host, x, ids, scores, bf16_bits(res))
    got = bits_to_f32(bf16_bits(out))
    err = rel_l2(got, bits_to_f32(want))
    r = bits_to_f32(bf16_bits(res))
    err_moe = rel_l2(got - r, bits_to_f32(want) - r)
    say(f"  rel_l2={err:.3e} moe-part={err_moe:.3e}")
    assert err <= 1e-3 and err_moe <= 1e-3


def test_mxfp4_config1_full_layer(cuda, orc):
    """257 experts, batch 1, routed by the GPU router; parity of the whole block."""
    from mlxlr8_amd import synth
    from mlxlr8_amd.fast_router import route, router_logits
    say("case: mxfp4 config 1 full layer")
    joined, host = _layer(cuda, 257, 4242)
    w, bias = synth.router(cuda, 4242)
    x, res = synth.activations(cuda, 4242, 1)
    ids, scores = route(router_logits(x, w), bias)
    out = joined.finish(x, ids, scores, res)
    want, _ = _oracle(orc, host, x, ids.cpu().numpy(), scores.cpu().numpy(), bf16_bits(res))
    err = rel_l2(bits_to_f32(bf16_bits(out)), bits_to_f32(want))
    say(f"  rel_l2={err:.3e}")
    assert err <= 1e-3


def test_mxfp4_decode_block_one_call(cuda, orc):
    """Router + route + MXFP4 MLP + combine in one library call, rows 1 and 8 (config 1 path)."""
    from mlxlr8_amd import synth
    say("case: mxfp4 decode block (one call) rows=1,8")
    joined, host = _layer(cuda, 257, 515)
    w, bias = synth.router(cuda, 515)
    for rows in (1, 8):
        x, res = synth.activations(cuda, 516 + rows, rows)
        out, ids, scores = joined.decode_block(x, res, w, bias)
        torch.cuda.synchronize()
        logits = orc.router_logits(bf16_bits(x), w.cpu().numpy())
        oids, _ = orc.route(logits, bias.cpu().numpy())
        got_ids = ids.cpu().numpy().astype(np.uint32)
        mism = (got_ids != oids).any(axis=1)
        if mism.any():
            sig = 1 / (1 + np.exp(-logits.astype(np.float64)))
            choice = sig + bias.cpu().numpy()
            for r in np.where(mism)[0]:
                srt = np.sort(choice[r])[::-1]
                assert srt[7] - srt[8] < 1e-5, f"row {r}: routing differs without a near tie"
        want, _ = _oracle(orc, host, x, got_ids, scores.cpu().numpy(), bf16_bits(res))
        got = bits_to_f32(bf16_bits(out))
        r = bits_to_f32(bf16_bits(res))
        err, err_moe = rel_l2(got, bits_to_f32(want)), rel_l2(got - r, bits_to_f32(want) - r)
        say(f"  rows={rows} rel_l2={err:.3e} moe-part={err_moe:.3e} routing mismatches={int(mism.sum())}")
        assert err <= 1e-3 and err_moe <= 1e-3
        again, _, _ = joined.decode_block(x, res, w, bias)
        assert torch.equal(out.view(torch.int16), again.view(torch.int16))


def test_mxfp4_fused_block_equals_three_launch_path(cuda):
    """One-row decode runs the single-launch block (router, both projections, combine); given the
    ids and scores it routed, the three-launch finish produces the same output bits, call after
    call (the block's words are tagged per launch, so replays never read stale values)."""
    from mlxlr8_amd import synth
    say("case: mxfp4 fused one-row block vs three-launch finish")
    joined, _ = _layer(cuda, 257, 6161)
    w, bias = synth.router(cuda, 6161)
    for seed in range(4):
        x, res = synth.activations(cuda, 6200 + seed, 1)
        out, ids, scores = joined.decode_block(x, res, w, bias)
        ref = joined.finish(x, ids, scores, res)
        torch.cuda.synchronize()
        same = torch.equal(out.view(torch.int16), ref.view(torch.int16))
        say(f"  seed={seed} ids={ids.cpu().numpy().tolist()} identical={same}")
        assert same


def test_mxfp4_fused_block_scales_outside_exact_window(cuda, orc):
    """e8m0 scale bytes far from the synthetic layers' (whose fp16 widening, as in the grouped
    prefill GEMMs, would overflow or flush): gate/up groups at 2^14 dominate their rows, down groups
    at 2^-14 and 2^14 mix with ordinary ones; the one-row block (fp32 products for every scale)
    still matches the oracle."""
    from mlxlr8_amd import synth

    def edit(gs, ds):
        r = torch.arange(gs.shape[1], device=gs.device)[:, None]
        g = torch.arange(gs.shape[2], device=gs.device)[None, :]
        gs[:, (r + g) % 13 == 0] = 141
        r = torch.arange(ds.shape[1], device=ds.device)[:, None]
        g = torch.arange(ds.shape[2], device=ds.device)[None, :]
        ds[:, (3 * r + g) % 11 == 0] = 113
        ds[:, (r + 2 * g) % 17 == 0] = 141

    say("case: mxfp4 fused block, scales outside the exact window")
    joined, host = _layer(cuda, 257, 7171, edit)
    assert not joined.grouped_exact
    w, bias = synth.router(cuda, 7171)
    x, res = synth.activations(cuda, 7172, 1)
    out, ids, scores = joined.decode_block(x, res, w, bias)
    torch.cuda.synchronize()
    want, _ = _oracle(orc, host, x, ids.cpu().numpy(), scores.cpu().numpy(), bf16_bits(res))
    got = bits_to_f32(bf16_bits(out))
    r = bits_to_f32(bf16_bits(res))
    err, err_moe = rel_l2(got, bits_to_f32(want)), rel_l2(got - r, bits_to_f32(want) - r)
    say(f"  rel_l2={err:.3e} moe-part={err_moe:.3e} max|out|={np.abs(got).max():.3e}")
    assert np.isfinite(got).all() and err <= 1e-3 and err_moe <= 1e-3
