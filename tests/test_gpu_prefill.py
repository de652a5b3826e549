"""Prefill path on the MI355X: sorted work order (bit-exact) and the joined-MXFP4 prefill chunk
(grouped GEMMs on the scaled MX matrix cores) against the oracle."""
import sys

import numpy as np
import pytest
import torch

from conftest import bf16_bits, bits_to_f32, f16_bits, rel_l2

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.mark.parametrize("n,experts,block_rows,skew", [(4608, 257, 128, True), (4608, 257, 8, False),
                                                        (72, 257, 32, False), (1000, 5, 16, True), (0, 7, 8, False),
                                                        (3, 1, 2, False)])
def test_segment_table_matches_oracle(cuda, orc, n, experts, block_rows, skew):
    from mlxlr8_amd.fast_prefill import segment_table
    say(f"case: segment table n={n} experts={experts} block_rows={block_rows} skew={skew}")
    rng = np.random.default_rng(n + experts)
    if skew:
        p = 1.0 / np.arange(1, experts + 1) ** 1.1
        ids = rng.choice(experts, size=n, p=p / p.sum()).astype(np.uint32)
    else:
        ids = rng.integers(0, experts, n).astype(np.uint32)
    order, counts, starts, table = segment_table(torch.from_numpy(ids.astype(np.int32)).to(cuda), experts,
                                                 block_rows)
    oorder, ocounts, ostarts, otable = orc.segment_table(ids, experts, block_rows)
    np.testing.assert_array_equal(counts.cpu().numpy(), ocounts)
    np.testing.assert_array_equal(starts.cpu().numpy(), ostarts)
    np.testing.assert_array_equal(order.cpu().numpy(), oorder)
    np.testing.assert_array_equal(table.cpu().numpy(), otable)
    # invariants: every slot once, segments contiguous and sorted by expert
    if n:
        assert sorted(order.cpu().numpy().tolist()) == list(range(n))
        assert np.all(np.diff(ids[order.cpu().numpy()].astype(np.int64)) >= 0)


def _mx_layer(cuda, seed, hidden, inter):
    from mlxlr8_amd import synth
    from mlxlr8_amd.joined_mxfp4 import JoinedMXFP4
    L = synth.mxfp4_layer(cuda, seed, hidden=hidden, intermediate=inter)
    (gc, gs), (dc, ds) = L["weights"]["gate_up"], L["weights"]["down"]
    side = L["side"]
    joined = JoinedMXFP4(L["weights"], L["unit"],
                         {"gate": (None, side["out_gate"]), "up": (None, side["out_up"]),
                          "down": (side["in_down"], side["out_down"])}, hidden, inter)
    host = dict(gc=gc.cpu().numpy(), gs=gs.cpu().numpy(), dc=dc.cpu().numpy(), ds=ds.cpu().numpy(),
                unit=f16_bits(L["unit"]), og=f16_bits(side["out_gate"]), ou=f16_bits(side["out_up"]),
                idn=f16_bits(side["in_down"]), od=f16_bits(side["out_down"]))
    return joined, host


def _check_prefill(orc, joined, host, hidden, inter, x, res, w, bias, sample):
    out, ids, scores = joined.prefill(x, res, w, bias)
    torch.cuda.synchronize()
    ids = ids.cpu().numpy().astype(np.uint32)
    scores = scores.cpu().numpy()
    xb, rb = bf16_bits(x), bf16_bits(res)
    logits = orc.router_logits(xb, w.cpu().numpy())
    oids, oscores = orc.route(logits, bias.cpu().numpy())
    mism = (ids != oids).any(axis=1)
    if mism.any():
        sig = 1 / (1 + np.exp(-logits.astype(np.float64)))
        choice = sig + bias.cpu().numpy()
        for r in np.where(mism)[0]:
            srt = np.sort(choice[r])[::-1]
            assert srt[7] - srt[8] < 1e-5, f"row {r}: routing differs without a near tie"
    rows = np.asarray(sample)
    want = orc.mxfp4_moe(xb[rows], ids[rows], scores[rows], rb[rows], hidden, inter, host["gc"], host["gs"],
                         host["dc"], host["ds"], host["unit"], host["og"], host["ou"], host["idn"], host["od"])
    got = bits_to_f32(bf16_bits(out))[rows]
    wantf = bits_to_f32(want)
    r = bits_to_f32(rb[rows])
    err, err_moe = rel_l2(got, wantf), rel_l2(got - r, wantf - r)
    counts = np.bincount(ids.ravel(), minlength=257)
    say(f"  rows={x.shape[0]} sampled={len(rows)} experts used={int((counts > 0).sum())} "
        f"max tokens/expert={counts[:256].max()} rel_l2={err:.3e} moe-part={err_moe:.3e} "
        f"routing mismatches={int(mism.sum())}")
    assert err <= 1e-3
    assert err_moe <= 1e-3
    return out


def test_scales_outside_grouped_window(cuda, orc):
    """Block scales outside 114..140 (the window in which the grouped GEMMs' fp16 widening of the
    weights is exact): the layer notices at construction and runs prefill-sized batches through the
    decode GEMVs in chunks of 8 rows, so the result still matches the oracle and equals the 8-row
    chunks computed separately, bit for bit."""
    from mlxlr8_amd import synth
    from mlxlr8_amd.joined_mxfp4 import JoinedMXFP4
    say("case: mxfp4 scales outside the grouped window, rows=20, GLM shape with 16 experts")
    hidden, inter = 6144, 2048   # the decode GEMVs' shape
    L = synth.mxfp4_layer(cuda, 41, hidden=hidden, intermediate=inter, experts=16)
    (gc, gs), (dc, ds) = L["weights"]["gate_up"], L["weights"]["down"]
    gs, ds = gs.clone(), ds.clone()
    gs[3, 5, 0] = 150   # 2^23: e2m1 x scale above the fp16 range
    ds[7, 1, 2] = 100   # 2^-27: below the smallest normal fp16
    side = L["side"]
    joined = JoinedMXFP4({"gate_up": (gc, gs), "down": (dc, ds)}, L["unit"],
                         {"gate": (None, side["out_gate"]), "up": (None, side["out_up"]),
                          "down": (side["in_down"], side["out_down"])}, hidden, inter)
    assert not joined.grouped_exact
    rows = 20
    g = torch.Generator(device=cuda)
    g.manual_seed(5)
    ids = torch.randint(0, joined.experts, (rows, 9), generator=g, device=cuda, dtype=torch.int32)
    ids[:4, 0] = 3
    ids[4:8, 1] = 7
    x, _ = synth.activations(cuda, 43, rows, hidden)
    values = joined.slots(x, ids)
    for r0 in range(0, rows, 8):
        part = joined.slots(x[r0:r0 + 8].contiguous(), ids[r0:r0 + 8].contiguous())
        assert torch.equal(values[r0:r0 + 8].view(torch.int16), part.view(torch.int16))
    host = dict(gc=gc.cpu().numpy(), gs=gs.cpu().numpy(), dc=dc.cpu().numpy(), ds=ds.cpu().numpy())
    res = np.zeros((rows, hidden), np.uint16)
    _, want = orc.mxfp4_moe(bf16_bits(x), ids.cpu().numpy().astype(np.uint32), np.zeros((rows, 8), np.float32), res,
                            hidden, inter, host["gc"], host["gs"], host["dc"], host["ds"], f16_bits(L["unit"]),
                            f16_bits(side["out_gate"]), f16_bits(side["out_up"]), f16_bits(side["in_down"]),
                            f16_bits(side["out_down"]), want_values=True)
    got = bits_to_f32(bf16_bits(values.reshape(rows * 9, hidden)))
    err = rel_l2(got, bits_to_f32(want).reshape(rows * 9, hidden))
    say(f"  rel_l2={err:.3e}")
    assert err <= 1e-3


def test_prefill_small_width(cuda, orc):
    from mlxlr8_amd import synth
    say("case: mxfp4 prefill rows=40 h=2048 m=512")
    hidden, inter = 2048, 512
    joined, host = _mx_layer(cuda, 11, hidden, inter)
    w, bias = synth.router(cuda, 12, hidden, zipf=True)
    x, res = synth.activations(cuda, 13, 40, hidden)
    _check_prefill(orc, joined, host, hidden, inter, x, res, w, bias, range(40))


def test_prefill_config3_glm(cuda, orc):
    """512-token chunk at GLM shapes with Zipf-skewed routing; every 64th row against the oracle."""
    from mlxlr8_amd import synth
    say("case: mxfp4 prefill rows=512 GLM shapes")
    hidden, inter = 6144, 2048
    joined, host = _mx_layer(cuda, 21, hidden, inter)
    w, bias = synth.router(cuda, 22, hidden, zipf=True)
    x, res = synth.activations(cuda, 23, 512, hidden)
    out = _check_prefill(orc, joined, host, hidden, inter, x, res, w, bias, range(0, 512, 64))
    again, _, _ = joined.prefill(x, res, w, bias)
    assert torch.equal(out.view(torch.int16), again.view(torch.int16))
