"""Residual + RMSNorm and the normed decode layer / layer stack on the MI355X against the oracle."""
import sys

import numpy as np
import pytest
import torch

from conftest import bf16_bits, bits_to_f32, f16_bits, rel_l2

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _norm_weight(device, seed, n):
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return (0.5 + torch.rand(n, generator=g, device=device)).to(torch.bfloat16)


def _bf16_ulps(a_bits, b_bits):
    """Distance in bf16 ulps (sign-magnitude order) between two bf16 bit arrays."""
    def key(b):
        b = np.asarray(b, np.int32)
        return np.where(b & 0x8000, -(b & 0x7FFF), b & 0x7FFF)
    return np.abs(key(a_bits) - key(b_bits))


@pytest.mark.parametrize("rows,n,with_res", [(1, 6144, True), (3, 6144, False), (8, 2048, True), (2, 8192, True)])
def test_residual_rmsnorm_matches_oracle(cuda, orc, rows, n, with_res):
    from mlxlr8_amd.norm import residual_rms_pair
    say(f"case: rmsnorm rows={rows} n={n} residual={with_res}")
    g = torch.Generator(device=cuda)
    g.manual_seed(rows * 100 + n)
    x = torch.randn((rows, n), generator=g, device=cuda).to(torch.bfloat16)
    r = torch.randn((rows, n), generator=g, device=cuda).to(torch.bfloat16) if with_res else None
    w = _norm_weight(cuda, 3, n)
    h, out = residual_rms_pair(x, r, w)
    torch.cuda.synchronize()
    oh, oout = orc.residual_rmsnorm(bf16_bits(x), bf16_bits(r) if r is not None else None, bf16_bits(w))
    np.testing.assert_array_equal(bf16_bits(h).reshape(oh.shape), oh)
    d = _bf16_ulps(bf16_bits(out).reshape(oout.shape), oout)
    # the mean of squares is summed in a different order (fp32 here, fp64 in the oracle): the inverse
    # RMS may differ in its last bits, which moves a rounding boundary for a few elements by one ulp
    assert d.max() <= 1
    assert (d > 0).mean() <= 2e-3


def test_rmsnorm_constant_row_known_answer(cuda):
    from mlxlr8_amd.norm import rms_norm
    say("case: rmsnorm constant row")
    n = 2048
    x = torch.full((1, n), 3.0, device=cuda).to(torch.bfloat16)
    w = torch.full((n,), 0.5, device=cuda).to(torch.bfloat16)
    out = rms_norm(x, w).float()
    # mean(h^2) = 9 -> h * inv = 3 / sqrt(9 + 1e-5) -> bf16 1.0 -> times 0.5
    assert torch.all(out == 0.5)


def _layer(device, seed, hidden, inter):
    from mlxlr8_amd import synth
    from mlxlr8_amd.experts import ExpertLayer
    lay = synth.k4_layer(device, seed, hidden, inter)
    w, bias = synth.router(device, seed, hidden, zipf=True)
    norm = _norm_weight(device, seed + 7, hidden)
    experts = ExpertLayer(lay["packed"], lay["scales"], hidden, inter)
    host = {p: t.cpu().numpy() for p, t in lay["packed"].items()}
    sc = {p: (f16_bits(a), f16_bits(b)) for p, (a, b) in lay["scales"].items()}
    return experts, w, bias, norm, host, sc


def _check_layer(orc, layer, hidden, inter, x_bits, attn_bits, got_out, got_ids, got_scores, tag):
    """Oracle for one normed layer from the GPU layer's own input."""
    experts, w, bias, norm, host, sc = layer
    h, xn = orc.residual_rmsnorm(x_bits, attn_bits, bf16_bits(norm))
    logits = orc.router_logits(xn, w.cpu().numpy())
    oids, oscores = orc.route(logits, bias.cpu().numpy())
    ids = got_ids.astype(np.uint32)
    mism = (ids != oids).any(axis=1)
    if mism.any():
        sig = 1 / (1 + np.exp(-logits.astype(np.float64)))
        choice = sig + bias.cpu().numpy()
        for r in np.where(mism)[0]:
            srt = np.sort(choice[r])[::-1]
            assert srt[7] - srt[8] < 1e-5, f"{tag} row {r}: routing differs without a near tie"
    want = orc.k4_moe(xn, ids, got_scores, h, hidden, inter, host["gate"], host["up"], host["down"],
                      sc["gate"][0], sc["gate"][1], sc["up"][0], sc["up"][1], sc["down"][0], sc["down"][1])
    got = bits_to_f32(got_out)
    wantf = bits_to_f32(want)
    res = bits_to_f32(h)
    err, err_moe = rel_l2(got, wantf), rel_l2(got - res, wantf - res)
    say(f"  {tag}: rel_l2={err:.3e} moe-part rel_l2={err_moe:.3e} routing mismatches={int(mism.sum())}")
    assert err <= 1e-3
    assert err_moe <= 1e-3


def test_layer_decode_small_width(cuda, orc):
    """hidden 2048: the norm runs as its own kernel before the router (non-fused path)."""
    say("case: normed decode layer hidden=2048 rows=3 with attention residual")
    hidden, inter = 2048, 256
    layer = _layer(cuda, 61, hidden, inter)
    g = torch.Generator(device=cuda)
    g.manual_seed(62)
    x = torch.randn((3, hidden), generator=g, device=cuda).to(torch.bfloat16)
    attn = torch.randn((3, hidden), generator=g, device=cuda).to(torch.bfloat16)
    out, ids, scores = layer[0].layer_decode(x, layer[3], layer[1], layer[2], attn=attn)
    torch.cuda.synchronize()
    _check_layer(orc, layer, hidden, inter, bf16_bits(x), bf16_bits(attn), bf16_bits(out), ids.cpu().numpy(),
                 scores.cpu().numpy(), "h2048")


def test_layer_stack_glm(cuda, orc):
    """Two GLM-shaped K4 layers chained as in the 20-layer stack (fused norm in the router)."""
    from mlxlr8_amd.model import DecoderMoELayer, DecoderMoEStack, MoEArgs
    from mlxlr8_amd import synth
    say("case: 2-layer GLM stack rows=1")
    hidden, inter = 6144, 2048
    layers = [_layer(cuda, 300 + i, hidden, inter) for i in range(2)]
    args = MoEArgs()
    mods = [DecoderMoELayer(args, l[3], l[1], l[2], l[0]) for l in layers]
    x, _ = synth.activations(cuda, 77, 1)
    # run layer by layer to keep every layer's input for the oracle
    inputs, h = [], x
    for i, m in enumerate(mods):
        inputs.append(bf16_bits(h))
        out, ids, scores = m.experts.layer_decode(h, m.norm, m.gate, m.bias)
        torch.cuda.synchronize()
        # the module form and a second call reproduce the first bit for bit
        again, _ = m(h)
        assert torch.equal(out.view(torch.int16), again.view(torch.int16))
        _check_layer(orc, layers[i], hidden, inter, inputs[i], None, bf16_bits(out), ids.cpu().numpy(),
                     scores.cpu().numpy(), f"layer {i}")
        h = out
    stacked = DecoderMoEStack(mods)(x)
    assert torch.equal(stacked.view(torch.int16), h.view(torch.int16))


@pytest.mark.parametrize("with_attn", [True, False])
def test_one_row_layer_folds_norm_bit_exact(cuda, with_attn):
    """One GLM row: the layer call forms the residual add + RMSNorm inside the fused block; its
    outputs equal the norm kernel followed by the plain fused block bit for bit (same per-thread
    sums and reduction order), over three consecutive calls."""
    from mlxlr8_amd.norm import residual_rms_pair
    say(f"case: folded norm vs norm kernel + block, attn={with_attn}")
    hidden, inter = 6144, 2048
    experts, w, bias, norm, _, _ = _layer(cuda, 410, hidden, inter)
    g = torch.Generator(device=cuda)
    g.manual_seed(411)
    for step in range(3):
        x = torch.randn((1, hidden), generator=g, device=cuda).to(torch.bfloat16)
        attn = torch.randn((1, hidden), generator=g, device=cuda).to(torch.bfloat16) if with_attn else None
        out, ids, scores = experts.layer_decode(x, norm, w, bias, attn=attn)
        h, xn = residual_rms_pair(x, attn, norm)
        call = experts.prepare_decode(xn, h, w, bias)
        ref = call.run()
        torch.cuda.synchronize()
        assert torch.equal(ids, call.ids), f"step {step}: routing differs"
        assert torch.equal(scores, call.scores), f"step {step}: scores differ"
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), f"step {step}: outputs differ"
