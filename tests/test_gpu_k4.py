"""K4 trellis path on the MI355X: bit-exact codebook/decode/routing and layer parity with the oracle."""
import sys

import numpy as np
import pytest
import torch

import refmath
from conftest import bf16_bits, bits_to_f32, f16_bits, rel_l2
from test_oracle_router import greedy_route, router_case

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def test_codebook_table_bit_exact(cuda, orc):
    import mlxlr8_amd
    from mlxlr8_amd._lib import check, lib, ptr, stream
    say("case: codebook table")
    t = torch.empty(65536, dtype=torch.uint8, device=cuda)
    check(lib().moe_codebook_e4m3(ptr(t), stream(cuda)))
    torch.cuda.synchronize()
    got = refmath.fp8_e4m3_decode(t.cpu().numpy())
    want = orc.codebook().astype(np.float64)
    np.testing.assert_array_equal(got, want)
    assert mlxlr8_amd.lib() is not None


@pytest.mark.parametrize("side", [1, 2])
def test_decode_inner_bit_exact_small(cuda, orc, side):
    from mlxlr8_amd.trellis import decode_inner
    say(f"case: decode small side={side}")
    rng = np.random.default_rng(11 + side)
    nibs = [rng.integers(0, 16, (16, 24, 256), dtype=np.uint32) for _ in range(2)]
    host = np.concatenate([refmath.build_trellis_matrix(n, side) for n in nibs])
    packed = torch.from_numpy(host).to(cuda)
    for e in range(2):
        got = decode_inner(packed, 4, 256, 384, side, e).cpu().numpy().astype(np.float32)
        np.testing.assert_array_equal(got, refmath.expected_inner(nibs[e]))


@pytest.mark.parametrize("side,in_f,out_f", [(1, 6144, 2048), (2, 2048, 6144)])
def test_decode_inner_bit_exact_glm_shapes(cuda, orc, side, in_f, out_f):
    """The K4 piece decoder of the GEMVs, the fused block and the grouped GEMM, with the
    arithmetic/table mixes those use (1/2, 2/3) and every per-word count, on both code tables."""
    from mlxlr8_amd.trellis import decode_inner
    say(f"case: decode glm side={side}")
    g = torch.Generator(device=cuda)
    g.manual_seed(5 + side)
    packed = torch.randint(0, 256, (3 * in_f * out_f // 2,), generator=g, device=cuda, dtype=torch.uint8)
    host = packed.cpu().numpy()
    for e in (0, 2):
        got = decode_inner(packed, 4, in_f, out_f, side, e).cpu().numpy().astype(np.float32)
        np.testing.assert_array_equal(got, orc.decode(host, 4, in_f, out_f, side, e))


@pytest.mark.parametrize("rows", [1, 2, 4, 8, 33])
@pytest.mark.parametrize("case", ["random", "bias", "ties", "saturated", "zero"])
def test_route_bit_exact(cuda, orc, rows, case):
    from mlxlr8_amd.fast_router import route
    say(f"case: route rows={rows} {case}")
    host, bias = router_case(case, rows)
    ids, scores = route(torch.from_numpy(host).to(cuda), torch.from_numpy(bias).to(cuda))
    ids, scores = ids.cpu().numpy().astype(np.int64), scores.cpu().numpy()
    oids, oscores = orc.route(host, bias)
    np.testing.assert_array_equal(ids, oids.astype(np.int64))
    np.testing.assert_allclose(scores, oscores, rtol=1e-6, atol=1e-7)
    chosen, _ = greedy_route(host, bias)
    np.testing.assert_array_equal(ids[:, :8], chosen)


@pytest.mark.parametrize("rows", [1, 8, 37, 512])
def test_router_logits(cuda, orc, rows):
    from mlxlr8_amd.fast_router import router_logits
    say(f"case: router logits rows={rows}")
    g = torch.Generator(device=cuda)
    g.manual_seed(rows)
    x = torch.randn((rows, 6144), generator=g, device=cuda).to(torch.bfloat16)
    w = torch.randn((256, 6144), generator=g, device=cuda) * 0.02
    got = router_logits(x, w).cpu().numpy()
    want = orc.router_logits(bf16_bits(x), w.cpu().numpy())
    assert np.abs(got - want).max() <= 2e-5 * np.abs(want).max()


def _small_layer(cuda, seed, h=256, m=128, E=4):
    from mlxlr8_amd import synth
    layer = synth.k4_layer(cuda, seed, hidden=h, intermediate=m, experts=E)
    host = {p: t.cpu().numpy() for p, t in layer["packed"].items()}
    sc = {p: (f16_bits(a), f16_bits(b)) for p, (a, b) in layer["scales"].items()}
    return layer, host, sc


@pytest.mark.parametrize("side", [1, 2])
@pytest.mark.parametrize("per_slot", [False, True])
def test_expert_linear_small(cuda, orc, side, per_slot):
    from mlxlr8_amd.trellis import expert_linear
    say(f"case: expert_linear side={side} per_slot={per_slot}")
    layer, host, sc = _small_layer(cuda, 31)
    proj = "down" if side == 2 else "gate"
    in_f, out_f = (128, 256) if side == 2 else (256, 128)
    ids = torch.tensor([[2, 0], [1, 2], [3, 3]], dtype=torch.int32, device=cuda)
    g = torch.Generator(device=cuda)
    g.manual_seed(3)
    shape = (3, 2, in_f) if per_slot else (3, in_f)
    x = torch.randn(shape, generator=g, device=cuda).to(torch.bfloat16)
    ins, outs = layer["scales"][proj]
    y = expert_linear(x, ids, layer["packed"][proj], ins, outs, 4, in_f, out_f, side)
    assert y.shape == (3, 2, out_f) and y.dtype == torch.bfloat16
    xf = bits_to_f32(bf16_bits(x)).reshape(-1, in_f)
    if not per_slot:
        xf = np.repeat(xf, 2, axis=0)
    want = orc.k4_linear(xf, ids.cpu().numpy().ravel(), host[proj], in_f, out_f, side, sc[proj][0], sc[proj][1])
    got = bits_to_f32(bf16_bits(y)).reshape(-1, out_f)
    assert rel_l2(got, want) < 4e-3  # bf16 output rounding only
    np.testing.assert_allclose(got, want, rtol=2 ** -7, atol=1e-6)


@pytest.mark.parametrize("rows", [1, 3, 8])
def test_mlp_values_small(cuda, orc, rows):
    from mlxlr8_amd.fast_decode import fast_expert_mlp
    say(f"case: mlp small rows={rows}")
    layer, host, sc = _small_layer(cuda, 181, E=5)
    rng = np.random.default_rng(rows)
    ids = torch.from_numpy(rng.integers(0, 5, (rows, 9)).astype(np.int32)).to(cuda)
    x = torch.from_numpy(rng.normal(size=(rows, 256)).astype(np.float32)).to(cuda).to(torch.bfloat16)
    values = fast_expert_mlp(x, ids, layer["packed"], layer["scales"], 4, 256, 128)
    res = np.zeros((rows, 256), np.uint16)
    _, want = orc.k4_moe(bf16_bits(x), ids.cpu().numpy(), np.zeros((rows, 8), np.float32), res, 256, 128,
                         host["gate"], host["up"], host["down"],
                         sc["gate"][0], sc["gate"][1], sc["up"][0], sc["up"][1], sc["down"][0], sc["down"][1],
                         want_values=True)
    got = bits_to_f32(bf16_bits(values))
    err = rel_l2(got, bits_to_f32(want))
    say(f"  rel_l2={err:.3e}")
    assert err <= 1e-3


@pytest.fixture(scope="module")
def glm_layer(cuda):
    from mlxlr8_amd import synth
    say("building GLM-shaped K4 layer (257 experts)")
    layer = synth.k4_layer(cuda, 1234)
    w, bias = synth.router(cuda, 1234)
    host = {p: t.cpu().numpy() for p, t in layer["packed"].items()}
    sc = {p: (f16_bits(a), f16_bits(b)) for p, (a, b) in layer["scales"].items()}
    from mlxlr8_amd.experts import ExpertLayer
    experts = ExpertLayer(layer["packed"], layer["scales"], 6144, 2048)
    return experts, layer, host, sc, w, bias


def _check_decode_block(orc, glm_layer, rows, correlated, seed):
    from mlxlr8_amd import synth
    experts, layer, host, sc, w, bias = glm_layer
    x, residual = synth.activations(w.device, seed, rows, correlated=correlated)
    out, ids, scores = experts.decode_block_routes(x, residual, w, bias)
    torch.cuda.synchronize()
    ids = ids.cpu().numpy().astype(np.uint32)
    logits = orc.router_logits(bf16_bits(x), w.cpu().numpy())
    oids, oscores = orc.route(logits, bias.cpu().numpy())
    mism = (ids != oids).any(axis=1)
    if mism.any():
        # only a near tie of corrected scores may flip (logits differ by fp32 summation order)
        sig = 1 / (1 + np.exp(-logits.astype(np.float64)))
        choice = sig + bias.cpu().numpy()
        for r in np.where(mism)[0]:
            srt = np.sort(choice[r])[::-1]
            assert srt[7] - srt[8] < 1e-5, f"row {r}: routing differs without a near tie"
    np.testing.assert_allclose(scores.cpu().numpy()[~mism], oscores[~mism], rtol=2e-6, atol=1e-7)
    want = orc.k4_moe(bf16_bits(x), ids, scores.cpu().numpy(), bf16_bits(residual), 6144, 2048,
                      host["gate"], host["up"], host["down"],
                      sc["gate"][0], sc["gate"][1], sc["up"][0], sc["up"][1], sc["down"][0], sc["down"][1])
    got = bits_to_f32(bf16_bits(out))
    wantf = bits_to_f32(want)
    err = rel_l2(got, wantf)
    # the layer adds a N(0,1) residual; also check the MoE contribution alone
    res = bits_to_f32(bf16_bits(residual))
    err_moe = rel_l2(got - res, wantf - res)
    say(f"  rows={rows} unique={len(np.unique(ids))} rel_l2={err:.3e} moe-part rel_l2={err_moe:.3e}")
    assert err <= 1e-3
    assert err_moe <= 1e-3
    return out


def test_moe_decode_block_config0(cuda, orc, glm_layer):
    say("case: GLM decode block rows=1")
    out = _check_decode_block(orc, glm_layer, 1, False, 7)
    # deterministic: a second call reproduces every bit
    experts, layer, host, sc, w, bias = glm_layer
    from mlxlr8_amd import synth
    x, residual = synth.activations(w.device, 7, 1)
    out2 = experts.decode_block(x, residual, w, bias)
    assert torch.equal(out.view(torch.int16), out2.view(torch.int16))


def test_moe_decode_block_verify_batch(cuda, orc, glm_layer):
    say("case: GLM decode block rows=8 correlated")
    _check_decode_block(orc, glm_layer, 8, True, 21)


@pytest.mark.parametrize("rows", [3, 8])
def test_batch_rows_equal_single_rows(cuda, glm_layer, rows):
    """A token's output does not depend on the batch it is decoded in: every row of a routed
    rows-token decode block equals, bit for bit, the same token decoded alone (ids, scores and the
    combined output).  The reference requires this of its multi-row reuse
    (tests/test_fast_decode.py:218-243); here every output is summed over fixed 128-row parts in
    part order, whatever the batch's units."""
    from mlxlr8_amd import synth
    say(f"case: batch of {rows} rows vs single rows, bit for bit")
    experts, layer, host, sc, w, bias = glm_layer
    x, residual = synth.activations(w.device, 31 + rows, rows, correlated=True)
    out, ids, scores = experts.decode_block_routes(x, residual, w, bias)
    for r in range(rows):
        o1, i1, s1 = experts.decode_block_routes(x[r:r + 1].contiguous(), residual[r:r + 1].contiguous(), w, bias)
        assert torch.equal(ids[r], i1[0]), f"row {r}: ids differ"
        assert torch.equal(scores[r].view(torch.int32), s1[0].view(torch.int32)), f"row {r}: scores differ"
        assert torch.equal(out[r].view(torch.int16), o1[0].view(torch.int16)), f"row {r}: output differs"


@pytest.mark.parametrize("rows", [2, 3, 4, 8])
@pytest.mark.parametrize("pattern", ["shared", "all", "changing", "duplicates"])
def test_values_batch_equals_single_rows(cuda, glm_layer, rows, pattern):
    """The reference's id patterns for multi-row reuse (tests/test_fast_decode.py:218-243): rows
    sharing only the shared expert, rows using the same nine experts in rotated order, overlapping
    windows, and ids repeated inside a row.  Each row's nine slot values from the batch equal the
    row's values computed alone, bit for bit."""
    say(f"case: values rows={rows} pattern={pattern} vs single rows")
    experts, layer, host, sc, w, bias = glm_layer
    if pattern == "shared":
        routed = np.arange(rows * 8).reshape(rows, 8)
        ids = np.concatenate([routed, np.full((rows, 1), 256)], axis=-1)
    elif pattern == "all":
        ids = np.stack([np.roll(np.arange(9), r) for r in range(rows)])
    elif pattern == "changing":
        routed = np.stack([np.arange(r * 4, r * 4 + 8) for r in range(rows)])
        ids = np.concatenate([routed, np.full((rows, 1), 256)], axis=-1)
    else:
        ids = np.tile([0, 0, 1, 1, 2, 2, 0, 1, 2], (rows, 1))
    ids = torch.tensor(ids, dtype=torch.int32, device=cuda)
    g = torch.Generator(device=cuda)
    g.manual_seed(431 + rows)
    x = torch.randn((rows, 6144), generator=g, device=cuda).to(torch.bfloat16)
    values = experts(x, ids)
    for r in range(rows):
        v1 = experts(x[r:r + 1].contiguous(), ids[r:r + 1].contiguous())
        assert torch.equal(values[r].view(torch.int16), v1[0].view(torch.int16)), f"row {r} differs"


def test_two_streams_keep_separate_scratch(cuda, glm_layer):
    """Decode calls prepared on two streams use separate workspaces, so interleaved launches on the
    two streams reproduce the single-stream results bit for bit."""
    from mlxlr8_amd import synth
    say("case: decode on two streams")
    experts, layer, host, sc, w, bias = glm_layer
    x, r = synth.activations(w.device, 55, 2)
    want = [experts.decode_block(x[i:i + 1].contiguous(), r[i:i + 1].contiguous(), w, bias)[0] for i in range(2)]
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    calls = []
    for i, st in enumerate(streams):
        with torch.cuda.stream(st):
            calls.append(experts.prepare_decode(x[i:i + 1].contiguous(), r[i:i + 1].contiguous(), w, bias))
    torch.cuda.synchronize()
    for _ in range(10):
        for c in calls:
            c.run()
    torch.cuda.synchronize()
    for i in range(2):
        assert torch.equal(calls[i].out.reshape(-1).view(torch.int16), want[i].reshape(-1).view(torch.int16))


def test_mlp_values_glm(cuda, orc, glm_layer):
    from mlxlr8_amd.fast_decode import fast_expert_mlp
    say("case: GLM values rows=2")
    experts, layer, host, sc, w, bias = glm_layer
    ids = torch.tensor([[5, 17, 256, 40, 5, 99, 1, 2, 3], [17, 0, 256, 250, 7, 8, 9, 10, 11]],
                       dtype=torch.int32, device=cuda)
    g = torch.Generator(device=cuda)
    g.manual_seed(9)
    x = torch.randn((2, 6144), generator=g, device=cuda).to(torch.bfloat16)
    values = experts(x, ids)
    res = np.zeros((2, 6144), np.uint16)
    _, want = orc.k4_moe(bf16_bits(x), ids.cpu().numpy(), np.zeros((2, 8), np.float32), res, 6144, 2048,
                         host["gate"], host["up"], host["down"],
                         sc["gate"][0], sc["gate"][1], sc["up"][0], sc["up"][1], sc["down"][0], sc["down"][1],
                         want_values=True)
    err = rel_l2(bits_to_f32(bf16_bits(values)), bits_to_f32(want))
    say(f"  rel_l2={err:.3e}")
    assert err <= 1e-3
    assert values.shape == (2, 9, 6144)


@pytest.mark.parametrize("rows", [1, 3])
def test_large_activations_stay_exact(cuda, orc, glm_layer, rows):
    """Activations whose transformed blocks reach 2^15 and beyond (the fp16 hi row of the staged
    input tops out at 65504; the reference computes in fp32): such a block is staged scaled by a
    power of two and its partial sums are scaled back, so the slot values still match the oracle to
    the usual bar.  An unguarded fp16 conversion would give inf."""
    say(f"case: large activations rows={rows}")
    experts, layer, host, sc, w, bias = glm_layer
    ids = torch.tensor([[5, 17, 256, 40, 99, 1, 2, 3, 4], [17, 0, 256, 250, 7, 8, 9, 10, 11],
                        [200, 201, 256, 5, 17, 30, 31, 32, 33]][:rows], dtype=torch.int32, device=cuda)
    g = torch.Generator(device=cuda)
    g.manual_seed(97 + rows)
    x = (torch.randn((rows, 6144), generator=g, device=cuda) * 3.0e4).to(torch.bfloat16)
    values = experts(x, ids)
    assert torch.isfinite(values.float()).all()
    res = np.zeros((rows, 6144), np.uint16)
    _, want = orc.k4_moe(bf16_bits(x), ids.cpu().numpy(), np.zeros((rows, 8), np.float32), res, 6144, 2048,
                         host["gate"], host["up"], host["down"],
                         sc["gate"][0], sc["gate"][1], sc["up"][0], sc["up"][1], sc["down"][0], sc["down"][1],
                         want_values=True)
    err = rel_l2(bits_to_f32(bf16_bits(values)), bits_to_f32(want))
    say(f"  rel_l2={err:.3e}")
    assert err <= 1e-3


def test_fp32_accumulation_known_answer(cuda):
    """Known answer of the reference (tests/golden, from its tests/test_fast_prefill.py:208-228): an
    all-zero K4 bitstream decodes to codebook[0] = 1.875 everywhere, so with unit scales and one
    spike per 128-block the inner sum (6144 * 1.875 * spike / sqrt(128)) exceeds the fp16 range;
    after the output H128 all of it sits in column 0 and the other columns are exactly zero."""
    import json
    from pathlib import Path
    from mlxlr8_amd.trellis import expert_linear
    say("case: fp32 accumulation known answer")
    g = json.loads((Path(__file__).parent / "golden" / "reference_known_answers.json").read_text())["fp32_accumulation"]
    w, n = g["width"], g["output"]
    packed = torch.zeros(w * n // 2, dtype=torch.uint8, device=cuda)
    x = torch.zeros((1, w), dtype=torch.float32, device=cuda)
    x[0, ::128] = g["spike"]
    x = x.to(torch.bfloat16)  # activations are bf16 here: the spike rounds to bf16
    spike = float(x[0, 0])
    ones_in = torch.ones((1, w), dtype=torch.float16, device=cuda)
    ones_out = torch.ones((1, n), dtype=torch.float16, device=cuda)
    ids = torch.zeros((1, 1), dtype=torch.int32, device=cuda)
    y = expert_linear(x, ids, packed, ones_in, ones_out, 4, w, n, 1).float().cpu().numpy().reshape(-1)
    inner = w * 1.875 * spike / np.sqrt(128)
    assert inner > g["fp16_max"]
    want0 = w * 1.875 * spike
    say(f"  col0={y[0]} want={want0} max|other|={np.abs(y[1:]).max()}")
    assert abs(y[0] - want0) <= want0 * 2.0 ** -8
    assert np.all(y[1:] == 0.0)


@pytest.mark.parametrize("k", [2, 3])
@pytest.mark.parametrize("side", [1, 2])
def test_decode_inner_k2_k3_bit_exact(cuda, orc, k, side):
    """The K2 / K3 trellis decode (the MTP layer's K3 experts): brute-force symbols and the oracle.
    K3 runs the fused decode block's piece decoder (decode_k3_pair_words) with its arithmetic/table
    mix on the small matrix and five mixes across the GLM-size one, so that decoder is pinned bit
    for bit; K2 runs the per-codeword reference decode."""
    from mlxlr8_amd.trellis import decode_inner
    say(f"case: decode k={k} side={side}")
    rng = np.random.default_rng(60 + 10 * k + side)
    syms = [rng.integers(0, 1 << k, (8, 16, 256), dtype=np.uint32) for _ in range(2)]
    host = np.concatenate([refmath.build_trellis_matrix(s, side, k) for s in syms])
    packed = torch.from_numpy(host).to(cuda)
    for e in range(2):
        got = decode_inner(packed, k, 128, 256, side, e).cpu().numpy().astype(np.float32)
        np.testing.assert_array_equal(got, refmath.expected_inner(syms[e], k))
        np.testing.assert_array_equal(got, orc.decode(host, k, 128, 256, side, e))
    # GLM-size K3 matrix against the oracle
    g = torch.Generator(device=cuda)
    g.manual_seed(70 + k)
    big = torch.randint(0, 256, (6144 * 2048 * k // 8,), generator=g, device=cuda, dtype=torch.uint8)
    in_f, out_f = (6144, 2048) if side == 1 else (2048, 6144)
    got = decode_inner(big, k, in_f, out_f, side, 0).cpu().numpy().astype(np.float32)
    np.testing.assert_array_equal(got, orc.decode(big.cpu().numpy(), k, in_f, out_f, side, 0))
