"""The plain (unfused) operator chain on the MI355X: SwiGLU, the dense trellis inspection and
linear entries, and ExpertLayer with ``store.optimize = False`` (exlr8/experts.py:176-188)."""
import sys

import numpy as np
import pytest
import torch

import refmath
from conftest import bf16_bits, bits_to_f32, f16_bits, rel_l2

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _bf16(rng, shape, scale=1.0):
    return torch.from_numpy((rng.standard_normal(shape) * scale).astype(np.float32)).to(torch.bfloat16)


@pytest.mark.parametrize("n", [8, 1003, 70000])
def test_swiglu_bit_exact(cuda, orc, n):
    from mlxlr8_amd.trellis import swiglu
    say(f"case: swiglu n={n}")
    rng = np.random.default_rng(n)
    gate, up = _bf16(rng, n, 4.0), _bf16(rng, n, 2.0)
    gate[: min(n, 4)] = torch.tensor([0.0, -30.0, 30.0, 1e-3][: min(n, 4)])
    got = swiglu(gate.to(cuda), up.to(cuda)).cpu()
    want = orc.swiglu_bf16(bits_to_f32(bf16_bits(gate)), bits_to_f32(bf16_bits(up)))
    np.testing.assert_array_equal(bits_to_f32(bf16_bits(got)), want)
    # in place over the gate array gives the same bits
    g2 = gate.to(cuda)
    from mlxlr8_amd._lib import check, lib, ptr, stream
    u2 = up.to(cuda)
    check(lib().moe_swiglu_bf16(ptr(g2), ptr(u2), n, ptr(g2), stream(cuda)))
    assert torch.equal(g2.cpu(), got)


def _dense_oracle(orc, host, k, in_f, out_f, side, suh, svh):
    """float64 public matrix [out, in] from the oracle's inner decode and the Sylvester Hadamard."""
    inner = orc.decode(host, k, in_f, out_f, side, 0).astype(np.float64)          # [in, out]
    a = refmath.block_hadamard(inner)                                            # H along out
    w = refmath.block_hadamard(np.ascontiguousarray(a.T))                        # [out, in], H along in
    return w * svh.astype(np.float64)[:, None] * suh.astype(np.float64)[None, :]


@pytest.mark.parametrize("k", [2, 3, 4])
@pytest.mark.parametrize("side", [1, 2])
def test_dequantize_and_trellis_linear(cuda, orc, k, side):
    """dequantize_trellis against the oracle's dense public matrix, and trellis_linear against x @ W^T
    of that matrix (exlr8/trellis.py:157-214)."""
    from mlxlr8_amd.trellis import dequantize_trellis, trellis_linear
    in_f, out_f = (256, 384) if side == 1 else (384, 256)
    say(f"case: dense trellis k={k} side={side} {in_f}x{out_f}")
    rng = np.random.default_rng(10 * k + side)
    host = rng.integers(0, 256, in_f * out_f * k // 8, dtype=np.uint8)
    signs = lambda n: np.where(rng.random(n) < 0.5, -1.0, 1.0)
    suh = (signs(in_f) * rng.uniform(0.5, 1.5, in_f)).astype(np.float16)
    svh = (signs(out_f) * rng.uniform(0.01, 0.03, out_f)).astype(np.float16)
    packed = torch.from_numpy(host).to(cuda)
    suh_t, svh_t = torch.from_numpy(suh).to(cuda), torch.from_numpy(svh).to(cuda)
    want = _dense_oracle(orc, host, k, in_f, out_f, side, suh, svh)
    got = dequantize_trellis(packed, suh_t, svh_t, k, in_f, out_f, side).cpu().numpy()
    assert got.shape == (out_f, in_f)
    np.testing.assert_allclose(got, want, rtol=0, atol=2e-6 * np.abs(want).max())
    x = _bf16(rng, (5, in_f))
    y = trellis_linear(x.to(cuda), packed, suh_t, svh_t, k, in_f, out_f, side)
    assert y.shape == (5, out_f) and y.dtype == torch.bfloat16
    exact = bits_to_f32(bf16_bits(x)).astype(np.float64) @ want.T
    np.testing.assert_allclose(bits_to_f32(bf16_bits(y.cpu())), exact, rtol=2 ** -7, atol=1e-5 * np.abs(exact).max())


def _chain_oracle(orc, x, ids, host, sc, k, h, m):
    """gate/up expert linears, typed SwiGLU, down expert linear, all on the oracle."""
    rows, slots = ids.shape
    xf = np.repeat(bits_to_f32(bf16_bits(x)).reshape(rows, h), slots, axis=0)
    flat = ids.reshape(-1)
    g = orc.k4_linear(xf, flat, host["gate"], h, m, 1, *sc["gate"], k=k)
    u = orc.k4_linear(xf, flat, host["up"], h, m, 1, *sc["up"], k=k)
    hid = orc.swiglu_bf16(g, u)
    return orc.k4_linear(hid, flat, host["down"], m, h, 2, *sc["down"], k=k).reshape(rows, slots, h)


@pytest.mark.parametrize("k", [3, 4])
@pytest.mark.parametrize("rows", [1, 5, 20])
def test_expert_layer_unoptimized_chain(cuda, orc, k, rows):
    from mlxlr8_amd import synth
    from mlxlr8_amd.experts import ExpertLayer
    h, m, E = 256, 128, 5
    say(f"case: ExpertLayer optimize=False k={k} rows={rows}")
    layer = synth.k4_layer(cuda, 300 + k, hidden=h, intermediate=m, experts=E, k=k)
    experts = ExpertLayer(layer["packed"], layer["scales"], h, m, k=k)
    rng = np.random.default_rng(rows)
    ids = torch.from_numpy(rng.integers(0, E, (rows, 9)).astype(np.int32)).to(cuda)
    x = _bf16(rng, (rows, h)).to(cuda)
    fused = experts(x, ids)
    experts.store.optimize = False
    plain = experts(x, ids)
    assert plain.shape == (rows, 9, h) and plain.dtype == torch.bfloat16
    host = {p: t.cpu().numpy() for p, t in layer["packed"].items()}
    sc = {p: (f16_bits(a), f16_bits(b)) for p, (a, b) in layer["scales"].items()}
    want = _chain_oracle(orc, x.cpu(), ids.cpu().numpy(), host, sc, k, h, m)
    got = bits_to_f32(bf16_bits(plain.cpu())).reshape(rows, 9, h)
    err = rel_l2(got, want)
    say(f"  chain rel_l2 vs oracle={err:.3e}  vs fused={rel_l2(got, bits_to_f32(bf16_bits(fused.cpu()))):.3e}")
    assert err <= 4e-3          # bf16 rounding of the three linear outputs and the activation
    assert rel_l2(got, bits_to_f32(bf16_bits(fused.cpu()))) <= 8e-3
