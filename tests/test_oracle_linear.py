"""Pin the oracle's linear algebra (trellis linear, MXFP4 linear, full MoE layer) against dense
numpy matrices built independently from per-tile symbols (no GPU)."""
import numpy as np
import pytest

import refmath
from conftest import bits_to_f32


def _bf16(x):
    u = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return bits_to_f32(u.astype(np.uint32))


def _k4_matrix(rng, experts, in_f, out_f, side, k=4):
    nibs = [rng.integers(0, 1 << k, (in_f // 16, out_f // 16, 256), dtype=np.uint32) for _ in range(experts)]
    packed = np.concatenate([refmath.build_trellis_matrix(n, side, k) for n in nibs])
    return packed, [refmath.expected_inner(n, k) for n in nibs]


def test_k4_linear_matches_dense_public_matrix(orc):
    rng = np.random.default_rng(21)
    for side in (1, 2):
        packed, inners = _k4_matrix(rng, 3, 256, 128, side)
        ins = rng.uniform(-.3, .3, (3, 256)).astype(np.float16)
        outs = rng.uniform(-.3, .3, (3, 128)).astype(np.float16)
        x = rng.normal(size=(5, 256)).astype(np.float32)
        ids = np.array([2, 0, 1, 2, 0], np.uint32)
        got = orc.k4_linear(x, ids, packed, 256, 128, side, ins.view(np.uint16), outs.view(np.uint16))
        for s, e in enumerate(ids):
            h_in, h_out = refmath.hadamard_matrix(), refmath.hadamard_matrix()
            # public W[out, in] = diag(out) H_out inner^T H_in diag(in), with block-diagonal H
            hi = np.kron(np.eye(2), h_in)
            ho = h_out
            w = outs[e].astype(np.float64)[:, None] * (ho @ inners[e].T.astype(np.float64) @ hi) \
                * ins[e].astype(np.float64)[None, :]
            np.testing.assert_allclose(got[s], w @ x[s].astype(np.float64), rtol=2e-5, atol=2e-5)


def test_mxfp4_linear_matches_dequantised_matrix(orc):
    rng = np.random.default_rng(9)
    E, N, K = 3, 64, 256
    codes = rng.integers(0, 256, (E, N, K // 2), dtype=np.uint8)
    scales = rng.integers(118, 130, (E, N, K // 32), dtype=np.uint8)
    scales[0, 0, 0] = 0  # e8m0 zero -> 2^-127 (exlr8/metal/joined_gather_order.metal:20)
    e2m1 = np.array([0, .5, 1, 1.5, 2, 3, 4, 6], np.float64)
    nib = np.stack([codes & 15, codes >> 4], -1).reshape(E, N, K)
    vals = np.where(nib & 8, -1, 1) * e2m1[nib & 7]
    sc = np.where(scales == 0, 2.0 ** -127, np.ldexp(1.0, scales.astype(np.int64) - 127))
    deq = vals * np.repeat(sc, 32, axis=-1)
    x = rng.normal(size=(4, K)).astype(np.float32)
    ids = np.array([0, 2, 1, 0], np.uint32)
    got = orc.mxfp4_linear(x, ids, codes, scales, K, N)
    want = np.stack([deq[e] @ x[i].astype(np.float64) for i, e in enumerate(ids)])
    np.testing.assert_allclose(got, want, rtol=1e-6, atol=1e-6)
    assert orc.h.orc_f32_to_bf16(1.0) == 0x3F80


@pytest.mark.parametrize("k", [4, 3, 2])
def test_k4_moe_layer_matches_dense_composition(orc, k):
    """The oracle's MoE layer (K4, and the K3/K2 experts of the same chain) against dense maths."""
    rng = np.random.default_rng(181 + k)
    h, m, E = 256, 128, 3
    pg, ig = _k4_matrix(rng, E, h, m, 1, k)
    pu, iu = _k4_matrix(rng, E, h, m, 1, k)
    pd, idd = _k4_matrix(rng, E, m, h, 2, k)
    sc = {k: rng.uniform(-.3, .3, shape).astype(np.float16) for k, shape in
          (("in_g", (E, h)), ("out_g", (E, m)), ("in_u", (E, h)), ("out_u", (E, m)), ("in_d", (E, m)), ("out_d", (E, h)))}
    rows = 2
    x = _bf16(rng.normal(size=(rows, h)))
    res = _bf16(rng.normal(size=(rows, h)))
    idx = np.array([[2, 0, 1, 2, 0, 1, 2, 0, 1], [0, 1, 2, 0, 1, 2, 0, 1, 2]], np.uint32)
    scores = rng.uniform(.03, .4, (rows, 8)).astype(np.float32)
    bits = lambda a: (a.view(np.uint32) >> 16).astype(np.uint16)
    out, values = orc.k4_moe(bits(x), idx, scores, bits(res), h, m, pg, pu, pd,
                             *[sc[n].view(np.uint16) for n in ("in_g", "out_g", "in_u", "out_u", "in_d", "out_d")],
                             want_values=True, k=k)

    def lin(v, inner, s_in, s_out):
        return refmath.block_hadamard(refmath.block_hadamard(v * s_in.astype(np.float64)) @ inner.astype(np.float64)) \
            * s_out.astype(np.float64)

    def swiglu(g, u):
        g, u = _bf16(g), _bf16(u)
        tail = (1 / (1 + np.exp(np.abs(g).astype(np.float32)))).astype(np.float32)
        sig = _bf16(np.where(g < 0, tail, 1 - tail))
        return _bf16(_bf16(g * sig) * u)

    for r in range(rows):
        ys = []
        for j, e in enumerate(idx[r]):
            g = lin(x[r], ig[e], sc["in_g"][e], sc["out_g"][e])
            u = lin(x[r], iu[e], sc["in_u"][e], sc["out_u"][e])
            a = swiglu(g.astype(np.float32), u.astype(np.float32))
            y = _bf16(lin(a, idd[e], sc["in_d"][e], sc["out_d"][e]).astype(np.float32))
            ys.append(y)
            got = bits_to_f32(values[r, j])
            # bf16 outputs: allow one bf16 ulp where the float64 dense order rounds differently
            np.testing.assert_allclose(got, y, rtol=2 ** -7, atol=1e-6)
        ys = np.stack(ys)
        routed = _bf16((ys[:8] * scores[r][:, None]).astype(np.float32).sum(0, dtype=np.float32))
        comb = _bf16(routed + ys[8])
        want = _bf16(res[r] + comb)
        np.testing.assert_allclose(bits_to_f32(out[r]), want, rtol=2 ** -6, atol=1e-5)


def test_residual_rmsnorm(orc):
    rng = np.random.default_rng(2)
    n = 6144
    x = _bf16(rng.normal(size=(2, n)))
    r = _bf16(rng.normal(size=(2, n)))
    w = _bf16(rng.uniform(.5, 1.5, n))
    bits = lambda a: (a.view(np.uint32) >> 16).astype(np.uint16)
    h_out, out = orc.residual_rmsnorm(bits(x), bits(r), bits(w))
    h = _bf16(x + r)
    np.testing.assert_array_equal(bits_to_f32(h_out), h)
    inv = 1 / np.sqrt((h.astype(np.float64) ** 2).mean(-1, keepdims=True) + 1e-5)
    want = _bf16(w * _bf16((h * inv).astype(np.float32)))
    np.testing.assert_allclose(bits_to_f32(out), want, rtol=2 ** -7)
