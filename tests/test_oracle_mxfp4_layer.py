"""Pin the oracle's joined-MXFP4 MoE layer (``orc_mxfp4_moe``) against an independent numpy
composition over dequantised matrices, with the structure of the reference's
tests/test_joined_mxfp4.py:61-86 (slots) and :89-107 (finish): common = H(x * unit), gate_up =
common @ W_gu^T with gate rows [0, m) and up rows [m, 2m), gate = T(H(g) * out_gate), up =
T(H(u) * out_up), a = swiglu_T(gate, up), value = T(H(H(a * in_down) @ W_down^T) * out_down); the
finish is residual + T(T(sum_i values_i * scores_i) + shared).  No GPU.

Each mistake a restatement could plausibly make -- gate/up halves swapped, the unit sign dropped,
the gate and up output scales exchanged, in_down not applied -- is planted by feeding the oracle
the corresponding transformed inputs: each must move its output far outside the tolerance.
"""
import numpy as np
import pytest

import refmath
from conftest import bits_to_f32

H, M, E = 256, 128, 257
E2M1 = np.array([0, .5, 1, 1.5, 2, 3, 4, 6], np.float64)


def _bf16(x):
    u = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return bits_to_f32(u.astype(np.uint32))


def _bits(a):
    return (np.asarray(a, np.float32).view(np.uint32) >> 16).astype(np.uint16)


def _dequantise(codes, scales):
    """MXFP4 rows: e2m1 nibbles (low nibble = even k, bit 3 = sign) x 2^(s - 127) per 32 along K."""
    nib = np.stack([codes & 15, codes >> 4], -1).reshape(*codes.shape[:-1], codes.shape[-1] * 2)
    vals = np.where(nib & 8, -1.0, 1.0) * E2M1[nib & 7]
    return vals * np.repeat(np.ldexp(1.0, scales.astype(np.int64) - 127), 32, axis=-1)


def _swiglu_t(g, u):
    g, u = _bf16(g), _bf16(u)
    tail = (1 / (1 + np.exp(np.abs(g).astype(np.float32)))).astype(np.float32)
    sig = _bf16(np.where(g < 0, tail, 1 - tail))
    return _bf16(_bf16(g * sig) * u)


@pytest.fixture(scope="module")
def layer():
    rng = np.random.default_rng(817)
    gu_codes = rng.integers(0, 256, (E, 2 * M, H // 2), dtype=np.uint8)
    gu_scales = rng.integers(120, 126, (E, 2 * M, H // 32), dtype=np.uint8)
    d_codes = rng.integers(0, 256, (E, H, M // 2), dtype=np.uint8)
    d_scales = rng.integers(120, 126, (E, H, M // 32), dtype=np.uint8)
    unit = rng.choice([-1.0, 1.0], H).astype(np.float16)
    side = {"og": rng.uniform(-.5, .5, (E, M)), "ou": rng.uniform(-.5, .5, (E, M)),
            "idn": rng.uniform(.01, .04, (E, M)) * rng.choice([-1, 1], (E, M)), "od": rng.uniform(-.5, .5, (E, H))}
    side = {k: v.astype(np.float16) for k, v in side.items()}
    deq = {e: (_dequantise(gu_codes[e], gu_scales[e]), _dequantise(d_codes[e], d_scales[e])) for e in (0, 1, 255, 256)}
    return dict(gu_codes=gu_codes, gu_scales=gu_scales, d_codes=d_codes, d_scales=d_scales, unit=unit, deq=deq,
                **side)


def _numpy_slots(L, x, ids):
    """values [rows, 9, H] (float32, bf16-valued), composed as the reference test does."""
    unit = L["unit"].astype(np.float64)
    out = np.empty((x.shape[0], ids.shape[1], H), np.float32)
    for r in range(x.shape[0]):
        common = refmath.block_hadamard(x[r].astype(np.float64) * unit)
        for j, e in enumerate(ids[r]):
            w_gu, w_d = L["deq"][int(e)]
            gu = w_gu @ common
            gate = _bf16((refmath.block_hadamard(gu[:M]) * L["og"][e]).astype(np.float32))
            up = _bf16((refmath.block_hadamard(gu[M:]) * L["ou"][e]).astype(np.float32))
            act = _swiglu_t(gate, up).astype(np.float64)
            inner = w_d @ refmath.block_hadamard(act * L["idn"][e])
            out[r, j] = _bf16((refmath.block_hadamard(inner) * L["od"][e]).astype(np.float32))
    return out


def _oracle(orc, L, x, ids, scores, res, **over):
    a = dict(L, **over)
    return orc.mxfp4_moe(_bits(x), ids, scores, _bits(res), H, M, a["gu_codes"], a["gu_scales"], a["d_codes"],
                         a["d_scales"], a["unit"].view(np.uint16), a["og"].view(np.uint16), a["ou"].view(np.uint16),
                         a["idn"].view(np.uint16), a["od"].view(np.uint16), want_values=True)


def _case(rows, seed):
    rng = np.random.default_rng(seed)
    x = _bf16(rng.normal(size=(rows, H)))
    res = _bf16(rng.normal(size=(rows, H)))
    ids = rng.choice([0, 1, 255], (rows, 9)).astype(np.uint32)
    ids[:, 8] = 256
    ids[0, :4] = [0, 1, 255, 256]
    scores = rng.uniform(.03, .2, (rows, 8)).astype(np.float32)
    return x, ids, scores, res


def _rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


@pytest.mark.parametrize("rows", [1, 3])
def test_oracle_mxfp4_layer_matches_dequantised_composition(orc, layer, rows):
    x, ids, scores, res = _case(rows, 840 + rows)
    out, values = _oracle(orc, layer, x, ids, scores, res)
    want = _numpy_slots(layer, x, ids)
    got = bits_to_f32(values).reshape(want.shape)
    # bf16-valued outputs: the float64 dense order may round a value one bf16 step the other way
    np.testing.assert_allclose(got, want, rtol=2 ** -7, atol=1e-6)
    assert _rel(got, want) < 1e-3
    # finish = residual + T(T(sum_i values_i * scores_i) + shared) over the numpy values
    for r in range(rows):
        routed = _bf16((want[r, :8] * scores[r][:, None]).astype(np.float32).sum(0, dtype=np.float32))
        wanted = _bf16(res[r] + _bf16(routed + want[r, 8]))
        np.testing.assert_allclose(bits_to_f32(out[r]), wanted, rtol=2 ** -6, atol=1e-5)


def _swap_halves(a):
    return np.ascontiguousarray(np.concatenate([a[:, M:], a[:, :M]], axis=1))


@pytest.mark.parametrize("mistake", ["gate_up_swapped", "unit_dropped", "out_scales_exchanged", "in_down_dropped"])
def test_planted_composition_mistakes_are_caught(orc, layer, mistake):
    """The comparison above fails for each plausible composition mistake of a restatement."""
    x, ids, scores, res = _case(2, 901)
    over = {
        "gate_up_swapped": dict(gu_codes=_swap_halves(layer["gu_codes"]), gu_scales=_swap_halves(layer["gu_scales"])),
        "unit_dropped": dict(unit=np.ones(H, np.float16)),
        "out_scales_exchanged": dict(og=layer["ou"], ou=layer["og"]),
        "in_down_dropped": dict(idn=np.ones((E, M), np.float16)),
    }[mistake]
    assert np.any(layer["unit"] < 0)
    _, values = _oracle(orc, layer, x, ids, scores, res, **over)
    want = _numpy_slots(layer, x, ids)
    assert _rel(bits_to_f32(values).reshape(want.shape), want) > 0.1
