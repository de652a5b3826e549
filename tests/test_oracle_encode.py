"""Pin the oracle's K4 -> joined-MXFP4 encode (exlr8/joined_mxfp4.py:12-47) without a GPU.

The quantiser's scale/rounding choice of MLX's mx.quantize is not available here (parity
unpinned); what is pinned: exact groups come back unchanged, every element is the nearest E2M1
step (ties to the even code) of its value at the group scale, the scale exponent is
floor(log2 amax) - 2 computed independently, zero and saturating groups, and the orientation /
fold / gate||up layout of the reference's tests/test_joined_mxfp4.py:44-58.
"""
import numpy as np

E2M1 = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0])


def dequant(codes, scales):
    lo, hi = codes & 15, codes >> 4
    nib = np.stack([lo, hi], -1).reshape(*codes.shape[:-1], codes.shape[-1] * 2)
    mag = E2M1[nib & 7] * np.where(nib & 8, -1.0, 1.0)
    sc = np.exp2(scales.astype(np.float64) - 127)
    return mag * np.repeat(sc, 32, axis=-1)


def test_exact_groups_round_trip(orc):
    rng = np.random.default_rng(5)
    codes = rng.integers(0, 256, (64, 64), dtype=np.uint8)
    codes[:, ::16] = (codes[:, ::16] & 0xF0) | 7      # every group holds a 6 (its amax): scale is unique
    scales = rng.integers(100, 150, (64, 4), dtype=np.uint8)
    v = dequant(codes, scales).astype(np.float32)
    c2, s2 = orc.mx_quantize(v)
    np.testing.assert_array_equal(s2, scales)
    # -0 keeps its sign bit; every other code is reproduced
    np.testing.assert_array_equal(c2, codes)


def test_nearest_even_and_scale_by_brute_force(orc):
    rng = np.random.default_rng(6)
    v = (rng.standard_normal((256, 128)) * np.exp2(rng.integers(-20, 20, (256, 1)))).astype(np.float32)
    v[3, :32] = 0.0                                    # all-zero group
    v[4, 5] = -0.0
    codes, scales = orc.mx_quantize(v)
    groups = v.reshape(256, 4, 32).astype(np.float64)
    amax = np.abs(groups).max(-1)
    s_expect = np.where(amax > 0, np.floor(np.log2(np.where(amax > 0, amax, 1))) - 2, -127)
    np.testing.assert_array_equal(scales.astype(int) - 127, s_expect.astype(int))
    assert scales[3, 0] == 0 and not codes[3, :16].any()
    nib = np.stack([codes & 15, codes >> 4], -1).reshape(256, 128)
    a = np.abs(v.astype(np.float64)) / np.repeat(np.exp2(s_expect), 32, axis=-1)
    # brute force: distance to all 8 magnitudes, ties to the even code
    d = np.abs(a[..., None] - E2M1)
    best = np.min(d, -1, keepdims=True)
    cand = d == best
    even = cand & (np.arange(8) % 2 == 0)
    pick = np.where(even.any(-1), np.argmax(even, -1), np.argmax(cand, -1))
    np.testing.assert_array_equal(nib & 7, pick)
    np.testing.assert_array_equal(nib >> 3, np.signbit(v).astype(int))


def test_saturating_group(orc):
    v = np.zeros((1, 32), np.float32)
    v[0, 0], v[0, 1], v[0, 2] = 7.9, -7.0, 6.5      # amax in [4, 8): s = 0, all three saturate to 6
    codes, scales = orc.mx_quantize(v)
    assert scales[0, 0] == 127
    assert codes[0, 0] == (7 | (0xF << 4)) and (codes[0, 1] & 15) == 7


def test_encode_orientation_fold_and_joined_rows(orc):
    # the reference fixture's shapes and scale structure (tests/test_joined_mxfp4.py:18-41)
    rng = np.random.default_rng(817)
    h, m, count = 256, 128, 3
    signs = rng.choice([-1, 1], h).astype(np.float16)
    raw, scales = {}, {}
    for projection in ("gate", "up", "down"):
        incoming, outgoing = (m, h) if projection == "down" else (h, m)
        raw[projection] = rng.integers(0, 256, (count, h * m // 2), np.uint8)
        incoming_scale = rng.uniform(.01, .04, (count, incoming)).astype(np.float16)
        if projection != "down":
            block = rng.uniform(.01, .04, (count, h // 128)).astype(np.float16)
            block *= rng.choice([-1, 1], block.shape).astype(np.float16)
            incoming_scale = np.repeat(block, 128, axis=-1) * signs
        scales[projection] = incoming_scale
    unit = np.sign(scales["gate"][0]).astype(np.float16)
    gu = (np.zeros((count, 2 * m, h // 2), np.uint8), np.zeros((count, 2 * m, h // 32), np.uint8))
    dn = (np.zeros((count, h, m // 2), np.uint8), np.zeros((count, h, m // 32), np.uint8))
    orc.k4_to_mxfp4(raw["gate"], h, m, 1, count, scales["gate"].view(np.uint16), unit.view(np.uint16), *gu, 0)
    orc.k4_to_mxfp4(raw["up"], h, m, 1, count, scales["up"].view(np.uint16), unit.view(np.uint16), *gu, m)
    orc.k4_to_mxfp4(raw["down"], m, h, 2, count, None, None, *dn, 0)
    for projection, offset in (("gate", 0), ("up", m), ("down", 0)):
        incoming, outgoing, side = (m, h, 2) if projection == "down" else (h, m, 1)
        dest = dn if projection == "down" else gu
        for i in range(count):
            matrix = orc.decode(raw[projection].reshape(-1), 4, incoming, outgoing, side, i).astype(np.float64)
            if projection != "down":
                factor = scales[projection][i].astype(np.float64) * unit.astype(np.float64)
                matrix = matrix * factor[:, None]
            c, s = orc.mx_quantize(matrix.T.astype(np.float32))
            np.testing.assert_array_equal(dest[0][i, offset:offset + outgoing], c)
            np.testing.assert_array_equal(dest[1][i, offset:offset + outgoing], s)
            # the encoded rows dequantise to within half an E2M1 step (at most 2^s), or the
            # saturation distance (below 2^(s+1)), of the folded matrix
            err = np.abs(dequant(c, s) - matrix.T)
            unit_step = np.repeat(np.exp2(s.astype(np.float64) - 127), 32, axis=-1)
            assert (err <= 2 * unit_step).all()
