"""The oracle against the known answers of the reference's own tests (tests/golden)."""
import json
from pathlib import Path

import numpy as np

GOLD = json.loads((Path(__file__).parent / "golden" / "reference_known_answers.json").read_text())


def _f(v):
    return float(v)  # json holds "inf" / "-inf" as strings; float() parses both


def test_codebook_state_zero(orc):
    cb = orc.codebook()
    g = GOLD["codebook"]
    assert float(cb[g["state"]]) == g["value"]


def test_e4m3_midpoints_tie_to_even(orc):
    g = GOLD["e4m3_midpoints"]
    x = np.asarray(g["inputs"], np.float32)
    want = np.asarray(g["expected"], np.float32)
    np.testing.assert_array_equal(orc.round_e4m3(x), want)
    np.testing.assert_array_equal(orc.round_e4m3(-x), -want)


def test_e4m3_saturation_and_signed_zero(orc):
    g = GOLD["e4m3_saturation"]
    x = np.asarray([_f(v) for v in g["inputs"]], np.float32)
    np.testing.assert_array_equal(orc.round_e4m3(x), np.asarray(g["expected"], np.float32))
    assert np.signbit(orc.round_e4m3(np.asarray([-0.0], np.float32))[0]) == g["negative_zero_keeps_sign"]


def test_resident_projection_bytes(orc):
    g = GOLD["resident_bytes"]
    packed = g["in_features"] * g["out_features"] * g["k"] // 8
    assert packed + 2 * g["in_features"] * 2 == g["per_projection_bytes"]
    assert orc.check_format(packed * g["experts"], g["k"], g["in_features"], g["out_features"], 1) == g["experts"]


def test_fp32_accumulation_known_answer(orc):
    """All-zero bitstream -> every weight codebook[0]; the inner sum exceeds the fp16 range."""
    g = GOLD["fp32_accumulation"]
    w, n = g["width"], g["output"]
    packed = np.zeros(w * n // 2, np.uint8)
    x = np.zeros(w, np.float32)
    x[::128] = g["spike"]
    one = np.uint16(0x3C00)  # fp16 1.0
    y = orc.k4_linear(x[None, :], np.zeros(1, np.uint32), packed, w, n, 1, np.full(w, one), np.full(n, one))[0]
    assert g["inner_sum"] > g["fp16_max"]
    np.testing.assert_allclose(y[0], g["expected_col0"], rtol=1e-6)
    np.testing.assert_allclose(y[1:], g["expected_other_cols"], atol=1e-3)
