"""Pin the CPU oracle's codebook, E4M3 rounding, trellis geometry and Hadamard (no GPU)."""
import hashlib

import numpy as np
import pytest

import refmath


def test_codebook_known_answers(orc):
    cb = orc.codebook()
    # tests/test_trellis.py:63 (reference known answer) and further entries of the codebook as
    # exlr8/trellis.py:22-50 defines it
    assert cb[0] == np.float16(1.875)
    assert cb[1] == np.float16(0.140625) and cb[2] == np.float16(-0.75)
    assert cb[3] == np.float16(0.8125) and cb[65535] == np.float16(0.875)


def test_codebook_matches_frexp_restatement(orc):
    # independent route: E4M3 rounding through frexp/ldexp (exlr8/trellis.py:22-50 defines the codebook)
    np.testing.assert_array_equal(orc.codebook().view(np.uint16), refmath.codebook_frexp().view(np.uint16))


def test_frexp_rounding_catches_planted_mistakes():
    # the restatement itself: ties go to even, the subnormal quantum is 2**-9, signs survive
    got = refmath.round_e4m3_frexp([1.0625, 1.1875, 2.0 ** -9 * 1.5, -0.3, 0.0, 3.0 * 2 ** -10])
    np.testing.assert_array_equal(got, [1.0, 1.25, 2.0 ** -8, -0.3125, 0.0, 2.0 ** -8])


def test_codebook_digest_and_e4m3_property(orc):
    cb = orc.codebook()
    digest = hashlib.sha256(cb.view("<u2").tobytes()).hexdigest()
    assert digest == "04f9e17b1eceec00fd88c2b77dba69dda41f522f8526a2be513ae36383ec2c4b"
    levels = refmath.e4m3_levels()
    mags = np.abs(cb.astype(np.float64))
    assert np.isin(mags, levels).all()          # every value is an exact E4M3 magnitude
    assert len(np.unique(cb)) == 189 and np.abs(cb).max() <= 4


def test_round_e4m3_ties_saturation_signed_zero(orc):
    # tests/test_trellis.py:48-57
    values = refmath.e4m3_levels().astype(np.float32)
    mid = (values[:-1] + values[1:]) / 2
    expected = values[np.arange(126) + (np.arange(126) & 1)]
    np.testing.assert_array_equal(orc.round_e4m3(mid), expected)
    np.testing.assert_array_equal(orc.round_e4m3(-mid), -expected)
    np.testing.assert_array_equal(orc.round_e4m3([500, -500, np.inf, -np.inf]), [448, -448, 448, -448])
    assert np.signbit(orc.round_e4m3(np.array([-0.0], np.float32)))[0]


@pytest.mark.parametrize("side", [0, 1, 2])
def test_decode_brute_force_both_storage_orders(orc, side):
    rng = np.random.default_rng(8 + side)
    in_f, out_f = 256, 384
    nib = rng.integers(0, 16, (in_f // 16, out_f // 16, 256), dtype=np.uint32)
    stored = refmath.build_trellis_matrix(nib, side if side == 2 else 1)
    np.testing.assert_array_equal(orc.decode(stored, 4, in_f, out_f, side), refmath.expected_inner(nib))


def test_decode_second_expert_offset(orc):
    rng = np.random.default_rng(3)
    nibs = [rng.integers(0, 16, (8, 8, 256), dtype=np.uint32) for _ in range(3)]
    for side in (1, 2):
        packed = np.concatenate([refmath.build_trellis_matrix(n, side) for n in nibs])
        for e in range(3):
            np.testing.assert_array_equal(orc.decode(packed, 4, 128, 128, side, e), refmath.expected_inner(nibs[e]))


def test_direct_k4_windows_match_general_formula(orc):
    # the direct form (exlr8/metal/fast_decode_linear.metal:148-155; tests/test_fast_decode.py:56-69)
    rng = np.random.default_rng(235)
    words = rng.integers(0, 2**32, (4, 32), dtype=np.uint64).astype(np.uint32)
    prior = np.roll(words, 1, axis=-1)
    direct = np.stack([((prior << 4) | (words >> 28)) & 65535, ((prior << 8) | (words >> 24)) & 65535,
                       ((prior << 12) | (words >> 20)) & 65535, words >> 16, (words >> 12) & 65535,
                       (words >> 8) & 65535, (words >> 4) & 65535, words & 65535], axis=-1).reshape(4, 256)
    packed = words.view(np.uint8).reshape(-1)
    # four tiles of one 16x64 side-0 matrix? use per-tile codeword probe through a 128x128 layout
    full = np.zeros((8 * 8, 32), np.uint32)
    full[:4] = words
    blob = full.reshape(-1).view(np.uint8)
    for t in range(4):
        for i in range(256):
            lane, slot = divmod(i, 8)
            r = (lane % 4) * 2 + (slot & 1) + (slot & 2) * 4
            c = lane // 4 + (slot & 4) * 2
            # side 1: tile index (tn/8*IT + tk)*8 + tn%8 with IT=8: tile t -> tk=0, tn=t
            cw = orc.h.orc_codeword_at(blob.ctypes.data, 4, 128, 128, 1, 0, r, 16 * t + c)
            assert cw == direct[t, i]
    assert packed.size == 4 * 128


def test_format_errors(orc):
    assert orc.check_format(5, 4, 128, 128, 1) < 0
    assert orc.check_format(128 * 128 // 2, 4, 128, 128, 1) == 1
    assert orc.check_format(128 * 128 // 2, 4, 100, 128, 1) < 0
    assert orc.check_format(128 * 128 // 2, 5, 128, 128, 1) < 0


def test_hadamard_matches_sylvester_matrix(orc):
    rng = np.random.default_rng(5)
    x = rng.normal(size=(3, 256)).astype(np.float32)
    np.testing.assert_allclose(orc.hadamard(x), refmath.block_hadamard(x), rtol=2e-6, atol=2e-6)
    # self-inverse and block-local (tests/test_trellis.py:72-76)
    e = np.zeros((2, 256), np.float32)
    e[0, 0], e[1, 129] = 1, 2
    np.testing.assert_allclose(orc.hadamard(orc.hadamard(e)), e, atol=3e-7)
    assert np.all(orc.hadamard(e)[0, 128:] == 0)


@pytest.mark.parametrize("k", [2, 3])
@pytest.mark.parametrize("side", [1, 2])
def test_oracle_decode_k2_k3_brute_force(orc, k, side):
    # random k-bit symbols packed MSB-first (ponyexl3/ref/trellis.py:13-49 semantics), two experts
    rng = np.random.default_rng(40 + 10 * k + side)
    syms = [rng.integers(0, 1 << k, (8, 16, 256), dtype=np.uint32) for _ in range(2)]
    host = np.concatenate([refmath.build_trellis_matrix(s, side, k) for s in syms])
    for e in range(2):
        np.testing.assert_array_equal(orc.decode(host, k, 128, 256, side, e), refmath.expected_inner(syms[e], k))
