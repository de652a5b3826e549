"""Independent numpy restatements used to pin the oracle (not the oracle's own formulas).

* codebook_frexp: the K4 codebook (exlr8/trellis.py:22-50) as hash -> fp16 half sum -> E4M3
  rounding, with the rounding done through frexp/ldexp in float64 (a different route from the
  oracle's nearest-level search).
* pack_k4 / pack_trellis: MSB-first bit packing per ponyexl3/ref/trellis.py:13-49 semantics.
* tensor_core_perm: ponyexl3/ref/perm.py:8-26 as an explicit table.
* hadamard_matrix: the Sylvester definition H[i,j] = (-1)^popcount(i&j) / sqrt(128).
"""
import numpy as np


def _halves_sum(states):
    """fp16(lo + hi) of the masked MCG hash of each 16-bit state."""
    word = (np.asarray(states, np.uint64) * 0xCBAC1FED) % (1 << 32)
    word = (word & 0x8FFF8FFF) ^ 0x3B603B60
    lo = (word & 0xFFFF).astype(np.uint16).view(np.float16)
    hi = (word >> 16).astype(np.uint16).view(np.float16)
    return lo + hi  # numpy adds two float16 arrays with one fp16 rounding


def round_e4m3_frexp(v):
    """Round float values to E4M3 (3 mantissa bits, minimum normal exponent -6, ties to even)."""
    v = np.asarray(v, np.float64)
    _, e = np.frexp(np.abs(v))                   # |v| = m * 2**e with m in [0.5, 1)
    quantum = np.ldexp(1.0, np.maximum(e - 1, -6) - 3)
    return np.copysign(np.round(np.abs(v) / quantum) * quantum, v)   # np.round is half-to-even


def codebook_frexp():
    return round_e4m3_frexp(_halves_sum(np.arange(1 << 16))).astype(np.float16)


def pack_trellis(values, k):
    """values [..., 256] of k-bit symbols -> [..., 8k] uint32 words, MSB-first bitstream."""
    values = np.asarray(values, np.uint64)
    shape = values.shape[:-1]
    flat = values.reshape(-1, 256)
    out = np.zeros((flat.shape[0], 8 * k), np.uint32)
    for t in range(flat.shape[0]):
        bits = 0
        for v in flat[t]:
            bits = (bits << k) | int(v)
        total = 256 * k
        for w in range(8 * k):
            out[t, w] = (bits >> (total - 32 * (w + 1))) & 0xFFFFFFFF
    return out.reshape(*shape, 8 * k)


def tensor_core_perm():
    perm = np.zeros(256, np.int32)
    for t in range(32):
        r0 = (t % 4) * 2
        c0 = t // 4
        rows = [r0, r0 + 1, r0 + 8, r0 + 9]
        for j in range(8):
            perm[t * 8 + j] = rows[j % 4] * 16 + c0 + (8 if j >= 4 else 0)
    return perm


def hadamard_matrix(n=128):
    i = np.arange(n)
    pc = np.vectorize(lambda v: bin(v).count("1"))(i[:, None] & i[None, :])
    return np.where(pc % 2 == 0, 1.0, -1.0) / np.sqrt(n)


def block_hadamard(x, n=128):
    x = np.asarray(x, np.float64)
    return (x.reshape(-1, n) @ hadamard_matrix(n)).reshape(x.shape)


def e4m3_levels():
    codes = np.arange(127)
    e, f = codes >> 3, codes & 7
    return np.where(e == 0, f * 2.0 ** -9, (8 + f) * 2.0 ** (e - 10))


def fp8_e4m3_decode(byte):
    """OCP E4M3 byte -> float (NaN for 0x7F/0xFF)."""
    b = np.asarray(byte, np.int64)
    e, f = (b >> 3) & 15, b & 7
    mag = np.where(e == 0, f / 512.0, np.ldexp(1 + f / 8.0, (e - 7).astype(np.int64)))
    mag = np.where((b & 127) == 127, np.nan, mag)
    return np.where(b & 128, -mag, mag)


def build_trellis_matrix(nibbles, side, k=4):
    """Per-tile k-bit symbols [IT, OT, 256] (kernel order) -> stored bytes for one matrix."""
    it, ot = nibbles.shape[:2]
    words = pack_trellis(nibbles, k)  # [IT, OT, 8k]
    if side == 2:
        stored = words.reshape(it // 8, 8, ot // 8, 8, 8 * k).transpose(0, 2, 1, 3, 4)
    else:
        stored = words.reshape(it, ot // 8, 8, 8 * k).transpose(1, 0, 2, 3)
    return np.ascontiguousarray(stored).reshape(-1).view(np.uint8)


def expected_inner(nibbles, k=4):
    """Inner [IT*16, OT*16] values from per-tile k-bit symbols: codeword i = the last 16 bits of the
    symbols up to and including symbol i (circular within the tile)."""
    from oracle import lib
    cb = lib().codebook().astype(np.float32)
    it, ot = nibbles.shape[:2]
    n = nibbles.astype(np.uint32)
    cw = np.zeros_like(n)
    for j in range(-(-16 // k)):
        cw |= np.roll(n, j, -1) << (k * j)
    cw &= 0xFFFF
    vals = cb[cw]  # kernel order
    perm = tensor_core_perm()
    tile = np.zeros((it, ot, 256), np.float32)
    tile[..., perm] = vals
    return tile.reshape(it, ot, 16, 16).transpose(0, 2, 1, 3).reshape(it * 16, ot * 16)
