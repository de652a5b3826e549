"""Helpers shared by the GPU parity tests: host copies of only the experts a routing touches, and
the routing check against the oracle (ids equal unless a near tie of corrected scores separates
the 8th and 9th expert; logits differ only by fp32 summation order)."""
import sys

import numpy as np
import torch

from conftest import bf16_bits, f16_bits


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def check_routing(orc, x, w, bias, ids, tag=""):
    """Compare GPU routing ids [rows, 9] with the oracle's on the same input; returns the mismatch mask."""
    logits = orc.router_logits(bf16_bits(x), w.cpu().numpy())
    oids, _ = orc.route(logits, bias.cpu().numpy())
    ids = np.asarray(ids, np.uint32)
    mism = (ids != oids).any(axis=1)
    if mism.any():
        choice = 1 / (1 + np.exp(-logits.astype(np.float64))) + bias.cpu().numpy()
        for r in np.where(mism)[0]:
            srt = np.sort(choice[r])[::-1]
            assert srt[7] - srt[8] < 1e-5, f"{tag} row {r}: routing differs without a near tie"
    return mism


def compact_k4(packed, scales, ids, hidden, intermediate):
    """Host arrays of the experts in `ids` only: (remapped ids, packed {p: uint8}, scales {p: (in, out)
    f16 bits}) with expert j of the compact arrays = j-th distinct id."""
    ids = np.asarray(ids, np.int64)
    uniq = np.unique(ids)
    per = hidden * intermediate // 2
    remap = np.searchsorted(uniq, ids).astype(np.uint32)
    sel = torch.from_numpy(uniq).to(packed["gate"].device)
    host_packed = {p: torch.cat([t[int(e) * per:(int(e) + 1) * per] for e in uniq]).cpu().numpy()
                   for p, t in packed.items()}
    host_scales = {p: (f16_bits(a.index_select(0, sel)), f16_bits(b.index_select(0, sel))) for p, (a, b) in scales.items()}
    return remap, host_packed, host_scales


def oracle_k4(orc, x_bits, ids, scores, residual_bits, packed, scales, hidden, intermediate, want_values=False):
    """orc.k4_moe over host copies of only the touched experts."""
    remap, hp, hs = compact_k4(packed, scales, ids, hidden, intermediate)
    return orc.k4_moe(x_bits, remap.reshape(np.shape(ids)), scores, residual_bits, hidden, intermediate,
                      hp["gate"], hp["up"], hp["down"], hs["gate"][0], hs["gate"][1], hs["up"][0], hs["up"][1],
                      hs["down"][0], hs["down"][1], want_values=want_values)
