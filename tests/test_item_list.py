"""The fused K4 decode block's work list (moe_k4_item_list, computed by the kernel's own list code
on the host): every item appears once, and every item's inputs come from items earlier in the list.
The launch is persistent and its waves only ever wait for earlier items, so this ordering is what
guarantees that the lowest unfinished item can always run (no deadlock) with any number of
resident blocks serving each of the 8 sub-lists.  CPU only."""
import ctypes

import numpy as np
import pytest

GU, DOWN, ROUTER, GF, DF, NONE, GS = 0, 1, 2, 3, 4, 5, 6
LAG_G = 2  # units whose gate finishes take group sums (the last ones); checked through the list


def item_list(h, m, units, route):
    from mlxlr8_amd._lib import lib
    L = lib()
    n = L.moe_k4_item_list(h, m, units, route, None, 0)
    assert n > 0, L.moe_last_error()
    buf = (ctypes.c_int32 * (5 * n))()
    got = L.moe_k4_item_list(h, m, units, route, buf, n)
    assert got == n, L.moe_last_error()
    return np.frombuffer(buf, dtype=np.int32).reshape(n, 5)


def check_list(items, h, m, units, route):
    HB, MB = h // 128, m // 128
    S = h // 1024
    pos = {}
    for j, (k, u, a, b, c) in enumerate(items.tolist()):
        key = (k, u, a, b, c)
        assert key not in pos, f"item {key} listed twice"
        assert k != NONE, f"position {j} holds no item"
        pos[key] = j
    routers = [j for (k, *_), j in pos.items() if k == ROUTER]
    assert len(routers) == (256 * S if route else 0)
    last_router = max(routers) if routers else -1
    gu = {(u, a, b, c): j for (k, u, a, b, c), j in pos.items() if k == GU}
    gs = {(u, a, b): j for (k, u, a, b, c), j in pos.items() if k == GS}
    gf = {(u, a): j for (k, u, a, b, c), j in pos.items() if k == GF}
    dn = {(u, a, c): j for (k, u, a, b, c), j in pos.items() if k == DOWN}
    dfin = {(u, a): j for (k, u, a, b, c), j in pos.items() if k == DF}
    assert len(gu) == units * 2 * MB * HB and len(dn) == units * HB * MB
    assert len(gf) == units * MB and len(dfin) == units * HB
    for (u, ob, p, kb), j in gu.items():
        if route and u >= 1:
            assert j > last_router, f"gate/up part of unit {u} before the routing it needs"
    grouped = sorted({u for (u, _, _) in gs})
    for (u, ob, g), j in gs.items():
        for p in (0, 1):
            for kb in range(8 * g, min(8 * g + 8, HB)):
                assert gu[(u, ob, p, kb)] < j, f"group sum ({u},{ob},{g}) before its part"
    for (u, ob), j in gf.items():
        if u in grouped:
            for g in range((HB + 7) // 8):
                assert gs[(u, ob, g)] < j
        else:
            for p in (0, 1):
                for kb in range(HB):
                    assert gu[(u, ob, p, kb)] < j, f"gate finish ({u},{ob}) before part kb {kb}"
    for (u, ob, kb), j in dn.items():
        assert gf[(u, kb)] < j, f"down part ({u},{ob},{kb}) before the gate finish of its input block"
    for (u, ob), j in dfin.items():
        for kb in range(MB):
            assert dn[(u, ob, kb)] < j, f"down finish ({u},{ob}) before its part {kb}"
        if u == units - 1:  # the combine of output block ob reads every unit's slot outputs
            for v in range(units - 1):
                assert dfin[(v, ob)] < j, f"combine of block {ob} before unit {v}'s down finish"
    return grouped


@pytest.mark.parametrize("h,m,route", [(6144, 2048, 1), (6144, 2048, 0), (1024, 256, 1), (1024, 256, 0),
                                       (256, 256, 0), (2048, 512, 1)])
def test_every_item_follows_its_inputs(h, m, route):
    for units in range(1, 73):
        grouped = check_list(item_list(h, m, units, route), h, m, units, route)
        assert len(grouped) <= LAG_G


def test_sub_lists_all_served():
    """The list is dealt round-robin over 8 sub-lists and block b serves sub-list b mod 8: every
    sub-list gets items and, with the launch's grid of max(CUs, 8) blocks, a block."""
    items = item_list(6144, 2048, 9, 1)
    counts = np.bincount(np.arange(len(items)) % 8, minlength=8)
    assert (counts > 0).all()
    for grid in (8, 64, 256, 304):
        assert set(np.arange(grid) % 8) == set(range(8))


def test_item_list_argument_errors():
    from mlxlr8_amd._lib import lib
    L = lib()
    assert L.moe_k4_item_list(6144, 2048, 0, 1, None, 0) == -1
    assert L.moe_k4_item_list(6144, 2048, 73, 1, None, 0) == -1
    assert L.moe_k4_item_list(6000, 2048, 9, 1, None, 0) == -1
    buf = (ctypes.c_int32 * 5)()
    assert L.moe_k4_item_list(6144, 2048, 9, 1, buf, 1) == -1
    assert b"capacity" in L.moe_last_error()


def test_checker_catches_a_misordered_list():
    """Planted mistakes: a gate finish moved ahead of its parts, a down part ahead of its gate
    finish, a routed part ahead of the router items -- each must fail the check."""
    h, m, units = 1024, 256, 5
    items = item_list(h, m, units, 1)
    kinds = items[:, 0]

    def moved(src, dst):
        lst = items.tolist()
        lst.insert(dst, lst.pop(src))
        return np.asarray(lst, np.int32)

    first_gf = int(np.argmax(kinds == GF))
    first_routed_gu = int(np.argmax((kinds == GU) & (items[:, 1] >= 1)))
    first_down = int(np.argmax(kinds == DOWN))
    for bad in (moved(first_gf, 0), moved(first_down, first_routed_gu), moved(first_routed_gu, 0)):
        with pytest.raises(AssertionError):
            check_list(bad, h, m, units, 1)
