"""moe_mxfp4_moe_decode_noalloc (the allocation-free decode block) against moe_mxfp4_moe_decode on
the same inputs, through the C ABI: bit-identical outputs, ids and scores on two calls in a row,
the second with fewer rows; shapes beyond the fixed scratch and bad row counts are rejected."""
import sys

import pytest
import torch

pytestmark = pytest.mark.gpu

H, M = 6144, 2048


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _same(a, b):
    return torch.equal(a.contiguous().view(torch.uint8), b.contiguous().view(torch.uint8))


def test_noalloc_decode_block_matches_workspace_entry(cuda):
    from mlxlr8_amd import synth
    from mlxlr8_amd._lib import check, lib, ptr, stream
    say("case: allocation-free MXFP4 decode block vs the workspace entry, rows 8 then 1")
    L = synth.mxfp4_layer(cuda, 919)
    w, bias = synth.router(cuda, 919)
    (gc, gs), (dc, ds) = L["weights"]["gate_up"], L["weights"]["down"]
    sd = L["side"]
    weights = [ptr(gc), ptr(gs), ptr(dc), ptr(ds), 257, ptr(L["unit"]), ptr(sd["out_gate"]), ptr(sd["out_up"]),
               ptr(sd["in_down"]), ptr(sd["out_down"]), H, M]
    ws = torch.zeros(lib().moe_mxfp4_workspace_bytes(H, M), dtype=torch.uint8, device=cuda)
    for rows in (8, 1):
        x, res = synth.activations(cuda, 920 + rows, rows)
        got = {}
        for kind in ("workspace", "noalloc"):
            out = torch.empty((rows, H), dtype=torch.bfloat16, device=cuda)
            ids = torch.empty((rows, 9), dtype=torch.int32, device=cuda)
            sc = torch.empty((rows, 8), dtype=torch.float32, device=cuda)
            args = [ptr(x), ptr(res), rows, ptr(w), ptr(bias)] + weights + [ptr(out), ptr(ids), ptr(sc)]
            if kind == "workspace":
                check(lib().moe_mxfp4_moe_decode(*args, ptr(ws), ws.numel(), stream(cuda)))
            else:
                check(lib().moe_mxfp4_moe_decode_noalloc(*args, stream(cuda)))
            got[kind] = (out, ids, sc)
        torch.cuda.synchronize()
        for a, b in zip(got["workspace"], got["noalloc"]):
            assert _same(a, b)
        say(f"  rows={rows}: identical")
    # rejected before any launch: a shape whose workspace exceeds the fixed scratch, 9 rows
    x, res = synth.activations(cuda, 930, 1)
    out = torch.empty((1, H), dtype=torch.bfloat16, device=cuda)
    big = [ptr(gc), ptr(gs), ptr(dc), ptr(ds), 257, ptr(L["unit"]), ptr(sd["out_gate"]), ptr(sd["out_up"]),
           ptr(sd["in_down"]), ptr(sd["out_down"]), 65536, M]
    rc = lib().moe_mxfp4_moe_decode_noalloc(ptr(x), ptr(res), 1, ptr(w), ptr(bias), *big, ptr(out), None, None,
                                            stream(cuda))
    assert rc == -2 and b"scratch" in lib().moe_last_error()
    rc = lib().moe_mxfp4_moe_decode_noalloc(ptr(x), ptr(res), 9, ptr(w), ptr(bias), *weights, ptr(out), None, None,
                                            stream(cuda))
    assert rc == -1
