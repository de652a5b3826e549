"""K3 experts (the multi-token-prediction layer's width) through the fused decode block: the routed
block, the decode MLP and batch-versus-single-row bits, against the oracle's K3 MoE layer."""
import sys

import numpy as np
import pytest
import torch

from conftest import bf16_bits, bits_to_f32, f16_bits, rel_l2

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def k3_layer(cuda):
    from mlxlr8_amd import synth
    from mlxlr8_amd.experts import ExpertLayer
    say("building GLM-shaped K3 layer (257 experts)")
    layer = synth.k4_layer(cuda, 3131, k=3)
    w, bias = synth.router(cuda, 3131)
    host = {p: t.cpu().numpy() for p, t in layer["packed"].items()}
    sc = {p: (f16_bits(a), f16_bits(b)) for p, (a, b) in layer["scales"].items()}
    experts = ExpertLayer(layer["packed"], layer["scales"], 6144, 2048, k=3, number=78)
    return experts, host, sc, w, bias


def _oracle_out(orc, host, sc, x, ids, scores, residual):
    return orc.k4_moe(bf16_bits(x), ids, scores, bf16_bits(residual), 6144, 2048, host["gate"], host["up"],
                      host["down"], sc["gate"][0], sc["gate"][1], sc["up"][0], sc["up"][1], sc["down"][0],
                      sc["down"][1], k=3)


@pytest.mark.parametrize("rows", [1, 8])
def test_k3_routed_decode_block(cuda, orc, k3_layer, rows):
    from mlxlr8_amd import synth
    experts, host, sc, w, bias = k3_layer
    say(f"case: K3 routed decode block rows={rows}")
    x, residual = synth.activations(cuda, 40 + rows, rows, correlated=rows > 1)
    out, ids, scores = experts.decode_block_routes(x, residual, w, bias)
    again, ids2, _ = experts.decode_block_routes(x, residual, w, bias)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), again.view(torch.int16)) and torch.equal(ids, ids2)
    logits = orc.router_logits(bf16_bits(x), w.cpu().numpy())
    oids, _ = orc.route(logits, bias.cpu().numpy())
    ids = ids.cpu().numpy().astype(np.uint32)
    mism = (ids != oids).any(axis=1)
    for r in np.where(mism)[0]:
        choice = 1 / (1 + np.exp(-logits[r].astype(np.float64))) + bias.cpu().numpy()
        srt = np.sort(choice)[::-1]
        assert srt[7] - srt[8] < 1e-5, f"row {r}: routing differs without a near tie"
    want = bits_to_f32(_oracle_out(orc, host, sc, x, ids, scores.cpu().numpy(), residual))
    got = bits_to_f32(bf16_bits(out))
    res = bits_to_f32(bf16_bits(residual))
    err, err_moe = rel_l2(got, want), rel_l2(got - res, want - res)
    say(f"  rel_l2={err:.3e} moe-part={err_moe:.3e} routing mismatches={int(mism.sum())}")
    assert err <= 1e-3 and err_moe <= 1e-3


def test_k3_decode_values_batch_equals_single_rows(cuda, orc, k3_layer):
    """Per-slot values of 5 rows in one call equal each row alone, bit for bit, and match the oracle."""
    experts, host, sc, w, bias = k3_layer
    say("case: K3 decode values, batch vs single rows")
    rng = np.random.default_rng(9)
    ids_np = np.concatenate([rng.choice(256, (5, 8), replace=True), np.full((5, 1), 256)], 1).astype(np.int32)
    ids_np[1, :3] = ids_np[0, :3]  # shared experts across rows
    ids = torch.from_numpy(ids_np).to(cuda)
    x = torch.from_numpy(rng.normal(size=(5, 6144)).astype(np.float32)).to(cuda).to(torch.bfloat16)
    batch = experts(x, ids)
    singles = torch.cat([experts(x[r:r + 1], ids[r:r + 1]) for r in range(5)])
    torch.cuda.synchronize()
    assert torch.equal(batch.view(torch.int16), singles.view(torch.int16))
    _, want = orc.k4_moe(bf16_bits(x), ids_np.astype(np.uint32), np.zeros((5, 8), np.float32),
                         np.zeros((5, 6144), np.uint16), 6144, 2048, host["gate"], host["up"], host["down"],
                         sc["gate"][0], sc["gate"][1], sc["up"][0], sc["up"][1], sc["down"][0], sc["down"][1],
                         want_values=True, k=3)
    err = rel_l2(bits_to_f32(bf16_bits(batch)).reshape(5, 9, 6144), bits_to_f32(want).reshape(5, 9, 6144))
    say(f"  values rel_l2={err:.3e}")
    assert err <= 1e-3
