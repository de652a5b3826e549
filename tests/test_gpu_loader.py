"""ExpertStore / ExpertLayer.from_store on the MI355X with a synthetic layer in the up1 on-disk
layout (hidden = intermediate = 128) and the reference's resident-bytes known answer for that shape
(its tests/test_experts.py:116)."""
import sys

import numpy as np
import pytest
import torch

from conftest import bf16_bits, bits_to_f32, f16_bits, rel_l2
from loader_fixture import write_up1_layer

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.mark.parametrize("rows", [2, 20])
def test_store_layer_resident_bytes_and_forward(cuda, orc, tmp_path, rows):
    from mlxlr8_amd.experts import ExpertStore
    say(f"case: store layer rows={rows}")
    raw, index = write_up1_layer(tmp_path)
    store = ExpertStore(tmp_path, resident=True)
    layer = store.layer(3)
    assert store.layer(3) is layer
    # the reference's known answer (tests/test_experts.py:109)
    assert store.stats()["resident_bytes"] == 3 * 257 * (8192 + 2 * 128 * 2)
    assert store.stats()["hits"] == store.stats()["misses"] == 0
    for projection in ("gate", "up", "down"):
        np.testing.assert_array_equal(layer.packed[projection].cpu().numpy(), np.concatenate(
            [raw["trellis." + projection], raw["shared.trellis." + projection]]))
    rng = np.random.default_rng(30 + rows)
    ids_np = rng.integers(0, 257, (rows, 9)).astype(np.int32)
    ids_np[:, 8] = 256
    x = torch.from_numpy(rng.normal(size=(rows, 128)).astype(np.float32)).to(cuda).to(torch.bfloat16)
    values = layer(x, torch.from_numpy(ids_np).to(cuda))  # <= 16 rows: decode MLP, else grouped prefill
    torch.cuda.synchronize()
    assert values.shape == (rows, 9, 128)
    sc = {p: tuple(f16_bits(v) for v in layer.scales[p]) for p in ("gate", "up", "down")}
    host = {p: layer.packed[p].cpu().numpy() for p in ("gate", "up", "down")}
    _, want = orc.k4_moe(bf16_bits(x), ids_np.astype(np.uint32), np.zeros((rows, 8), np.float32),
                         np.zeros((rows, 128), np.uint16), 128, 128, host["gate"], host["up"], host["down"],
                         sc["gate"][0], sc["gate"][1], sc["up"][0], sc["up"][1], sc["down"][0], sc["down"][1],
                         want_values=True)
    err = rel_l2(bits_to_f32(bf16_bits(values)), bits_to_f32(want))
    say(f"  rel_l2={err:.3e}")
    assert err <= 1e-3


@pytest.mark.parametrize("rows", [2, 20])
def test_store_k3_layer_forward(cuda, orc, tmp_path, rows):
    """Layer 78 (K3): resident trellis experts (no MXFP4 conversion), values against the oracle."""
    from mlxlr8_amd.experts import ExpertStore
    say(f"case: store K3 layer 78 rows={rows}")
    write_up1_layer(tmp_path, layer=78, k=3)
    store = ExpertStore(tmp_path, resident=True, optimize=True)
    layer = store.layer(78)
    assert layer.k == 3 and layer.affine is None
    assert store.stats()["resident_bytes"] == 3 * 257 * (6144 + 2 * 128 * 2)
    rng = np.random.default_rng(40 + rows)
    ids_np = rng.integers(0, 257, (rows, 9)).astype(np.int32)
    ids_np[:, 8] = 256
    x = torch.from_numpy(rng.normal(size=(rows, 128)).astype(np.float32)).to(cuda).to(torch.bfloat16)
    values = layer(x, torch.from_numpy(ids_np).to(cuda))
    torch.cuda.synchronize()
    sc = {p: tuple(f16_bits(v) for v in layer.scales[p]) for p in ("gate", "up", "down")}
    host = {p: layer.packed[p].cpu().numpy() for p in ("gate", "up", "down")}
    _, want = orc.k4_moe(bf16_bits(x), ids_np.astype(np.uint32), np.zeros((rows, 8), np.float32),
                         np.zeros((rows, 128), np.uint16), 128, 128, host["gate"], host["up"], host["down"],
                         sc["gate"][0], sc["gate"][1], sc["up"][0], sc["up"][1], sc["down"][0], sc["down"][1],
                         want_values=True, k=3)
    err = rel_l2(bits_to_f32(bf16_bits(values)), bits_to_f32(want))
    say(f"  rel_l2={err:.3e}")
    assert err <= 1e-3
