"""up1 checkpoint loading (exlr8/weights.py, exlr8/experts.py:12-131) on the reference's synthetic
checkpoint format, without a GPU."""
import json

import numpy as np
import pytest

from loader_fixture import write_checkpoint


@pytest.fixture
def checkpoint(tmp_path):
    raw, index = write_checkpoint(tmp_path)
    return tmp_path, raw, index


def test_safetensor_ranges_and_shapes(checkpoint):
    from mlxlr8_amd.weights import SafeTensorFile
    path, raw, index = checkpoint
    f = SafeTensorFile(path / "experts" / "exlr8-layer-003.k4.safetensors")
    for expert in (4, 8, 255):
        np.testing.assert_array_equal(f.raw("trellis.gate", expert * 8192, 8192),
                                      raw["trellis.gate"][expert * 8192:(expert + 1) * 8192])
    np.testing.assert_array_equal(f.raw("shared.trellis.down"), raw["shared.trellis.down"])
    g = SafeTensorFile(path / "experts" / "exlr8-layer-003.index.safetensors")
    assert g.raw("k4.gate.svh").shape == (256, 128) and g.raw("k4.gate.svh").dtype == np.float16
    np.testing.assert_array_equal(g.raw("signs.in"), index["signs.in"])
    with pytest.raises(ValueError):
        f.raw("trellis.gate", 256 * 8192 - 4, 8)  # past the end
    with pytest.raises(ValueError):
        g.raw("k4.gate.svh", 1, 2)  # not whole fp16 elements


def test_side_vectors_and_packed(checkpoint):
    from mlxlr8_amd.experts import layer_arrays
    path, raw, index = checkpoint
    k, hidden, inter, packed, scales = layer_arrays(path, 3)
    assert (k, hidden, inter) == (4, 128, 128)
    for projection in ("gate", "up", "down"):
        np.testing.assert_array_equal(packed[projection], np.concatenate(
            [raw["trellis." + projection], raw["shared.trellis." + projection]]))
    signs_in = index["signs.in"].astype(np.float64)
    signs_out = index["signs.out"].astype(np.float64)
    for projection in ("gate", "up"):
        incoming, outgoing = scales[projection]
        block = np.concatenate([index[f"k4.{projection}.su_block"], index[f"shared.k4.{projection}.su_block"]])
        assert incoming.shape == (257, 128) and incoming.dtype == np.float16
        # element i of expert e: its 128-block's scale times the input channel's sign
        np.testing.assert_array_equal(incoming.astype(np.float64), block.astype(np.float64)[:, [0] * 128] * signs_in)
        np.testing.assert_array_equal(outgoing[:256], index[f"k4.{projection}.svh"])
        np.testing.assert_array_equal(outgoing[256], index[f"shared.k4.{projection}.svh"][0])
    incoming, outgoing = scales["down"]
    np.testing.assert_array_equal(incoming[:256], index["k4.down.suh"])
    block = np.concatenate([index["k4.down.sv_block"], index["shared.k4.down.sv_block"]])
    np.testing.assert_array_equal(outgoing.astype(np.float64), block.astype(np.float64)[:, [0] * 128] * signs_out)


def test_manifest_and_width_errors(tmp_path):
    from mlxlr8_amd.experts import layer_arrays
    write_checkpoint(tmp_path, layer=5, widths=3)
    with pytest.raises(ValueError, match="not uniform K4"):
        layer_arrays(tmp_path, 5)
    m = tmp_path / "manifests" / "exlr8-manifest-up1.json"
    data = json.loads(m.read_text())
    data["name"] = "up2"
    m.write_text(json.dumps(data))
    with pytest.raises(ValueError, match="up1 manifest"):
        layer_arrays(tmp_path, 5)


def test_k3_layer_78(tmp_path):
    """Layer 78 is the K3 layer: its k3 file and k3 side vectors load with k = 3."""
    from mlxlr8_amd.experts import layer_arrays
    raw, index = write_checkpoint(tmp_path, layer=78, widths=3, width=3)
    k, hidden, inter, packed, scales = layer_arrays(tmp_path, 78)
    assert (k, hidden, inter) == (3, 128, 128)
    for projection in ("gate", "up", "down"):
        assert packed[projection].size == 257 * 128 * 128 * 3 // 8
        np.testing.assert_array_equal(packed[projection][:256 * 6144], raw["trellis." + projection])
    np.testing.assert_array_equal(scales["gate"][1][:256], index["k3.gate.svh"])
    np.testing.assert_array_equal(scales["down"][0][256], index["shared.k3.down.suh"][0])
    # a K4 manifest row at layer 78 is rejected
    write_checkpoint(tmp_path, layer=78, widths=4, width=4)
    with pytest.raises(ValueError, match="not uniform K3"):
        layer_arrays(tmp_path, 78)
