"""up1 checkpoint loading (the reference's exlr8/weights.py and exlr8/experts.py:77-131 behaviour)
on a synthetic layer in the up1 on-disk layout, without a GPU."""
import json
import struct

import numpy as np
import pytest

from loader_fixture import write_up1_layer


@pytest.fixture
def checkpoint(tmp_path):
    trellis, index = write_up1_layer(tmp_path)
    return tmp_path, trellis, index


def test_safetensors_arrays_and_spans(checkpoint):
    from mlxlr8_amd.weights import SafetensorsFile
    path, trellis, index = checkpoint
    f = SafetensorsFile(path / "experts" / "exlr8-layer-003.k4.safetensors")
    for expert in (0, 4, 255):
        np.testing.assert_array_equal(f.span("trellis.gate", expert * 8192, 8192),
                                      trellis["trellis.gate"][expert * 8192:(expert + 1) * 8192])
    np.testing.assert_array_equal(f.array("shared.trellis.down"), trellis["shared.trellis.down"])
    g = SafetensorsFile(path / "experts" / "exlr8-layer-003.index.safetensors")
    assert g.shape("k4.gate.svh") == (256, 128) and g.array("k4.gate.svh").dtype == np.float16
    np.testing.assert_array_equal(g.array("signs.in"), index["signs.in"])
    assert sorted(g.names) == sorted(index)
    with pytest.raises(ValueError):
        f.span("trellis.gate", 256 * 8192 - 4, 8)  # past the end
    with pytest.raises(ValueError):
        g.span("k4.gate.svh", 1, 2)  # splits an fp16 element
    with pytest.raises(KeyError):
        g.array("no.such.tensor")


def _write_raw(path, header, data=b""):
    blob = json.dumps(header).encode()
    path.write_bytes(struct.pack("<Q", len(blob)) + blob + data)


def test_safetensors_header_validation(tmp_path):
    from mlxlr8_amd.weights import SafetensorsFile
    p = tmp_path / "bad.safetensors"
    _write_raw(p, {"a": {"dtype": "F16", "shape": [4], "data_offsets": [0, 6]}}, bytes(8))
    with pytest.raises(ValueError, match="byte range"):  # 4 x fp16 is 8 bytes, not 6
        SafetensorsFile(p)
    _write_raw(p, {"a": {"dtype": "U8", "shape": [4], "data_offsets": [0, 4]},
                   "b": {"dtype": "U8", "shape": [4], "data_offsets": [2, 6]}}, bytes(8))
    with pytest.raises(ValueError, match="overlap"):
        SafetensorsFile(p)
    _write_raw(p, {"a": {"dtype": "U8", "shape": [16], "data_offsets": [0, 16]}}, bytes(8))
    with pytest.raises(ValueError, match="byte range"):  # past the end of the file
        SafetensorsFile(p)
    _write_raw(p, {"a": {"dtype": "Q4", "shape": [2], "data_offsets": [0, 2]}}, bytes(2))
    with pytest.raises(ValueError, match="malformed"):
        SafetensorsFile(p)
    p.write_bytes(struct.pack("<Q", 1 << 40))
    with pytest.raises(ValueError, match="header length"):
        SafetensorsFile(p)
    _write_raw(p, {"__metadata__": {"format": "pt"}, "a": {"dtype": "BF16", "shape": [2], "data_offsets": [0, 4]}},
               bytes([0, 0x3F, 0x80, 0xBF]))
    f = SafetensorsFile(p)
    assert f.metadata == {"format": "pt"}
    import torch
    assert f.tensor("a").tolist() == [0.5, -1.0]


def test_side_vectors_and_packed(checkpoint):
    from mlxlr8_amd.experts import layer_arrays
    path, trellis, index = checkpoint
    k, hidden, inter, packed, scales = layer_arrays(path, 3)
    assert (k, hidden, inter) == (4, 128, 128)
    for projection in ("gate", "up", "down"):
        np.testing.assert_array_equal(packed[projection], np.concatenate(
            [trellis["trellis." + projection], trellis["shared.trellis." + projection]]))
    signs_in = index["signs.in"].astype(np.float64)
    signs_out = index["signs.out"].astype(np.float64)
    for projection in ("gate", "up"):
        incoming, outgoing = scales[projection]
        block = np.concatenate([index[f"k4.{projection}.su_block"], index[f"shared.k4.{projection}.su_block"]])
        assert incoming.shape == (257, 128) and incoming.dtype == np.float16
        # element i of expert e: its 128-block's magnitude times the input channel's sign
        np.testing.assert_array_equal(incoming.astype(np.float64), block.astype(np.float64)[:, [0] * 128] * signs_in)
        np.testing.assert_array_equal(outgoing[:256], index[f"k4.{projection}.svh"])
        np.testing.assert_array_equal(outgoing[256], index[f"shared.k4.{projection}.svh"][0])
    incoming, outgoing = scales["down"]
    np.testing.assert_array_equal(incoming[:256], index["k4.down.suh"])
    block = np.concatenate([index["k4.down.sv_block"], index["shared.k4.down.sv_block"]])
    np.testing.assert_array_equal(outgoing.astype(np.float64), block.astype(np.float64)[:, [0] * 128] * signs_out)


def test_manifest_and_width_errors(tmp_path):
    from mlxlr8_amd.experts import layer_arrays
    write_up1_layer(tmp_path, layer=5, plan_width=3)
    with pytest.raises(ValueError, match="not uniform K4"):
        layer_arrays(tmp_path, 5)
    m = tmp_path / "manifests" / "exlr8-manifest-up1.json"
    data = json.loads(m.read_text())
    data["name"] = "up2"
    m.write_text(json.dumps(data))
    with pytest.raises(ValueError, match="up1 manifest"):
        layer_arrays(tmp_path, 5)


def test_plan_metadata_keys_are_not_widths(tmp_path):
    """A layer plan may carry keys besides the projections' widths (numbers or strings, at the top
    or inside ``shared``): they are not widths and do not fail the uniform-width check."""
    from mlxlr8_amd.experts import layer_arrays
    write_up1_layer(tmp_path, layer=6)
    m = tmp_path / "manifests" / "exlr8-manifest-up1.json"
    data = json.loads(m.read_text())
    plan = data["layers"]["6"]
    plan["bits_per_weight"] = 4.05
    plan["note"] = "calibrated"
    plan["shared"]["source"] = "shared-expert"
    plan["stats"] = {"mse": [0.1, 0.2]}
    m.write_text(json.dumps(data))
    k, hidden, inter, packed, scales = layer_arrays(tmp_path, 6)
    assert (k, hidden, inter) == (4, 128, 128)
    # a width of 3 inside the projections is still caught
    plan["down"][7] = 3
    m.write_text(json.dumps(data))
    with pytest.raises(ValueError, match="not uniform K4"):
        layer_arrays(tmp_path, 6)


def test_k3_layer_78(tmp_path):
    """Layer 78 is the K3 layer: its k3 file and k3 side vectors load with k = 3."""
    from mlxlr8_amd.experts import layer_arrays
    trellis, index = write_up1_layer(tmp_path, layer=78, k=3)
    k, hidden, inter, packed, scales = layer_arrays(tmp_path, 78)
    assert (k, hidden, inter) == (3, 128, 128)
    for projection in ("gate", "up", "down"):
        assert packed[projection].size == 257 * 128 * 128 * 3 // 8
        np.testing.assert_array_equal(packed[projection][:256 * 6144], trellis["trellis." + projection])
    np.testing.assert_array_equal(scales["gate"][1][:256], index["k3.gate.svh"])
    np.testing.assert_array_equal(scales["down"][0][256], index["shared.k3.down.suh"][0])
    # a manifest claiming K4 at layer 78 is rejected
    write_up1_layer(tmp_path, layer=78, k=3, plan_width=4)
    with pytest.raises(ValueError, match="not uniform K3"):
        layer_arrays(tmp_path, 78)
