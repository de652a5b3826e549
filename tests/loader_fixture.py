"""The reference's synthetic up1 checkpoint (its tests/test_experts.py:13-48 format): hidden =
intermediate = 128, 256 routed + 1 shared K4 expert per projection, written with safetensors.
``width`` writes the layer's files at another trellis width (K3 for the multi-token-prediction
layer 78, exlr8/experts.py:86-90)."""
import json

import numpy as np
from safetensors.numpy import save_file


def write_checkpoint(root, layer=3, widths=4, seed=17, width=4):
    directory = root / "experts"
    directory.mkdir(parents=True, exist_ok=True)
    manifests = root / "manifests"
    manifests.mkdir(parents=True, exist_ok=True)
    plan = {"gate": [[widths]] * 256, "up": [[widths]] * 256, "down": [widths] * 256,
            "shared": {"gate": [widths], "up": [widths], "down": widths}}
    (manifests / "exlr8-manifest-up1.json").write_text(json.dumps({"name": "up1", "layers": {str(layer): plan}}))
    rng = np.random.default_rng(seed)
    raw = {}
    index = {"signs.in": rng.choice([-1, 1], 128).astype(np.int8),
             "signs.out": rng.choice([-1, 1], 128).astype(np.int8)}
    for projection in ("gate", "up", "down"):
        per = 128 * 128 * width // 8
        raw["trellis." + projection] = rng.integers(0, 256, 256 * per, dtype=np.uint8)
        raw["shared.trellis." + projection] = rng.integers(0, 256, per, dtype=np.uint8)
        block_name = "sv_block" if projection == "down" else "su_block"
        channel_name = "suh" if projection == "down" else "svh"
        for prefix, count in ((f"k{width}", 256), (f"shared.k{width}", 1)):
            index[f"{prefix}.{projection}.{block_name}"] = rng.uniform(0.01, 0.02, (count, 1)).astype(np.float16)
            index[f"{prefix}.{projection}.{channel_name}"] = rng.uniform(-1, 1, (count, 128)).astype(np.float16)
    save_file(raw, str(directory / f"exlr8-layer-{layer:03d}.k{width}.safetensors"))
    save_file(index, str(directory / f"exlr8-layer-{layer:03d}.index.safetensors"))
    return raw, index
