"""A synthetic up1 expert layer written in its on-disk layout (manifest, trellis file, index file),
for the loader tests.  Sizes: `hidden` x `intermediate`, 256 routed experts plus the shared one,
trellis width `k` (packed bytes random: every bitstream is a valid trellis); `plan_width` is the
width the manifest claims (a mismatch exercises the loader's uniform-width check)."""
import json

import numpy as np
from safetensors.numpy import save_file

ROUTED = 256


def _plan(width):
    routed = {"gate": [[width]] * ROUTED, "up": [[width]] * ROUTED, "down": [width] * ROUTED}
    return dict(routed, shared={"gate": [width], "up": [width], "down": width})


def write_up1_layer(root, layer=3, k=4, hidden=128, intermediate=128, plan_width=None, seed=5):
    """Write layer `layer` under `root`; returns (trellis tensors, index tensors) as numpy dicts."""
    gen = np.random.default_rng([seed, layer, k])
    (root / "manifests").mkdir(parents=True, exist_ok=True)
    (root / "experts").mkdir(parents=True, exist_ok=True)
    manifest = root / "manifests" / "exlr8-manifest-up1.json"
    layers = json.loads(manifest.read_text())["layers"] if manifest.exists() else {}
    layers[str(layer)] = _plan(k if plan_width is None else plan_width)
    manifest.write_text(json.dumps({"name": "up1", "layers": layers}))

    expert_bytes = hidden * intermediate * k // 8
    trellis, index = {}, {}
    for side_name, n in (("signs.in", hidden), ("signs.out", hidden)):
        index[side_name] = np.where(gen.random(n) < 0.5, -1, 1).astype(np.int8)
    for projection in ("gate", "up", "down"):
        packed = gen.integers(0, 256, (ROUTED + 1) * expert_bytes, dtype=np.uint8)
        trellis[f"trellis.{projection}"] = packed[:ROUTED * expert_bytes]
        trellis[f"shared.trellis.{projection}"] = packed[ROUTED * expert_bytes:]
        # gate/up: a magnitude per 128 input channels (hidden) and a per-output-channel vector
        # (intermediate); down: a magnitude per 128 output channels (hidden) and a per-input-channel
        # vector (intermediate)
        blocks, channels = hidden // 128, intermediate
        block_name, channel_name = ("sv_block", "suh") if projection == "down" else ("su_block", "svh")
        mags = np.exp(gen.normal(np.log(0.015), 0.2, (ROUTED + 1, blocks))).astype(np.float16)
        chans = gen.normal(0.0, 0.5, (ROUTED + 1, channels)).astype(np.float16)
        for prefix, rows in ((f"k{k}", slice(0, ROUTED)), (f"shared.k{k}", slice(ROUTED, ROUTED + 1))):
            index[f"{prefix}.{projection}.{block_name}"] = mags[rows]
            index[f"{prefix}.{projection}.{channel_name}"] = chans[rows]
    save_file(trellis, str(root / "experts" / f"exlr8-layer-{layer:03d}.k{k}.safetensors"))
    save_file(index, str(root / "experts" / f"exlr8-layer-{layer:03d}.index.safetensors"))
    return trellis, index
