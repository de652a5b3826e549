"""Resident trellis expert layer (mirrors the reference ``exlr8/experts.py`` ExpertLayer).

The reference loads packed experts from safetensors; this class takes device tensors that
are already resident in HBM (288 GB per MI355X holds every expert of many layers), so the
SSD cache paths of the reference do not exist here.
"""
from types import SimpleNamespace

import torch

from ._lib import check, lib, ptr, require_cuda, stream, workspace
from .fast_decode import _weights, expert_values
from .trellis import BF16, _check_format


class ExpertLayer:
    """Packed gate/up/down trellis experts of one MoE layer (routed experts + shared expert last).

    Attributes mirror the reference (exlr8/experts.py:76-148): ``k``, ``hidden``,
    ``intermediate``, ``store.resident``, ``store.optimize``, ``packed`` (dict),
    ``scales`` (dict of (in, out) pairs), ``affine``, ``expert_bytes``.
    """

    def __init__(self, packed, scales, hidden, intermediate, k=4, number=0):
        if k not in (2, 3, 4):
            raise ValueError("EXLR8 trellis width must be 2, 3, or 4")
        self.k, self.hidden, self.intermediate, self.number = k, hidden, intermediate, number
        self.expert_bytes = hidden * intermediate * k // 8
        self.store = SimpleNamespace(resident=True, optimize=True)
        self.affine = None
        self.packed = dict(packed)
        self.scales = {p: tuple(v) for p, v in scales.items()}
        for projection in ("gate", "up", "down"):
            a, b, side = (intermediate, hidden, 2) if projection == "down" else (hidden, intermediate, 1)
            experts = _check_format(self.packed[projection], k, a, b, side)
            if experts != self.experts:
                raise ValueError("gate, up and down must hold the same experts")
        require_cuda(*self.packed.values())

    @property
    def experts(self):
        return _check_format(self.packed["gate"], self.k, self.hidden, self.intermediate, 1)

    def __call__(self, x, ids):
        """values[*ids.shape, hidden] for the selected experts (exlr8/experts.py:150-188): up to 16
        rows through the decode MLP, more through the grouped (sorted-by-expert) prefill MLP (K2/K3
        experts take the grouped MLP at every row count)."""
        if self.affine is not None:
            return self.affine.slots(x, ids)
        return expert_values(x, ids, self.packed, self.scales, self.k, self.hidden, self.intermediate)

    def decode_block(self, x, residual, router_weight, bias):
        """Router GEMV + route + expert MLP + combine in one C call (decode batches, <= 8 rows).

        Returns residual + routed + shared; exlr8/fast_router.py:27-37 compiled_finish(...).call.
        """
        out, _, _ = self.decode_block_routes(x, residual, router_weight, bias)
        return out

    def prepare_decode(self, x, residual, router_weight, bias):
        """Bind device buffers once and return a zero-argument callable that enqueues the whole
        decode block (one C call, no per-call tensor work); results land in `.out`, `.ids`, `.scores`."""
        h = self.hidden
        rows = x.numel() // h
        if rows > 8 or self.experts != 257 or x.dtype != BF16 or self.k != 4:
            raise ValueError("prepare_decode needs <= 8 bf16 rows and 256 routed + 1 shared K4 experts")
        require_cuda(x, residual, router_weight, bias)
        call = SimpleNamespace()
        call.x = x.reshape(rows, h).contiguous()
        call.residual = residual.reshape(rows, h).to(BF16).contiguous()
        call.w = router_weight.to(torch.float32).contiguous()
        call.bias = bias.to(torch.float32).contiguous()
        call.out = torch.empty((rows, h), dtype=BF16, device=x.device)
        call.ids = torch.empty((rows, 9), dtype=torch.int32, device=x.device)
        call.scores = torch.empty((rows, 8), dtype=torch.float32, device=x.device)
        ws = workspace(x.device, h, self.intermediate)
        args = (ptr(call.x), ptr(call.residual), rows, ptr(call.w), ptr(call.bias), *_weights(self.packed, self.scales),
                h, self.intermediate, ptr(call.out), ptr(call.ids), ptr(call.scores), ptr(ws), ws.numel(),
                stream(x.device))
        fn = lib().moe_k4_moe_decode

        def run():
            check(fn(*args))
            return call.out

        call.run = run
        return call

    def prepare_layer_decode(self, x, norm_weight, router_weight, bias, attn=None, eps=1e-5):
        """Like prepare_decode for a whole decode layer's MoE half: h = T(x + attn), the routed
        block runs on rms_norm(h, norm_weight) with residual h (one C call per run).  `x` is bound
        by reference, so a stack can feed one layer's `.out` to the next layer's `x`."""
        h = self.hidden
        rows = x.numel() // h
        if rows > 8 or self.experts != 257 or x.dtype != BF16 or self.k != 4:
            raise ValueError("prepare_layer_decode needs <= 8 bf16 rows and 256 routed + 1 shared K4 experts")
        if not x.is_contiguous():
            raise ValueError("the layer input must be contiguous (it is bound by address)")
        require_cuda(x, norm_weight, router_weight, bias)
        call = SimpleNamespace()
        call.x = x
        call.attn = attn.reshape(rows, h).to(BF16).contiguous() if attn is not None else None
        call.norm = norm_weight.to(BF16).contiguous()
        call.w = router_weight.to(torch.float32).contiguous()
        call.bias = bias.to(torch.float32).contiguous()
        call.out = torch.empty((rows, h), dtype=BF16, device=x.device)
        call.ids = torch.empty((rows, 9), dtype=torch.int32, device=x.device)
        call.scores = torch.empty((rows, 8), dtype=torch.float32, device=x.device)
        ws = workspace(x.device, h, self.intermediate)
        args = (ptr(x), ptr(call.attn) if call.attn is not None else None, ptr(call.norm), float(eps), rows,
                ptr(call.w), ptr(call.bias), *_weights(self.packed, self.scales), h, self.intermediate,
                ptr(call.out), ptr(call.ids), ptr(call.scores), ptr(ws), ws.numel(), stream(x.device))
        fn = lib().moe_k4_layer_decode

        def run():
            check(fn(*args))
            return call.out

        call.run = run
        return call

    def layer_decode(self, x, norm_weight, router_weight, bias, attn=None, eps=1e-5):
        """One-shot form of prepare_layer_decode: returns (out, indices [rows,9], scores [rows,8])."""
        h = self.hidden
        xr = x.reshape(x.numel() // h, h).to(BF16).contiguous()
        call = self.prepare_layer_decode(xr, norm_weight, router_weight, bias, attn, eps)
        call.run()
        return call.out.reshape(x.shape), call.ids, call.scores

    def decode_block_routes(self, x, residual, router_weight, bias):
        h = self.hidden
        rows = x.numel() // h
        if rows > 8:
            raise ValueError("decode_block handles up to 8 token rows")
        if self.experts != 257 or self.k != 4:
            raise ValueError("decode_block needs 256 routed K4 experts plus the shared expert")
        if x.dtype != BF16:
            raise ValueError("this build computes bf16 activations")
        require_cuda(x, residual, router_weight, bias)
        xr = x.reshape(rows, h).contiguous()
        res = residual.reshape(rows, h).to(BF16).contiguous()
        w = router_weight.to(torch.float32).contiguous()
        b = bias.to(torch.float32).contiguous()
        out = torch.empty((rows, h), dtype=BF16, device=x.device)
        ids = torch.empty((rows, 9), dtype=torch.int32, device=x.device)
        scores = torch.empty((rows, 8), dtype=torch.float32, device=x.device)
        ws = workspace(x.device, h, self.intermediate)
        check(lib().moe_k4_moe_decode(ptr(xr), ptr(res), rows, ptr(w), ptr(b), *_weights(self.packed, self.scales),
                                      h, self.intermediate, ptr(out), ptr(ids), ptr(scores), ptr(ws), ws.numel(),
                                      stream(x.device)))
        return out.reshape(residual.shape), ids, scores


# ---------------------------------------------------------------- checkpoint loading
def layer_arrays(path, number):
    """Host arrays of one up1 layer (exlr8/experts.py:80-131): ``(k, hidden, intermediate, packed,
    scales)`` with ``packed[p]`` = routed experts then the shared expert (uint8) and ``scales[p]`` =
    (in, out) fp16 [257, features]: gate/up in = su_block per 128-block x signs.in, out = svh;
    down in = suh, out = sv_block per 128-block x signs.out."""
    import json
    from pathlib import Path

    import numpy as np

    from .weights import SafeTensorFile
    path = Path(path)
    manifest = json.loads((path / "manifests/exlr8-manifest-up1.json").read_text())
    if manifest["name"] != "up1":
        raise ValueError("This loader requires the up1 manifest")
    plan = manifest["layers"][str(number)]
    widths = {v for rows in (plan["gate"], plan["up"]) for row in rows for v in row}
    widths.update(plan["down"])
    widths.update(plan["shared"]["gate"])
    widths.update(plan["shared"]["up"])
    widths.add(plan["shared"]["down"])
    k = 3 if number == 78 else 4
    if widths != {k}:
        raise ValueError(f"Layer {number} is not uniform K{k}")
    directory = path / "experts"
    weights = SafeTensorFile(directory / f"exlr8-layer-{number:03d}.k{k}.safetensors")
    index = SafeTensorFile(directory / f"exlr8-layer-{number:03d}.index.safetensors")
    hidden = index.header["signs.in"]["shape"][0]
    intermediate = index.header[f"k{k}.gate.svh"]["shape"][-1]
    signs_in = index.raw("signs.in").astype(np.float16)
    signs_out = index.raw("signs.out").astype(np.float16)
    scales, packed = {}, {}
    for projection in ("gate", "up", "down"):
        down = projection == "down"
        block_name, channel_name = ("sv_block", "suh") if down else ("su_block", "svh")
        block = np.concatenate([index.raw(f"k{k}.{projection}.{block_name}"),
                                index.raw(f"shared.k{k}.{projection}.{block_name}")])
        channel = np.concatenate([index.raw(f"k{k}.{projection}.{channel_name}"),
                                  index.raw(f"shared.k{k}.{projection}.{channel_name}")])
        hidden_scale = np.repeat(block, 128, axis=-1) * (signs_out if down else signs_in)
        scales[projection] = (channel, hidden_scale) if down else (hidden_scale, channel)
        packed[projection] = np.concatenate([weights.raw("trellis." + projection),
                                             weights.raw("shared.trellis." + projection)])
    return k, hidden, intermediate, packed, scales


class ExpertStore:
    """Resident up1 expert store (exlr8/experts.py:12-76).  On an MI355X every layer's experts fit in
    HBM, so layers are always loaded resident; ``cache_gib`` is accepted for signature parity and
    ``resident=False`` loads resident as well (the reference's SSD cache is not built)."""

    def __init__(self, path, cache_gib=32, resident=False, optimize=True, device=None):
        import json
        from pathlib import Path
        self.path = Path(path)
        self.resident, self.optimize = True, optimize
        self.manifest = json.loads((self.path / "manifests/exlr8-manifest-up1.json").read_text())
        if self.manifest["name"] != "up1":
            raise ValueError("This loader requires the up1 manifest")
        if cache_gib < 0:
            raise ValueError("cache_gib must be nonnegative")
        self.limit = int(cache_gib * 1024 ** 3)
        self.device = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
        self.cache, self.cache_bytes, self.hits, self.misses = {}, 0, 0, 0
        self.resident_bytes = 0
        self._layers = {}

    def layer(self, number):
        if number not in self._layers:
            self._layers[number] = ExpertLayer.from_store(self, number)
        return self._layers[number]

    def stats(self):
        return {"cache_bytes": self.cache_bytes, "cache_limit_bytes": self.limit,
                "resident_bytes": self.resident_bytes, "hits": self.hits, "misses": self.misses}


def _from_store(cls, store, number):
    """ExpertLayer of layer `number` of an ExpertStore, resident on the store's device; with
    ``optimize``, K4 and the GLM-5.3 shape (6144, 2048) its experts are converted to joined MXFP4
    and served by them (exlr8/experts.py:132-148); K3 layers stay trellis."""
    k, hidden, intermediate, packed, scales = layer_arrays(store.path, number)
    dev = store.device
    layer = cls({p: torch.from_numpy(a).to(dev) for p, a in packed.items()},
                {p: tuple(torch.from_numpy(v).to(dev) for v in pair) for p, pair in scales.items()},
                hidden, intermediate, k=k, number=number)
    layer.store = store
    store.resident_bytes += sum(a.nbytes for a in packed.values())
    store.resident_bytes += sum(v.nbytes for pair in scales.values() for v in pair)
    if store.optimize and k == 4 and (hidden, intermediate) == (6144, 2048):
        from .joined_mxfp4 import JoinedMXFP4
        layer.affine = JoinedMXFP4(layer)
        store.resident_bytes += (sum(a.numel() * a.element_size() for v in layer.affine.weights.values() for a in v)
                                 - sum(a.nbytes for a in packed.values()) + layer.affine.unit.numel() * 2)
        for projection in ("gate", "up"):
            incoming, outgoing = layer.scales[projection]
            store.resident_bytes -= incoming.numel() * incoming.element_size()
            layer.scales[projection] = (None, outgoing)
        del layer.packed
    return layer


ExpertLayer.from_store = classmethod(_from_store)
