"""Resident trellis expert layer (mirrors the reference ``exlr8/experts.py`` ExpertLayer).

The reference loads packed experts from safetensors; this class takes device tensors that
are already resident in HBM (288 GB per MI355X holds every expert of many layers), so the
SSD cache paths of the reference do not exist here.
"""
from types import SimpleNamespace

import torch

from ._lib import check, lib, ptr, require_cuda, stream, workspace
from .fast_decode import _weights, expert_values
from .trellis import BF16, _check_format, expert_linear, swiglu


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
        """values[*ids.shape, hidden] for the selected experts (exlr8/experts.py:150-188).

        With ``store.optimize`` (the default) up to 16 rows run through the decode MLP and more
        through the grouped (sorted-by-expert) prefill MLP; K2/K3 experts take the grouped MLP at
        every row count.  With ``store.optimize = False`` the layer runs the reference's plain
        chain instead: gate and up expert linears, SwiGLU, down expert linear
        (exlr8/experts.py:176-188)."""
        if self.affine is not None:
            return self.affine.slots(x, ids)
        if self.store.optimize:
            return expert_values(x, ids, self.packed, self.scales, self.k, self.hidden, self.intermediate)
        gate, up = (expert_linear(x, ids, self.packed[p], *self.scales[p], self.k, self.hidden, self.intermediate, 1)
                    for p in ("gate", "up"))
        hidden = swiglu(gate, up)
        return expert_linear(hidden, ids, self.packed["down"], *self.scales["down"], self.k, self.intermediate,
                             self.hidden, 2)

    def decode_block(self, x, residual, router_weight, bias):
        """Router GEMV + route + expert MLP + combine in one C call (decode batches, <= 8 rows).

        Returns residual + routed + shared; exlr8/fast_router.py:27-37 compiled_finish(...).call.
        """
        out, _, _ = self.decode_block_routes(x, residual, router_weight, bias)
        return out

    def prepare_decode(self, x, residual, router_weight, bias):
        """Bind device buffers once and return a zero-argument callable that enqueues the whole
        decode block (one C call, no per-call tensor work); results land in `.out`, `.ids`, `.scores`.
        The call runs on the stream that is current now (its workspace belongs to that stream)."""
        h = self.hidden
        rows = x.numel() // h
        if rows > 8 or self.experts != 257 or x.dtype != BF16 or self.k not in (3, 4):
            raise ValueError("prepare_decode needs <= 8 bf16 rows and 256 routed + 1 shared K3 or K4 experts")
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
        if self.k == 4:
            fn = lib().moe_k4_moe_decode
        else:
            k, fn3 = self.k, lib().moe_trellis_moe_decode
            fn = lambda *a: fn3(k, *a)

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
        if self.experts != 257 or self.k not in (3, 4):
            raise ValueError("decode_block needs 256 routed K3 or K4 experts plus the shared expert")
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
        args = (ptr(xr), ptr(res), rows, ptr(w), ptr(b), *_weights(self.packed, self.scales), h, self.intermediate,
                ptr(out), ptr(ids), ptr(scores), ptr(ws), ws.numel(), stream(x.device))
        check(lib().moe_k4_moe_decode(*args) if self.k == 4 else lib().moe_trellis_moe_decode(self.k, *args))
        return out.reshape(residual.shape), ids, scores


# ---------------------------------------------------------------- checkpoint loading
#
# The up1 expert checkpoint (the reference's layout, README.md:62-72 and exlr8/experts.py:77-131):
#   manifests/exlr8-manifest-up1.json     {"name": "up1", "layers": {"<n>": plan}}; every trellis
#                                          width listed in a layer's plan must be that layer's K
#   experts/exlr8-layer-<nnn>.k<K>.safetensors    trellis.<p> (256 routed experts, concatenated)
#                                                  and shared.trellis.<p> (the shared expert)
#   experts/exlr8-layer-<nnn>.index.safetensors   signs.in [hidden], signs.out [hidden] (int8),
#                                                  per projection a per-128-block magnitude and a
#                                                  per-channel vector, routed (k<K>.*) and shared
#                                                  (shared.k<K>.*)
# Every layer is K4 except the multi-token-prediction layer 78, which is K3.

MTP_LAYER, MTP_WIDTH, MAIN_WIDTH = 78, 3, 4

# Per projection: (block tensor, channel tensor, signs tensor, side the block vector scales).
# The block vector, repeated over its 128 channels and signed, is the in-scale of gate/up and the
# out-scale of down; the channel vector is the other side (exlr8/experts.py:99-115).
SIDE_VECTORS = {
    "gate": ("su_block", "svh", "signs.in", "in"),
    "up": ("su_block", "svh", "signs.in", "in"),
    "down": ("sv_block", "suh", "signs.out", "out"),
}


def _flat(node):
    """The numbers of a nested list (or a single number)."""
    if isinstance(node, (list, tuple)):
        return set().union(*(_flat(v) for v in node)) if node else set()
    return {int(node)}


def _widths(plan):
    """The trellis widths a manifest layer plan assigns to the expert projections: the routed
    experts' ``gate``, ``up`` and ``down`` entries and the shared expert's (``shared``).  Other keys
    of a plan (metadata) are not widths and are ignored (exlr8/experts.py:81-85 reads the same six)."""
    shared = plan["shared"]
    return set().union(*(_flat(plan[p]) for p in ("gate", "up", "down")),
                       *(_flat(shared[p]) for p in ("gate", "up", "down")))


def _manifest(path):
    import json
    manifest = json.loads((path / "manifests" / "exlr8-manifest-up1.json").read_text())
    if manifest.get("name") != "up1":
        raise ValueError("This loader requires the up1 manifest")
    return manifest


def layer_arrays(path, number):
    """Host arrays of up1 layer `number`: ``(k, hidden, intermediate, packed, scales)``.

    ``packed[p]`` is uint8 [257 * expert_bytes] (routed experts, then the shared expert);
    ``scales[p]`` = (in_scale, out_scale) fp16 [257, features] built from SIDE_VECTORS.
    """
    from pathlib import Path

    import numpy as np

    from .weights import SafetensorsFile
    path = Path(path)
    k = MTP_WIDTH if number == MTP_LAYER else MAIN_WIDTH
    widths = _widths(_manifest(path)["layers"][str(number)])
    if widths != {k}:
        raise ValueError(f"Layer {number} is not uniform K{k}")
    stem = path / "experts" / f"exlr8-layer-{number:03d}"
    trellis = SafetensorsFile(f"{stem}.k{k}.safetensors")
    index = SafetensorsFile(f"{stem}.index.safetensors")
    hidden = index.shape("signs.in")[0]
    intermediate = index.shape(f"k{k}.gate.svh")[-1]
    signs = {name: index.array(name).astype(np.float16) for name in ("signs.in", "signs.out")}

    def both(name):  # routed rows then the shared expert's row
        return np.concatenate([index.array(f"k{k}.{name}"), index.array(f"shared.k{k}.{name}")])

    packed, scales = {}, {}
    for projection, (block, channel, sign, block_side) in SIDE_VECTORS.items():
        mags = both(f"{projection}.{block}")                       # [257, features / 128]
        expanded = (mags[:, :, None] * np.ones(128, np.float16)).reshape(len(mags), -1) * signs[sign]
        per_channel = both(f"{projection}.{channel}")
        scales[projection] = (expanded, per_channel) if block_side == "in" else (per_channel, expanded)
        packed[projection] = np.concatenate([trellis.array(f"trellis.{projection}"),
                                             trellis.array(f"shared.trellis.{projection}")])
    return k, hidden, intermediate, packed, scales


class ExpertStore:
    """Resident up1 expert store (exlr8/experts.py:12-76).  On an MI355X every layer's experts fit in
    HBM, so layers are always loaded resident; ``cache_gib`` is accepted for signature parity and
    ``resident=False`` loads resident as well (the reference's SSD cache is not built)."""

    def __init__(self, path, cache_gib=32, resident=False, optimize=True, device=None):
        from pathlib import Path
        self.path = Path(path)
        self.resident, self.optimize = True, optimize
        self.manifest = _manifest(self.path)
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


def _nbytes(t):
    return 0 if t is None else t.numel() * t.element_size()


def _from_store(cls, store, number):
    """ExpertLayer of layer `number` of an ExpertStore, resident on the store's device.  With
    ``optimize``, K4 and the GLM-5.3 shape (6144, 2048) the experts are served as joined MXFP4 and
    the trellis tensors and gate/up in-scales are released (exlr8/experts.py:132-148); K3 layers stay
    trellis.  The store counts the bytes of what stays resident."""
    k, hidden, intermediate, packed, scales = layer_arrays(store.path, number)
    dev = store.device
    layer = cls({p: torch.from_numpy(a).to(dev) for p, a in packed.items()},
                {p: tuple(torch.from_numpy(v).to(dev) for v in pair) for p, pair in scales.items()},
                hidden, intermediate, k=k, number=number)
    layer.store = store
    if store.optimize and k == 4 and (hidden, intermediate) == (6144, 2048):
        from .joined_mxfp4 import JoinedMXFP4
        layer.affine = JoinedMXFP4(layer)
        for projection in ("gate", "up"):
            layer.scales[projection] = (None, layer.scales[projection][1])
        del layer.packed
        resident = [t for pair in layer.affine.weights.values() for t in pair] + [layer.affine.unit]
    else:
        resident = list(layer.packed.values())
    resident += [t for pair in layer.scales.values() for t in pair]
    store.resident_bytes += sum(_nbytes(t) for t in resident)
    return layer


ExpertLayer.from_store = classmethod(_from_store)
