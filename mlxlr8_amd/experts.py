"""Resident K4 expert layer (mirrors the reference ``exlr8/experts.py`` ExpertLayer).

The reference loads packed experts from safetensors; this class takes device tensors that
are already resident in HBM (288 GB per MI355X holds every expert of many layers), so the
SSD cache paths of the reference do not exist here.
"""
from types import SimpleNamespace

import torch

from ._lib import check, lib, ptr, require_cuda, stream, workspace
from .fast_decode import _weights, fast_expert_mlp
from .fast_prefill import grouped_expert_mlp
from .trellis import BF16, _check_format


class ExpertLayer:
    """Packed gate/up/down trellis experts of one MoE layer (routed experts + shared expert last).

    Attributes mirror the reference (exlr8/experts.py:76-148): ``k``, ``hidden``,
    ``intermediate``, ``store.resident``, ``store.optimize``, ``packed`` (dict),
    ``scales`` (dict of (in, out) pairs), ``affine``, ``expert_bytes``.
    """

    def __init__(self, packed, scales, hidden, intermediate, k=4, number=0):
        if k != 4:
            raise ValueError(f"Layer {number} is not uniform K4")
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
        rows through the decode MLP, more through the grouped (sorted-by-expert) prefill MLP."""
        if self.affine is not None:
            return self.affine.slots(x, ids)
        mlp = fast_expert_mlp if ids.numel() // ids.shape[-1] <= 16 else grouped_expert_mlp
        return mlp(x, ids, self.packed, self.scales, self.k, self.hidden, self.intermediate)

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
        if rows > 8 or self.experts != 257 or x.dtype != BF16:
            raise ValueError("prepare_decode needs <= 8 bf16 rows and 256 routed + 1 shared experts")
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
        if rows > 8 or self.experts != 257 or x.dtype != BF16:
            raise ValueError("prepare_layer_decode needs <= 8 bf16 rows and 256 routed + 1 shared experts")
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
        if self.experts != 257:
            raise ValueError("decode_block needs 256 routed experts plus the shared expert")
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
