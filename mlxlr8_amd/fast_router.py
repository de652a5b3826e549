"""Fused router for small GLM target batches (mirrors the reference ``exlr8/fast_router.py``)."""
import torch

from ._lib import check, lib, ptr, require_cuda, stream


def router_logits(x, weight):
    """logits = f32(x) @ weight^T with an fp32 [experts, hidden] weight (exlr8/dense.py:158-159)."""
    require_cuda(x, weight)
    hidden = x.shape[-1]
    rows = x.numel() // hidden
    xb = x.reshape(rows, hidden).to(torch.bfloat16).contiguous()
    w = weight.to(torch.float32).contiguous()
    out = torch.empty((rows, w.shape[0]), dtype=torch.float32, device=x.device)
    check(lib().moe_router_logits(ptr(xb), ptr(w), rows, hidden, w.shape[0], ptr(out), stream(x.device)))
    return out.reshape(*x.shape[:-1], w.shape[0])


def route(logits, bias):
    """(indices [...,9] with slot 8 = 256, scores [...,8]) (exlr8/fast_router.py:17-24)."""
    require_cuda(logits, bias)
    if logits.shape[-1] != 256 or bias.numel() != 256:
        raise ValueError("the fused router takes 256 expert logits and a 256-entry bias")
    rows = logits.numel() // 256
    lg = logits.reshape(rows, 256).to(torch.float32).contiguous()
    b = bias.to(torch.float32).contiguous()
    ids = torch.empty((rows, 9), dtype=torch.int32, device=logits.device)
    scores = torch.empty((rows, 8), dtype=torch.float32, device=logits.device)
    check(lib().moe_route_f32(ptr(lg), ptr(b), rows, ptr(ids), ptr(scores), stream(logits.device)))
    return ids.reshape(*logits.shape[:-1], 9), scores.reshape(*logits.shape[:-1], 8)


def compiled_finish(experts, gate, bias):
    """exlr8/fast_router.py:27-37: call(x, residual) = experts' finish(x, route(gate(x)), residual).

    ``gate`` is the fp32 router weight [256, hidden] (or a callable returning logits).  With the
    weight given, one library call covers router, routing, experts and combine: joined-MXFP4
    experts take the decode block for <= 8 rows and the grouped prefill block beyond; K4 experts
    the decode block for <= 8 rows.  Otherwise routing is followed by the experts' finish.
    """
    from .fast_decode import compiled_expert_mlp_finish

    finish = compiled_expert_mlp_finish(experts)
    weight = gate if isinstance(gate, torch.Tensor) else None

    def call(x, residual):
        h = x.shape[-1]
        rows = x.numel() // h
        affine = getattr(experts, "affine", None)
        if weight is not None and affine is not None and getattr(affine, "experts", 0) == 257:
            if rows <= affine.DECODE_ROWS:
                return affine.decode_block(x, residual, weight, bias)[0]
            return affine.prefill(x, residual, weight, bias)[0]
        if weight is not None and affine is None and getattr(experts, "k", None) == 4 and rows <= 8:
            return experts.decode_block(x, residual, weight, bias)
        logits = router_logits(x, weight) if weight is not None else gate(x.float())
        indices, scores = route(logits, bias)
        return finish(x, indices, scores, residual)

    return call
