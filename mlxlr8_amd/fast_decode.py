"""Selected-expert trellis MLP on MI355X (mirrors the reference ``exlr8/fast_decode.py``).

``fast_expert_mlp`` returns per-slot expert values; ``compiled_expert_mlp_finish`` returns
the combined ``residual + (routed + shared)`` output.  K4 experts run gate/up, typed SwiGLU and
down as decode-fused GEMVs in ``libmoe_mi355x.so``; K2/K3 experts (the K3 multi-token-prediction
layer) run through the library's generic-window grouped trellis MLP and its combine kernel.
"""
import torch

from ._lib import check, lib, ptr, require_cuda, stream, workspace
from .fast_prefill import grouped_expert_mlp
from .trellis import BF16, _check_format, _nbytes, _rows_for, expert_linear

MAX_ROWS = 8  # token rows per kernel call; larger batches are split on the host


def fast_expert_linear(x, indices, packed, in_scale, out_scale, k, in_features, out_features, sharded_side=1):
    """exlr8/fast_decode.py:153-165 -- same result as ``expert_linear``."""
    return expert_linear(x, indices, packed, in_scale, out_scale, k, in_features, out_features, sharded_side)


def _validate(x, indices, packed, scales, k, hidden, intermediate):
    if _rows_for(x, indices, hidden):
        raise ValueError("the expert MLP takes one activation row per token")
    for projection in ("gate", "up", "down"):
        a, b, side = (intermediate, hidden, 2) if projection == "down" else (hidden, intermediate, 1)
        experts = _check_format(packed[projection], k, a, b, side)
        if (tuple(scales[projection][0].shape) != (experts, a)
                or tuple(scales[projection][1].shape) != (experts, b)):
            raise ValueError("expert side vectors must contain full signed channel scales")
    if x.dtype != BF16:
        raise ValueError("this build computes bf16 activations")
    require_cuda(x, indices, *packed.values(), *(s for pair in scales.values() for s in pair))


def _weights(packed, scales):
    g, u, d = packed["gate"], packed["up"], packed["down"]
    return [ptr(g), ptr(u), ptr(d), _nbytes(g), ptr(scales["gate"][0]), ptr(scales["gate"][1]),
            ptr(scales["up"][0]), ptr(scales["up"][1]), ptr(scales["down"][0]), ptr(scales["down"][1])]


def fast_expert_mlp(x, indices, packed, scales, k, hidden, intermediate, *, reuse=False, fp8=None,
                    expert_to_slot=None):
    """Apply selected expert MLPs; return [*indices.shape, hidden] (exlr8/fast_decode.py:208-221).

    Repeated experts across rows are always read once (``reuse`` is accepted for signature
    compatibility); the FP8 expert cache of the reference is not part of this build.
    """
    if fp8 is not None or expert_to_slot is not None:
        raise NotImplementedError("FP8 expert caches are not part of the MI355X build")
    _validate(x, indices, packed, scales, k, hidden, intermediate)
    if k not in (3, 4):
        return grouped_expert_mlp(x, indices, packed, scales, k, hidden, intermediate)
    slots = indices.shape[-1]
    ids = indices.reshape(-1, slots).to(torch.int32).contiguous()
    rows = ids.shape[0]
    xr = x.reshape(rows, hidden).contiguous()
    values = torch.empty((rows * slots, hidden), dtype=BF16, device=x.device)
    ws = workspace(x.device, hidden, intermediate)
    w = _weights(packed, scales)
    st = stream(x.device)
    step = min(MAX_ROWS, max(1, 72 // slots))
    for r0 in range(0, rows, step):
        r1 = min(rows, r0 + step)
        args = (ptr(xr[r0:r1]), ptr(ids[r0:r1]), r1 - r0, slots, *w, hidden, intermediate,
                ptr(values[r0 * slots:r1 * slots]), ptr(ws), ws.numel(), st)
        check(lib().moe_k4_mlp(*args) if k == 4 else lib().moe_trellis_mlp(k, *args))
    return values.reshape(*indices.shape, hidden)


def combine_values(values, scores, residual):
    """exlr8/model.py:415-418: residual + T(T(sum_i values_i * scores_i) + values_8), bf16."""
    hidden = values.shape[-1]
    rows = values.numel() // (9 * hidden)
    if values.dtype != BF16 or values.numel() != rows * 9 * hidden or rows < 1:
        raise ValueError("values must be bf16 [..., 9, hidden]")
    if scores.numel() != rows * 8 or residual.numel() != rows * hidden:
        raise ValueError("scores and residual do not match the values")
    require_cuda(values, scores, residual)
    v = values.reshape(rows * 9, hidden).contiguous()
    sc = scores.reshape(rows, 8).to(torch.float32).contiguous()
    res = residual.reshape(rows, hidden).to(BF16).contiguous()
    out = torch.empty((rows, hidden), dtype=BF16, device=values.device)
    check(lib().moe_combine_values(ptr(v), ptr(sc), ptr(res), rows, hidden, ptr(out), stream(values.device)))
    return out.reshape(residual.shape)


def expert_values(x, indices, packed, scales, k, hidden, intermediate):
    """Per-slot values by the reference's row-count rule (exlr8/experts.py:170-175): up to 16 token
    rows through the decode MLP (K3 and K4 experts), more through the sorted grouped MLP (K2 experts
    always grouped)."""
    rows = indices.numel() // indices.shape[-1]
    if k in (3, 4) and rows <= 16:
        return fast_expert_mlp(x, indices, packed, scales, k, hidden, intermediate)
    return grouped_expert_mlp(x, indices, packed, scales, k, hidden, intermediate)


def mlp_finish(x, indices, scores, residual, packed, scales, hidden, intermediate, k=4):
    """Expert MLP plus the weighted combine with the shared expert (slot 8) and the residual:
    one fused call for K4 decode batches (<= 8 rows), else per-slot values and the combine."""
    _validate(x.reshape(-1, hidden), indices.reshape(-1, 9), packed, scales, k, hidden, intermediate)
    rows = x.numel() // hidden
    require_cuda(scores, residual)
    if k not in (3, 4) or rows > MAX_ROWS:
        values = expert_values(x.reshape(rows, hidden), indices.reshape(rows, 9), packed, scales, k, hidden,
                               intermediate)
        return combine_values(values, scores, residual)
    xr = x.reshape(rows, hidden).contiguous()
    ids = indices.reshape(rows, 9).to(torch.int32).contiguous()
    sc = scores.reshape(rows, 8).to(torch.float32).contiguous()
    res = residual.reshape(rows, hidden).to(BF16).contiguous()
    out = torch.empty((rows, hidden), dtype=BF16, device=x.device)
    ws = workspace(x.device, hidden, intermediate)
    args = (ptr(xr), ptr(ids), ptr(sc), ptr(res), rows, *_weights(packed, scales), hidden, intermediate, ptr(out),
            ptr(ws), ws.numel(), stream(x.device))
    check(lib().moe_k4_mlp_finish(*args) if k == 4 else lib().moe_trellis_mlp_finish(k, *args))
    return out.reshape(residual.shape)


def compiled_expert_mlp_finish(expert):
    """exlr8/fast_decode.py:224-244: f(x, indices, scores, residual) -> residual + routed + shared."""
    if getattr(expert, "affine", None) is not None:
        return expert.affine.finish
    h, m = expert.hidden, expert.intermediate

    def apply(x, indices, scores, residual):
        return mlp_finish(x, indices, scores, residual, expert.packed, expert.scales, h, m, expert.k)

    return apply
