"""The MoE branch of a GLM-5.3 decoder layer (mirrors ``exlr8/model.py:111-132,385-418``).

Only the expert path is built; attention, dense layers and the vocabulary head are outside
this package.
"""
from dataclasses import dataclass

import torch

from .fast_decode import combine_values
from .fast_router import compiled_finish, route, router_logits


@dataclass
class MoEArgs:
    """The ModelArgs fields the MoE branch reads (exlr8/model.py:23-98)."""
    hidden_size: int = 6144
    moe_intermediate_size: int = 2048
    n_routed_experts: int = 256
    n_shared_experts: int = 1
    num_experts_per_tok: int = 8
    n_group: int = 1
    topk_group: int = 1
    norm_topk_prob: bool = True
    routed_scaling_factor: float = 2.5
    scoring_func: str = "sigmoid"
    topk_method: str = "noaux_tc"

    def __post_init__(self):
        if (self.scoring_func, self.topk_method) != ("sigmoid", "noaux_tc"):
            raise ValueError("Unsupported GLM activation or router")
        if self.n_shared_experts != 1:
            raise ValueError("EXLR8 GLM requires one shared expert")


def _fast_router_args(args):
    return (args.n_routed_experts == 256 and args.num_experts_per_tok == 8 and args.n_group == args.topk_group == 1
            and args.norm_topk_prob and args.routed_scaling_factor == 2.5)


def route_experts(logits, bias, args):
    """Select with corrected scores; weight with the original sigmoid scores (exlr8/model.py:111-132).

    Returns (indices [...,8] int32, weights [...,8] f32), selected in descending order.
    """
    if not _fast_router_args(args):
        raise NotImplementedError("only the GLM-5.3 router configuration (256 experts, top-8, one group) is built")
    ids, scores = route(logits, bias)
    return ids[..., :8], scores


class MoEBlock:
    """`DecoderLayer.__call__`'s sparse branch: returns h + routed + shared (exlr8/model.py:385-418).

    With the GLM router configuration every row count goes through ``compiled_finish`` (one
    library call for decode batches and for joined-MXFP4 prefill chunks; K4 prefill rows are
    routed, run through the grouped trellis MLP and combined).  Other configurations take the
    reference's general branch: route_experts, experts(x, indices), then the model combine.
    """

    def __init__(self, args, router_weight, bias, experts):
        self.args, self.gate, self.bias, self.experts = args, router_weight, bias, experts
        self._routed_finish = None

    def __call__(self, x, h):
        a = self.args
        if _fast_router_args(a) and x.dtype == torch.bfloat16 and self.bias.shape == (256,):
            if self._routed_finish is None:
                self._routed_finish = compiled_finish(self.experts, self.gate, self.bias)
            return self._routed_finish(x, h)
        logits = router_logits(x, self.gate) if isinstance(self.gate, torch.Tensor) else self.gate(x.float())
        ids, scores = route_experts(logits, self.bias, a)
        shared = torch.full(ids.shape[:-1] + (1,), a.n_routed_experts, dtype=ids.dtype, device=ids.device)
        indices = torch.cat([ids, shared], dim=-1)
        values = self.experts(x, indices)
        return combine_values(values, scores, h)


class DecoderMoELayer:
    """A decoder layer's post-attention half: h = x + attn_out; out = h + MoE(rms_norm(h))
    (exlr8/model.py:376-418 with the fused residual/RMS pair of exlr8/fast_norm.py), for decode
    rows on the K4 experts.  One library call per layer."""

    def __init__(self, args, post_norm, router_weight, bias, experts, eps=1e-5):
        if not (_fast_router_args(args) and getattr(experts, "k", None) == 4):
            raise NotImplementedError("the fused decode layer is built for the GLM-5.3 K4 configuration")
        self.args, self.norm, self.gate, self.bias, self.experts, self.eps = (args, post_norm, router_weight, bias,
                                                                               experts, eps)

    def __call__(self, x, attn=None):
        out, ids, scores = self.experts.layer_decode(x, self.norm, self.gate, self.bias, attn, self.eps)
        return out, ids[..., :8]


class DecoderMoEStack:
    """Consecutive decoder MoE layers with no attention output between them (each layer:
    h <- h + MoE(rms_norm(h))): the 20-layer K4 decode stack."""

    def __init__(self, layers):
        self.layers = list(layers)

    def __call__(self, x):
        for layer in self.layers:
            x, _ = layer(x)
        return x
