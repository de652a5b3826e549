"""Seeded synthetic MoE layers (random-init weights of the GLM-5.3 expert shapes).

There is no checkpoint access; expert weights are drawn on the device from a seeded
``torch.Generator`` so a seed reproduces the same layer on any MI355X.

K4 trellis layer (the reference's resident K4 expert layout, exlr8/experts.py:99-124):
  packed gate/up [E * h*m/2] u8 (side 1), down [E * m*h/2] u8 (side 2): uniform random
  bitstreams (every bitstream is a valid trellis); in-scales +-1 per channel, out-scales
  +-1 * lognormal(ln(1/sqrt(h)), 0.3) as fp16.
Joined MXFP4 layer (exlr8/joined_mxfp4.py:12-47 layout): random e2m1 codes with e8m0 scales
  chosen so dequantised values have std ~ 1/sqrt(h).
Router: fp32 weight ~ N(0, 0.02), bias ~ N(0, 0.01), optional Zipf(1.1) ranked offset.
Router weights and activations are drawn on the host generator, so a seed gives the same routing
inputs on any device (and on the CPU).
"""
import math

import torch

HIDDEN, INTER, EXPERTS = 6144, 2048, 257


def _gen(device, seed):
    g = torch.Generator(device=device)
    g.manual_seed(int(seed))
    return g


def _signs(shape, g, device):
    return (torch.randint(0, 2, shape, generator=g, device=device, dtype=torch.int32) * 2 - 1).to(torch.float16)


def _lognormal_signed(shape, mu, sigma, g, device):
    mag = torch.exp(torch.randn(shape, generator=g, device=device) * sigma + mu)
    return (mag * _signs(shape, g, device).float()).to(torch.float16)


def zipf_offset(n, seed, s=1.1, scale=0.08, device="cpu"):
    """Ranked Zipf(s) popularity offset added to the router bias (random rank order)."""
    g = torch.Generator(device="cpu")
    g.manual_seed(int(seed) + 7919)
    rank = torch.randperm(n, generator=g).double() + 1.0
    return (scale * rank.pow(-s)).float().to(device)


def _host_gen(seed):
    g = torch.Generator(device="cpu")
    g.manual_seed(int(seed))
    return g


def router(device, seed, hidden=HIDDEN, experts=256, zipf=False):
    """fp32 router weight [experts, hidden] ~ N(0, 0.02) and bias [experts] ~ N(0, 0.01), drawn on the
    host generator (the same values on every device) and moved to ``device``."""
    g = _host_gen(seed)
    w = torch.randn((experts, hidden), generator=g) * 0.02
    bias = torch.randn((experts,), generator=g) * 0.01
    if zipf:
        bias = bias + zipf_offset(experts, seed)
    return w.to(device).contiguous(), bias.to(device).contiguous()


def k4_layer(device, seed, hidden=HIDDEN, intermediate=INTER, experts=EXPERTS, k=4):
    """dict(packed={gate,up,down}, scales={gate:(in,out), up:(in,out), down:(in,out)}) of k-bit
    trellis experts (every bitstream is a valid trellis)."""
    g = _gen(device, seed)
    nbytes = experts * hidden * intermediate * k // 8
    packed = {p: torch.randint(0, 256, (nbytes,), generator=g, device=device, dtype=torch.uint8)
              for p in ("gate", "up", "down")}
    mu = math.log(1.0 / math.sqrt(hidden))
    scales = {}
    for p in ("gate", "up", "down"):
        a, b = (intermediate, hidden) if p == "down" else (hidden, intermediate)
        scales[p] = (_signs((experts, a), g, device), _lognormal_signed((experts, b), mu, 0.3, g, device))
    return {"packed": packed, "scales": scales}


def mxfp4_layer(device, seed, hidden=HIDDEN, intermediate=INTER, experts=EXPERTS):
    """Joined MXFP4 experts: gate_up [E, 2m, h/2] codes + [E, 2m, h/32] e8m0, down [E, h, m/2] + [E, h, m/32]."""
    g = _gen(device, seed)
    # e2m1 codes uniform over 16 values: E[v^2] = 8.5625; target std 1/sqrt(h)
    target = 1.0 / math.sqrt(hidden)
    base = 127 + math.floor(math.log2(target / math.sqrt(8.5625)))
    w = {}
    for name, (n, k) in (("gate_up", (2 * intermediate, hidden)), ("down", (hidden, intermediate))):
        codes = torch.randint(0, 256, (experts, n, k // 2), generator=g, device=device, dtype=torch.uint8)
        scales = (base + torch.randint(0, 2, (experts, n, k // 32), generator=g, device=device,
                                       dtype=torch.int32)).to(torch.uint8)
        w[name] = (codes, scales)
    unit = _signs((hidden,), g, device)
    side = {
        "out_gate": _lognormal_signed((experts, intermediate), 0.0, 0.3, g, device),
        "out_up": _lognormal_signed((experts, intermediate), 0.0, 0.3, g, device),
        "in_down": _signs((experts, intermediate), g, device),
        "out_down": _lognormal_signed((experts, hidden), 0.0, 0.3, g, device),
    }
    return {"weights": w, "unit": unit, "side": side}


def activations(device, seed, rows, hidden=HIDDEN, correlated=False):
    """x, residual bf16 [rows, hidden] ~ N(0, 1), drawn on the host generator and moved to ``device``.

    correlated=True is the speculative-verify batch: consecutive token pairs share a base vector
    ~ N(0, 1) and each token adds its own N(0, 0.5^2) noise.  Through the GLM router this gives
    ~47 distinct experts per 8 tokens (8 routed + 1 shared each), i.e. ~30% of the routed experts
    repeat across tokens; one base vector for all 8 tokens gives only ~25 distinct experts.
    """
    g = _host_gen(seed + 1)
    if correlated:
        base = torch.randn(((rows + 1) // 2, hidden), generator=g)
        x = base[torch.arange(rows) // 2] + 0.5 * torch.randn((rows, hidden), generator=g)
    else:
        x = torch.randn((rows, hidden), generator=g)
    residual = torch.randn((rows, hidden), generator=g)
    return x.to(torch.bfloat16).to(device), residual.to(torch.bfloat16).to(device)


def norm_weight(device, seed, hidden=HIDDEN):
    """RMSNorm weight bf16 [hidden] ~ U(0.5, 1.5)."""
    g = _gen(device, seed)
    return (0.5 + torch.rand(hidden, generator=g, device=device)).to(torch.bfloat16)


def stack_layer(device, seed, index, hidden=HIDDEN, intermediate=INTER):
    """Layer `index` of the 20-layer K4 decode stack: independently seeded experts, a Zipf-skewed
    router bias and an RMSNorm weight.  Returns (k4_layer dict, router weight, bias, norm weight)."""
    lay = k4_layer(device, seed + 101 * index, hidden, intermediate)
    w, bias = router(device, seed + 101 * index, hidden, zipf=True)
    return lay, w, bias, norm_weight(device, seed + 7 * index, hidden)
