"""Resident joined-MXFP4 experts (mirrors the reference ``exlr8/joined_mxfp4.py``).

Gate and up of every expert are one ``[2m, h]`` MXFP4 matrix (e2m1 codes, one e8m0 scale per
32 along K, the per-128-block input scale magnitudes folded in); down is ``[h, m]``.  All
slots share ``xh = H128(x * unit)``.  ``slots`` returns per-slot expert values and ``finish``
the combined layer output; both run in ``libmoe_mi355x.so``.
"""
from types import SimpleNamespace

import torch

from ._lib import check, lib, ptr, require_cuda, stream, workspace

BF16 = torch.bfloat16


def encode(expert):
    """Load-time K4 -> joined MXFP4 (exlr8/joined_mxfp4.py:12-47), on the GPU.

    ``expert`` is a K4 ``ExpertLayer`` (packed gate/up/down, (in, out) scale pairs).  Returns
    ``(unit, weights)``: ``unit`` = sign of expert 0's gate input scales, fp16 [1, h];
    ``weights = {"gate_up": (codes [E, 2m, h/2], scales [E, 2m, h/32], None),
    "down": (codes [E, h, m/2], scales [E, h, m/32], None)}`` (uint8; low nibble = even k).  Gate
    and up are decoded, multiplied per input channel by ``in_scale * unit`` and quantised along
    their input dimension; down is quantised as decoded.  The MXFP4 rounding is the OCP MX
    conversion (shared exponent floor(log2 amax) - 2, E2M1 round-to-nearest-even, saturating):
    the reference's ``mx.quantize`` cannot be run here to confirm its choice.
    """
    h, m, experts = expert.hidden, expert.intermediate, expert.experts
    dev = expert.packed["gate"].device
    unit = torch.sign(expert.scales["gate"][0][:1]).to(torch.float16).contiguous()
    u8 = dict(dtype=torch.uint8, device=dev)
    gate_up = (torch.empty((experts, 2 * m, h // 2), **u8), torch.empty((experts, 2 * m, h // 32), **u8))
    down = (torch.empty((experts, h, m // 2), **u8), torch.empty((experts, h, m // 32), **u8))
    need = max(lib().moe_k4_to_mxfp4_workspace_bytes(h, m), lib().moe_k4_to_mxfp4_workspace_bytes(m, h))
    ws = torch.empty(need, **u8)
    st = stream(dev)
    for projection, (inc, out, side, dest, rows, offset) in (("gate", (h, m, 1, gate_up, 2 * m, 0)),
                                                            ("up", (h, m, 1, gate_up, 2 * m, m)),
                                                            ("down", (m, h, 2, down, h, 0))):
        packed = expert.packed[projection].contiguous()
        in_scale = expert.scales[projection][0].to(torch.float16).contiguous() if side == 1 else None
        check(lib().moe_k4_to_mxfp4(ptr(packed), packed.numel() * packed.element_size(), inc, out, side,
                                    ptr(in_scale) if in_scale is not None else None,
                                    ptr(unit) if in_scale is not None else None, ptr(dest[0]), ptr(dest[1]), rows,
                                    offset, ptr(ws), ws.numel(), st))
    return unit, {"gate_up": gate_up + (None,), "down": down + (None,)}


class JoinedMXFP4:
    """``weights = {"gate_up": (codes, scales), "down": (codes, scales)}``, ``unit`` fp16 [h],
    ``scales = {"gate": (None, out_gate), "up": (None, out_up), "down": (in_down, out_down)}``."""

    def __init__(self, weights, unit=None, scales=None, hidden=None, intermediate=None):
        if unit is None:
            # JoinedMXFP4(expert) as in the reference (exlr8/joined_mxfp4.py:137-142): encode the
            # K4 expert layer on the GPU
            expert = weights
            unit, weights = encode(expert)
            scales = {"gate": (None, expert.scales["gate"][1]), "up": (None, expert.scales["up"][1]),
                      "down": tuple(expert.scales["down"])}
            hidden, intermediate = expert.hidden, expert.intermediate
        weights = {p: tuple(v[:2]) for p, v in weights.items()}
        self.weights, self.unit, self.scales = weights, unit, scales
        self.hidden, self.intermediate = hidden, intermediate
        codes, sc = weights["gate_up"]
        if codes.dim() != 3 or tuple(codes.shape[1:]) != (2 * intermediate, hidden // 2) \
                or tuple(sc.shape) != (codes.shape[0], 2 * intermediate, hidden // 32):
            raise ValueError("gate_up must be [experts, 2m, h/2] codes with [experts, 2m, h/32] scales")
        dcodes, dsc = weights["down"]
        if tuple(dcodes.shape) != (codes.shape[0], hidden, intermediate // 2) \
                or tuple(dsc.shape) != (codes.shape[0], hidden, intermediate // 32):
            raise ValueError("down must be [experts, h, m/2] codes with [experts, h, m/32] scales")
        self.experts = codes.shape[0]
        require_cuda(codes, sc, dcodes, dsc, unit)
        # the grouped GEMMs (prefill-sized batches) widen the weights to fp16 with their block
        # scale, which is exact only for e8m0 scales in GROUPED_SCALES (scaled e2m1 values stay
        # normal fp16 numbers); a layer with any scale outside takes the decode GEMVs (exact for
        # every scale) in chunks of decode size instead
        lo, hi = self.GROUPED_SCALES
        self.grouped_exact = all(int(t.min()) >= lo and int(t.max()) <= hi for t in (sc, dsc))

    def _args(self):
        (gc, gs), (dc, ds) = self.weights["gate_up"], self.weights["down"]
        return [ptr(gc), ptr(gs), ptr(dc), ptr(ds), self.experts, ptr(self.unit), ptr(self.scales["gate"][1]),
                ptr(self.scales["up"][1]), ptr(self.scales["down"][0]), ptr(self.scales["down"][1])]

    # decode batches (<= 8 token rows) run the MXFP4 GEMVs; larger batches the sorted grouped
    # GEMM on the MX matrix cores (the reference switches to its sorted gather_qmm for prefill
    # sizes, exlr8/joined_mxfp4.py:98-113)
    DECODE_ROWS = 8
    GROUPED_SCALES = (114, 140)

    def slots(self, x, ids):
        """values [*ids.shape, h] (exlr8/joined_mxfp4.py:143-147)."""
        h = self.hidden
        if x.shape[-1] != h or tuple(x.shape[:-1]) != tuple(ids.shape[:-1]):
            raise ValueError("activation rows do not match the expert indices")
        if x.dtype != BF16:
            raise ValueError("this build computes bf16 activations")
        require_cuda(x, ids)
        slots = ids.shape[-1]
        idx = ids.reshape(-1, slots).to(torch.int32).contiguous()
        rows = idx.shape[0]
        xr = x.reshape(rows, h).contiguous()
        values = torch.empty((rows * slots, h), dtype=BF16, device=x.device)
        st = stream(x.device)
        if rows > self.DECODE_ROWS and self.grouped_exact:
            nbytes = lib().moe_mxfp4_grouped_mlp_workspace_bytes(rows, slots, h, self.intermediate, self.experts)
            ws = torch.empty(nbytes, dtype=torch.uint8, device=x.device)
            check(lib().moe_mxfp4_grouped_mlp(ptr(xr), ptr(idx), rows, slots, *self._args(), h, self.intermediate,
                                              ptr(values), ptr(ws), nbytes, st))
            return values.reshape(*ids.shape, h)
        ws = workspace(x.device, h, self.intermediate, "mxfp4")
        step = max(1, 72 // slots)
        for r0 in range(0, rows, step):
            r1 = min(rows, r0 + step)
            check(lib().moe_mxfp4_mlp(ptr(xr[r0:r1]), ptr(idx[r0:r1]), r1 - r0, slots, *self._args(), h,
                                      self.intermediate, ptr(values[r0 * slots:r1 * slots]), ptr(ws), ws.numel(), st))
        return values.reshape(*ids.shape, h)

    def finish(self, x, ids, scores, residual):
        """residual + T(sum_i values_i * scores_i) + shared (exlr8/joined_mxfp4.py:148-163)."""
        h = self.hidden
        rows = x.numel() // h
        if x.dtype != BF16:
            raise ValueError("this build computes bf16 activations")
        require_cuda(x, ids, scores, residual)
        if rows > self.DECODE_ROWS:
            from .fast_decode import combine_values
            return combine_values(self.slots(x.reshape(rows, h), ids.reshape(rows, 9)), scores, residual)
        xr = x.reshape(rows, h).contiguous()
        idx = ids.reshape(rows, 9).to(torch.int32).contiguous()
        sc = scores.reshape(rows, 8).to(torch.float32).contiguous()
        res = residual.reshape(rows, h).to(BF16).contiguous()
        out = torch.empty((rows, h), dtype=BF16, device=x.device)
        ws = workspace(x.device, h, self.intermediate, "mxfp4")
        check(lib().moe_mxfp4_mlp_finish(ptr(xr), ptr(idx), ptr(sc), ptr(res), rows, *self._args(), h,
                                         self.intermediate, ptr(out), ptr(ws), ws.numel(), stream(x.device)))
        return out.reshape(residual.shape)

    def prepare_decode(self, x, residual, router_weight, bias):
        """Bind device buffers once and return a callable that enqueues router GEMV + route +
        MXFP4 MLP + combine for <= 8 decode rows in one C call (exlr8/fast_router.py:27-37 with the
        joined experts); results land in `.out`, `.ids`, `.scores`.  The call runs on the stream that
        is current now (its workspace belongs to that stream)."""
        h = self.hidden
        rows = x.numel() // h
        if rows < 1 or rows > 8 or self.experts != 257 or x.dtype != BF16:
            raise ValueError("prepare_decode needs 1..8 bf16 rows and 256 routed + 1 shared experts")
        require_cuda(x, residual, router_weight, bias)
        call = SimpleNamespace()
        call.x = x.reshape(rows, h).contiguous()
        call.residual = residual.reshape(rows, h).to(BF16).contiguous()
        call.w = router_weight.to(torch.float32).contiguous()
        call.bias = bias.to(torch.float32).contiguous()
        call.out = torch.empty((rows, h), dtype=BF16, device=x.device)
        call.ids = torch.empty((rows, 9), dtype=torch.int32, device=x.device)
        call.scores = torch.empty((rows, 8), dtype=torch.float32, device=x.device)
        ws = workspace(x.device, h, self.intermediate, "mxfp4")
        args = (ptr(call.x), ptr(call.residual), rows, ptr(call.w), ptr(call.bias), *self._args(), h,
                self.intermediate, ptr(call.out), ptr(call.ids), ptr(call.scores), ptr(ws), ws.numel(),
                stream(x.device))
        fn = lib().moe_mxfp4_moe_decode

        def run():
            check(fn(*args))
            return call.out

        call.run = run
        return call

    def decode_block(self, x, residual, router_weight, bias):
        """One-shot form of prepare_decode: returns (out, indices [rows, 9], scores [rows, 8])."""
        call = self.prepare_decode(x, residual, router_weight, bias)
        call.run()
        return call.out.reshape(residual.shape), call.ids, call.scores

    def prefill(self, x, residual, router_weight, bias):
        """A prefill chunk through the routed block: routing, sorted grouped GEMMs on the MX
        matrix cores, combine (exlr8/joined_mxfp4.py:90-134,148-163 with exlr8/model.py:111-132).
        Returns (out [rows, h] bf16, indices [rows, 9] int32, scores [rows, 8] f32)."""
        h = self.hidden
        if x.dtype != BF16:
            raise ValueError("this build computes bf16 activations")
        if self.experts != 257:
            raise ValueError("the routed block needs 256 routed experts plus the shared expert")
        require_cuda(x, residual, router_weight, bias)
        rows = x.numel() // h
        xr = x.reshape(rows, h).contiguous()
        res = residual.reshape(rows, h).to(BF16).contiguous()
        w = router_weight.to(torch.float32).contiguous()
        b = bias.to(torch.float32).contiguous()
        if not self.grouped_exact:
            # block scales outside the grouped GEMMs' exact window: decode-sized routed blocks
            parts = [self.decode_block(xr[r0:r0 + 8], res[r0:r0 + 8], w, b) for r0 in range(0, rows, 8)]
            return (torch.cat([p[0] for p in parts]).reshape(residual.shape), torch.cat([p[1] for p in parts]),
                    torch.cat([p[2] for p in parts]))
        out = torch.empty((rows, h), dtype=BF16, device=x.device)
        ids = torch.empty((rows, 9), dtype=torch.int32, device=x.device)
        scores = torch.empty((rows, 8), dtype=torch.float32, device=x.device)
        nbytes = lib().moe_mxfp4_prefill_workspace_bytes(rows, h, self.intermediate, self.experts)
        ws = torch.empty(nbytes, dtype=torch.uint8, device=x.device)
        check(lib().moe_mxfp4_prefill(ptr(xr), ptr(res), rows, ptr(w), ptr(b), *self._args(), h, self.intermediate,
                                      ptr(out), ptr(ids), ptr(scores), ptr(ws), nbytes, stream(x.device)))
        return out.reshape(residual.shape), ids, scores
