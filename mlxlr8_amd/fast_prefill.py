"""Prefill over many rows (mirrors ``exlr8/fast_prefill.py``).

``plan(indices, experts, block_rows)`` returns ``(sorted_ids, order, table, count)`` as the
reference's ``_plan``: ``order`` sorts the flat ids (stable within an expert), ``table`` is the
``[3, blocks]`` (expert, first, length) block table and ``count`` the number of used blocks.
The table is computed on the GPU by ``moe_segment_table``.  ``grouped_expert_mlp`` runs the K2/K3/K4
expert MLP of every slot with one weight stream per sorted expert block
(``moe_trellis_grouped_mlp``).
"""
import torch

from ._lib import check, lib, ptr, require_cuda, stream

BF16 = torch.bfloat16
_grouped_ws = {}


def segment_table(ids, experts, block_rows):
    """(order [n], counts [experts], starts [experts], table [3, blocks]) for flat ids."""
    require_cuda(ids)
    flat = ids.reshape(-1).to(torch.int32).contiguous()
    n = flat.numel()
    cap = n // block_rows + experts + 1
    dev = flat.device
    order = torch.empty(n, dtype=torch.int32, device=dev)
    counts = torch.empty(experts, dtype=torch.int32, device=dev)
    starts = torch.empty(experts, dtype=torch.int32, device=dev)
    table = torch.empty((3, cap), dtype=torch.int32, device=dev)
    nblk = torch.empty(1, dtype=torch.int32, device=dev)
    check(lib().moe_segment_table(ptr(flat), n, experts, block_rows, ptr(order), ptr(counts), ptr(starts),
                                  ptr(table), cap, ptr(nblk), stream(dev)))
    used = int(nblk.item())
    return order, counts, starts, table[:, :used]


def plan(indices, experts, block_rows):
    """The reference's ``_plan``: (sorted_ids, order, table, count)."""
    order, _, _, table = segment_table(indices, experts, block_rows)
    flat = indices.reshape(-1).to(torch.int32)
    return flat[order.long()], order, table, table.shape[1]


def block_rows(rows, experts):
    """exlr8/fast_prefill.py:104-109: 8-row blocks for small segments, 32 otherwise."""
    return 8 if rows < experts * 8 else 32


def grouped_expert_mlp(x, indices, packed, scales, k, hidden, intermediate, *, half_dot=False):
    """values[*indices.shape, hidden] of the K-bit expert MLPs (exlr8/fast_prefill.py:188-211).

    ``packed``/``scales`` are the ``ExpertLayer`` dictionaries; ``k`` is 2, 3 or 4.  ``x`` holds
    one row per row of ``indices`` (the row's slots share it).  The matrix operands are fp16
    hi/lo splits of the fp32 activations with fp32 accumulation (``half_dot`` is accepted for
    signature parity; the result is the float32-dot one either way).
    """
    del half_dot
    if k not in (2, 3, 4):
        raise ValueError("EXLR8 trellis width must be 2, 3, or 4")
    if x.dtype != BF16:
        raise ValueError("this build computes bf16 activations")
    require_cuda(x, indices, *packed.values())
    slots = indices.shape[-1]
    ids = indices.reshape(-1, slots).to(torch.int32).contiguous()
    rows = ids.shape[0]
    xr = x.reshape(-1, hidden)
    if xr.shape[0] != rows:
        raise ValueError("activation rows do not match the expert indices")
    xr = xr.contiguous()
    pg, pu, pd = (packed[p].contiguous() for p in ("gate", "up", "down"))
    nbytes = pg.numel() * pg.element_size()
    experts = nbytes // (hidden * intermediate * k // 8)
    sc = {p: tuple(v.to(torch.float16).contiguous() for v in scales[p]) for p in ("gate", "up", "down")}
    values = torch.empty((rows * slots, hidden), dtype=BF16, device=x.device)
    need = lib().moe_k4_grouped_mlp_workspace_bytes(rows, slots, hidden, intermediate, experts)
    key = (str(x.device),)
    ws = _grouped_ws.get(key)
    if ws is None or ws.numel() < need:
        ws = torch.empty(need, dtype=torch.uint8, device=x.device)
        _grouped_ws[key] = ws
    check(lib().moe_trellis_grouped_mlp(k, ptr(xr), ptr(ids), rows, slots, ptr(pg), ptr(pu), ptr(pd), nbytes,
                                        ptr(sc["gate"][0]), ptr(sc["gate"][1]), ptr(sc["up"][0]),
                                        ptr(sc["up"][1]), ptr(sc["down"][0]), ptr(sc["down"][1]), hidden,
                                        intermediate, ptr(values), ptr(ws), ws.numel(), stream(x.device)))
    return values.reshape(*indices.shape, hidden)
