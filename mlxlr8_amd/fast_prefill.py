"""Sorted work order for prefill (mirrors ``exlr8/fast_prefill.py:19-46``).

``plan(indices, experts, block_rows)`` returns ``(sorted_ids, order, table, count)`` as the
reference's ``_plan``: ``order`` sorts the flat ids (stable within an expert), ``table`` is the
``[3, blocks]`` (expert, first, length) block table and ``count`` the number of used blocks.
The table is computed on the GPU by ``moe_segment_table``.
"""
import torch

from ._lib import check, lib, ptr, require_cuda, stream


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
