"""EXL3/QTIP-style trellis operators on MI355X (K4 GEMVs; K2/K3 grouped linears; K2/K3/K4 decode).

Mirrors the operator surface of the reference module ``exlr8/trellis.py`` (format check,
decode, ``trellis_linear``, ``expert_linear``, ``dequantize_trellis``) on PyTorch-ROCm
device tensors.  Decoding and the GEMVs run in ``libmoe_mi355x.so``.

Storage (reference ``exlr8/trellis.py:1-11,78-102``, ``exlr8/metal/trellis.metal:44-48``):
a K4 tile holds 256 weights in 128 bytes; side 1 stores output blocks first, side 2 input
blocks first; experts are concatenated with the shared expert last.
"""
import math

import torch

from ._lib import check, lib, ptr, require_cuda, stream, workspace

BF16 = torch.bfloat16


def _nbytes(packed):
    return packed.numel() * packed.element_size()


def _check_format(packed, k, in_features, out_features, sharded_side):
    """Validate a packed trellis tensor; return its expert count (exlr8/trellis.py:53-64)."""
    if k not in (2, 3, 4):
        raise ValueError("EXLR8 trellis width must be 2, 3, or 4")
    if in_features <= 0 or out_features <= 0 or in_features % 128 or out_features % 128:
        raise ValueError("trellis dimensions must be positive multiples of 128")
    if sharded_side not in (0, 1, 2):
        raise ValueError("sharded_side must be 0, 1, or 2")
    size = in_features * out_features * k // 8
    nbytes = _nbytes(packed)
    if nbytes == 0 or nbytes % size:
        raise ValueError("packed byte count does not match the trellis dimensions")
    return nbytes // size




def decode_inner(packed, k, in_features, out_features, sharded_side=1, expert=0):
    """Decoded inner weights [in, out] (fp16, bit-exact codebook values) of one expert (K2, K3, K4)."""
    experts = _check_format(packed, k, in_features, out_features, sharded_side)
    if not 0 <= expert < experts:
        raise ValueError("expert index out of range")
    require_cuda(packed)
    out = torch.empty((in_features, out_features), dtype=torch.float16, device=packed.device)
    check(lib().moe_trellis_decode_f16(ptr(packed), _nbytes(packed), k, in_features, out_features,
                                       sharded_side, expert, ptr(out), stream(packed.device)))
    return out


def hadamard_matrix(n=128, device=None):
    """Normalised Sylvester Hadamard matrix (inspection helper)."""
    h = torch.ones((1, 1), dtype=torch.float64)
    while h.shape[0] < n:
        h = torch.cat([torch.cat([h, h], 1), torch.cat([h, -h], 1)], 0)
    return (h / math.sqrt(n)).to(device=device, dtype=torch.float32)


def _block_hadamard(m, dim):
    """Apply H128 to independent 128-blocks along `dim` of a float32 matrix (inspection only)."""
    h = hadamard_matrix(128, m.device)
    m = m.transpose(dim, -1)
    shape = m.shape
    y = (m.reshape(-1, 128) @ h).reshape(shape)
    return y.transpose(dim, -1)


def dequantize_trellis(packed, suh, svh, k, in_features, out_features, sharded_side=1):
    """Public matrix [out, in] = diag(svh) H inner^T H diag(suh) (exlr8/trellis.py:199-214).

    For inspection and tests; the inner decode runs in the HIP kernel.
    """
    if _check_format(packed, k, in_features, out_features, sharded_side) != 1:
        raise ValueError("dense dequantization requires one matrix")
    inner = decode_inner(packed, k, in_features, out_features, sharded_side).float()    # [in, out]
    # H128 along the output axis, transpose to [out, in], then H128 along the input axis
    weight = _block_hadamard(_block_hadamard(inner, 1).T.contiguous(), 1)
    return weight * svh.float()[:, None] * suh.float()[None, :]


def swiglu(gate, up):
    """Typed SwiGLU of two bf16 tensors of one shape (the activation of exlr8/experts.py:183)."""
    if gate.shape != up.shape or gate.dtype != BF16 or up.dtype != BF16:
        raise ValueError("swiglu takes two bf16 tensors of one shape")
    require_cuda(gate, up)
    gate, up = gate.contiguous(), up.contiguous()
    out = torch.empty_like(gate)
    check(lib().moe_swiglu_bf16(ptr(gate), ptr(up), gate.numel(), ptr(out), stream(gate.device)))
    return out


def _rows_for(x, indices, in_features):
    if x.shape[-1] != in_features:
        raise ValueError("activation width does not match in_features")
    if tuple(x.shape[:-1]) == tuple(indices.shape):
        return True
    if tuple(x.shape[:-1]) == tuple(indices.shape[:-1]):
        return False
    raise ValueError("activation rows do not match the expert indices")


def expert_linear(x, indices, packed, in_scale, out_scale, k, in_features, out_features, sharded_side=1):
    """Apply selected experts; return [*indices.shape, out_features] (exlr8/trellis.py:172-196).

    ``x`` is bf16 with one row per token ([..., in]) or per expert slot ([..., slots, in]).
    """
    experts = _check_format(packed, k, in_features, out_features, sharded_side)
    per_slot = _rows_for(x, indices, in_features)
    if tuple(in_scale.shape) != (experts, in_features) or tuple(out_scale.shape) != (experts, out_features):
        raise ValueError("expert side vectors must contain full signed channel scales")
    if x.dtype != BF16:
        raise ValueError("this build computes bf16 activations")
    require_cuda(x, indices, packed, in_scale, out_scale)
    slots = indices.shape[-1] if indices.dim() else 1
    ids = indices.reshape(-1, slots).to(torch.int32).contiguous()
    rows = ids.shape[0]
    xr = x.reshape(-1, in_features).contiguous()
    y = torch.empty((rows * slots, out_features), dtype=BF16, device=x.device)
    if k != 4:
        # K2/K3: the generic-window grouped trellis kernel (all rows in one call)
        if sharded_side not in (1, 2):
            raise ValueError("K2/K3 expert linears take side 1 or 2 storage")
        need = lib().moe_trellis_grouped_linear_workspace_bytes(rows, slots, in_features, out_features, experts)
        ws = torch.empty(need, dtype=torch.uint8, device=x.device)
        check(lib().moe_trellis_grouped_linear(k, ptr(xr), int(per_slot), ptr(ids), rows, slots, ptr(packed),
                                               _nbytes(packed), ptr(in_scale), ptr(out_scale), in_features,
                                               out_features, sharded_side, ptr(y), ptr(ws), ws.numel(),
                                               stream(x.device)))
        return y.reshape(*indices.shape, out_features)
    ws = workspace(x.device, max(in_features, out_features), max(in_features, out_features))
    step = max(1, 72 // slots)
    st = stream(x.device)
    for r0 in range(0, rows, step):
        r1 = min(rows, r0 + step)
        xs = xr[r0 * slots:r1 * slots] if per_slot else xr[r0:r1]
        check(lib().moe_k4_expert_linear(ptr(xs), int(per_slot), ptr(ids[r0:r1]), r1 - r0, slots, ptr(packed),
                                         _nbytes(packed), ptr(in_scale), ptr(out_scale), in_features, out_features,
                                         sharded_side, ptr(y[r0 * slots:r1 * slots]), ptr(ws), ws.numel(), st))
    return y.reshape(*indices.shape, out_features)


def trellis_linear(x, packed, suh, svh, k, in_features, out_features, sharded_side=1):
    """One dense stored trellis matrix (exlr8/trellis.py:157-169)."""
    if _check_format(packed, k, in_features, out_features, sharded_side) != 1:
        raise ValueError("dense trellis requires one matrix")
    if x.shape[-1] != in_features or suh.numel() != in_features or svh.numel() != out_features:
        raise ValueError("activation or side vector dimensions do not match")
    ids = torch.zeros(x.shape[:-1] + (1,), dtype=torch.int32, device=x.device)
    y = expert_linear(x[..., None, :], ids, packed, suh.reshape(1, -1), svh.reshape(1, -1), k,
                      in_features, out_features, sharded_side)
    return y[..., 0, :]
