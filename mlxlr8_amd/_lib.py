"""ctypes loader for libmoe_mi355x.so and small helpers shared by the host modules."""
import ctypes
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "libmoe_mi355x.so"


class LibraryMissing(RuntimeError):
    """Raised when the HIP extension has not been built; there is no CPU fallback."""


class MoeError(RuntimeError):
    pass


_lib = None

_VP, _I32, _I64, _SZ = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_size_t
_SIGNATURES = {
    "moe_version": (ctypes.c_char_p, []),
    "moe_last_error": (ctypes.c_char_p, []),
    "moe_init": (_I32, []),
    "moe_decode_status": (_I32, [_VP, _I32, _I32, _I32, _VP, _VP]),
    "moe_set_wait_bound": (_I32, [_I32]),
    "moe_k4_item_list": (_I32, [_I32, _I32, _I32, _I32, _VP, _I32]),
    "moe_codebook_e4m3": (_I32, [_VP, _VP]),
    "moe_route_f32": (_I32, [_VP, _VP, _I32, _VP, _VP, _VP]),
    "moe_router_logits": (_I32, [_VP, _VP, _I32, _I32, _I32, _VP, _VP]),
    "moe_trellis_decode_f16": (_I32, [_VP, _I64, _I32, _I32, _I32, _I32, _I64, _VP, _VP]),
    "moe_swiglu_bf16": (_I32, [_VP, _VP, _I64, _VP, _VP]),
    "moe_k4_expert_linear": (_I32, [_VP, _I32, _VP, _I32, _I32, _VP, _I64, _VP, _VP, _I32, _I32, _I32, _VP,
                                    _VP, _SZ, _VP]),
    "moe_k4_mlp": (_I32, [_VP, _VP, _I32, _I32, _VP, _VP, _VP, _I64] + [_VP] * 6 + [_I32, _I32, _VP, _VP, _SZ, _VP]),
    "moe_k4_mlp_finish": (_I32, [_VP, _VP, _VP, _VP, _I32, _VP, _VP, _VP, _I64] + [_VP] * 6
                          + [_I32, _I32, _VP, _VP, _SZ, _VP]),
    "moe_k4_moe_decode": (_I32, [_VP, _VP, _I32, _VP, _VP, _VP, _VP, _VP, _I64] + [_VP] * 6
                          + [_I32, _I32, _VP, _VP, _VP, _VP, _SZ, _VP]),
    "moe_trellis_mlp": (_I32, [_I32, _VP, _VP, _I32, _I32, _VP, _VP, _VP, _I64] + [_VP] * 6
                        + [_I32, _I32, _VP, _VP, _SZ, _VP]),
    "moe_trellis_mlp_finish": (_I32, [_I32, _VP, _VP, _VP, _VP, _I32, _VP, _VP, _VP, _I64] + [_VP] * 6
                               + [_I32, _I32, _VP, _VP, _SZ, _VP]),
    "moe_trellis_moe_decode": (_I32, [_I32, _VP, _VP, _I32, _VP, _VP, _VP, _VP, _VP, _I64] + [_VP] * 6
                               + [_I32, _I32, _VP, _VP, _VP, _VP, _SZ, _VP]),
    "moe_k4_layer_decode": (_I32, [_VP, _VP, _VP, ctypes.c_float, _I32, _VP, _VP, _VP, _VP, _VP, _I64] + [_VP] * 6
                            + [_I32, _I32, _VP, _VP, _VP, _VP, _SZ, _VP]),
    "moe_residual_rmsnorm": (_I32, [_VP, _VP, _VP, _I32, _I32, ctypes.c_float, _VP, _VP, _VP]),
    "moe_workspace_bytes": (_SZ, [_I32, _I32]),
    "moe_profile_events": (_I32, [_VP, _I32]),
    "moe_mxfp4_mlp": (_I32, [_VP, _VP, _I32, _I32, _VP, _VP, _VP, _VP, _I64] + [_VP] * 5
                      + [_I32, _I32, _VP, _VP, _SZ, _VP]),
    "moe_mxfp4_mlp_finish": (_I32, [_VP, _VP, _VP, _VP, _I32, _VP, _VP, _VP, _VP, _I64] + [_VP] * 5
                             + [_I32, _I32, _VP, _VP, _SZ, _VP]),
    "moe_mxfp4_moe_decode": (_I32, [_VP, _VP, _I32, _VP, _VP, _VP, _VP, _VP, _VP, _I64] + [_VP] * 5
                             + [_I32, _I32, _VP, _VP, _VP, _VP, _SZ, _VP]),
    "moe_mxfp4_workspace_bytes": (_SZ, [_I32, _I32]),
    "moe_mxfp4_moe_decode_noalloc": (_I32, [_VP, _VP, _I32, _VP, _VP, _VP, _VP, _VP, _VP, _I64] + [_VP] * 5
                                     + [_I32, _I32, _VP, _VP, _VP, _VP]),
    "moe_segment_table": (_I32, [_VP, _I32, _I32, _I32, _VP, _VP, _VP, _VP, _I32, _VP, _VP]),
    "moe_mxfp4_prefill": (_I32, [_VP, _VP, _I32, _VP, _VP, _VP, _VP, _VP, _VP, _I64] + [_VP] * 5
                          + [_I32, _I32, _VP, _VP, _VP, _VP, _SZ, _VP]),
    "moe_mxfp4_prefill_workspace_bytes": (_SZ, [_I32, _I32, _I32, _I64]),
    "moe_mxfp4_grouped_mlp": (_I32, [_VP, _VP, _I32, _I32, _VP, _VP, _VP, _VP, _I64] + [_VP] * 5
                              + [_I32, _I32, _VP, _VP, _SZ, _VP]),
    "moe_mxfp4_grouped_mlp_workspace_bytes": (_SZ, [_I32, _I32, _I32, _I32, _I64]),
    "moe_k4_to_mxfp4": (_I32, [_VP, _I64, _I32, _I32, _I32, _VP, _VP, _VP, _VP, _I32, _I32, _VP, _SZ, _VP]),
    "moe_k4_to_mxfp4_workspace_bytes": (_SZ, [_I32, _I32]),
    "moe_k4_grouped_mlp": (_I32, [_VP, _VP, _I32, _I32, _VP, _VP, _VP, _I64] + [_VP] * 6 + [_I32, _I32, _VP, _VP, _SZ,
                                                                                      _VP]),
    "moe_k4_grouped_mlp_workspace_bytes": (_SZ, [_I32, _I32, _I32, _I32, _I64]),
    "moe_trellis_grouped_linear": (_I32, [_I32, _VP, _I32, _VP, _I32, _I32, _VP, _I64, _VP, _VP, _I32, _I32, _I32,
                                          _VP, _VP, _SZ, _VP]),
    "moe_trellis_grouped_linear_workspace_bytes": (_SZ, [_I32, _I32, _I32, _I32, _I64]),
    "moe_combine_values": (_I32, [_VP, _VP, _VP, _I32, _I32, _VP, _VP]),
    "moe_trellis_grouped_mlp": (_I32, [_I32, _VP, _VP, _I32, _I32, _VP, _VP, _VP, _I64] + [_VP] * 6
                                + [_I32, _I32, _VP, _VP, _SZ, _VP]),
}


def lib():
    """Load the HIP library (once).  Raises LibraryMissing if it was never built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise LibraryMissing(f"{LIB_PATH} is missing: run `python -m mlxlr8_amd.build` "
                                 "(the MoE path has no CPU fallback)")
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype, fn.argtypes = res, args
        _lib = handle
    return _lib


def exported_symbols():
    return list(_SIGNATURES)


def check(rc):
    """Map a C-ABI return code to the reference's exception types."""
    if rc == 0:
        return
    msg = lib().moe_last_error().decode(errors="replace")
    if rc < 0:
        raise ValueError(msg)
    raise MoeError(f"HIP error {rc}: {msg}")


def ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def stream(device=None):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


_workspaces = {}


def workspace(device, hidden, intermediate, kind="k4"):
    """A zero-initialised scratch buffer per (device, current stream, shape, kind): calls on one stream
    run in order and share it; calls on different streams get different buffers (sharing one would
    race)."""
    key = (str(device), torch.cuda.current_stream(device).cuda_stream, int(hidden), int(intermediate), kind)
    ws = _workspaces.get(key)
    if ws is None:
        size_fn = lib().moe_mxfp4_workspace_bytes if kind == "mxfp4" else lib().moe_workspace_bytes
        nbytes = size_fn(int(hidden), int(intermediate))
        ws = torch.zeros(nbytes, dtype=torch.uint8, device=device)
        _workspaces[key] = ws
    return ws


# workspace kinds of moe_decode_status (include/moe_mi355x.h)
STATUS_K4, STATUS_MXFP4, STATUS_MXFP4_NOALLOC = 0, 1, 2


def decode_status(ws, kind, hidden, intermediate, stream_handle):
    """Fused-block launches on one workspace whose bounded waits ran out since the last query (reset
    by the query; synchronises the workspace's stream)."""
    n = ctypes.c_int32(0)
    check(lib().moe_decode_status(ptr(ws) if ws is not None else None, int(kind), int(hidden), int(intermediate),
                                  ctypes.byref(n), ctypes.c_void_p(stream_handle)))
    return int(n.value)


def stalled_launches():
    """Fused decode launches, over every workspace this process created, in which a bounded
    cross-wave wait ran out since the last call (their outputs are unreliable); resets the counts.
    The reference raises on failure; the decode entries cannot without a host synchronisation per
    call, so a caller checks here at its own synchronisation points."""
    total = 0
    for (dev, stream_handle, hidden, inter, kind), ws in list(_workspaces.items()):
        status_kind = STATUS_MXFP4 if kind == "mxfp4" else STATUS_K4
        with torch.cuda.device(ws.device):
            total += decode_status(ws, status_kind, hidden, inter, stream_handle)
    return total


def set_wait_bound(polls):
    """Bound of the fused blocks' cross-wave waits (0 = the default ~50 ms); for tests."""
    check(lib().moe_set_wait_bound(int(polls)))


def require_cuda(*tensors):
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise ValueError("MoE kernels take device tensors (got a CPU tensor)")
