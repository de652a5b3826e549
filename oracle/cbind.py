"""ctypes binding of the C oracle (``moe_oracle.c``).  Test infrastructure only."""
import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
SO = HERE / "libmoe_oracle.so"


def build(force=False):
    """Compile ``libmoe_oracle.so`` with the committed Makefile."""
    if force or not SO.exists() or SO.stat().st_mtime < (HERE / "moe_oracle.c").stat().st_mtime:
        subprocess.run(["make", "-s", "-f", str(HERE / "Makefile")], check=True, cwd=HERE)
    return SO


_lib = None


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p) if a is not None else None


class _Oracle:
    def __init__(self, handle):
        self.h = handle
        vp, i32, i64, f32 = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_float
        sig = {
            "orc_codebook": (None, [vp]),
            "orc_round_e4m3": (f32, [f32]),
            "orc_check_format": (i32, [i64, i32, i32, i32, i32]),
            "orc_codeword_at": (ctypes.c_uint32, [vp, i32, i32, i32, i32, i64, i32, i32]),
            "orc_decode_trellis": (None, [vp, i32, i32, i32, i32, i64, vp]),
            "orc_hadamard128": (None, [vp, i64]),
            "orc_router_logits": (None, [vp, vp, i32, i32, i32, vp]),
            "orc_route": (None, [vp, vp, i32, vp, vp]),
            "orc_swiglu_bf16": (f32, [f32, f32]),
            "orc_k4_linear": (None, [vp, vp, i32, vp, i32, i32, i32, i32, vp, vp, vp]),
            "orc_mxfp4_linear": (None, [vp, vp, i32, vp, vp, i32, i32, vp]),
            "orc_mx_quantize_row": (None, [vp, i32, vp, vp]),
            "orc_k4_to_mxfp4": (None, [vp, i32, i32, i32, i64, vp, vp, vp, vp, i32, i32]),
            "orc_k4_moe": (None, [vp, vp, vp, vp, i32, i32, i32, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp]),
            "orc_trellis_moe": (None, [i32, vp, vp, vp, vp, i32, i32, i32, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp]),
            "orc_mxfp4_moe": (None, [vp, vp, vp, vp, i32, i32, i32, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp]),
            "orc_residual_rmsnorm": (None, [vp, vp, vp, i32, i32, f32, vp, vp]),
            "orc_segment_table": (i32, [vp, i32, i32, i32, vp, vp, vp, vp, vp, vp]),
            "orc_num_threads": (i32, []),
            "orc_f32_to_bf16": (ctypes.c_uint16, [f32]),
            "orc_f32_to_f16": (ctypes.c_uint16, [f32]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(handle, name)
            fn.restype, fn.argtypes = res, args

    # ---- thin numpy-facing wrappers ----
    def codebook(self):
        out = np.empty(65536, np.uint16)
        self.h.orc_codebook(_p(out))
        return out.view(np.float16)

    def round_e4m3(self, values):
        v = np.asarray(values, np.float32).ravel()
        return np.array([self.h.orc_round_e4m3(float(x)) for x in v], np.float32).reshape(np.shape(values))

    def check_format(self, nbytes, k, in_f, out_f, side):
        return self.h.orc_check_format(nbytes, k, in_f, out_f, side)

    def decode(self, packed, k, in_f, out_f, side, expert=0):
        packed = np.ascontiguousarray(packed, np.uint8)
        out = np.empty((in_f, out_f), np.float32)
        self.h.orc_decode_trellis(_p(packed), k, in_f, out_f, side, expert, _p(out))
        return out

    def hadamard(self, x):
        y = np.array(x, np.float32, copy=True, order="C")
        self.h.orc_hadamard128(_p(y), y.size)
        return y

    def router_logits(self, x_bf16_bits, w):
        x = np.ascontiguousarray(x_bf16_bits, np.uint16)
        w = np.ascontiguousarray(w, np.float32)
        rows, hidden = x.reshape(-1, w.shape[1]).shape
        out = np.empty((rows, w.shape[0]), np.float32)
        self.h.orc_router_logits(_p(x), _p(w), rows, hidden, w.shape[0], _p(out))
        return out

    def route(self, logits, bias):
        logits = np.ascontiguousarray(logits, np.float32).reshape(-1, 256)
        bias = np.ascontiguousarray(bias, np.float32)
        rows = logits.shape[0]
        idx = np.empty((rows, 9), np.uint32)
        sc = np.empty((rows, 8), np.float32)
        self.h.orc_route(_p(logits), _p(bias), rows, _p(idx), _p(sc))
        return idx, sc

    def swiglu_bf16(self, g, u):
        return np.array([self.h.orc_swiglu_bf16(float(a), float(b)) for a, b in zip(np.ravel(g), np.ravel(u))], np.float32)

    def k4_linear(self, x, ids, packed, in_f, out_f, side, in_scale, out_scale, k=4):
        x = np.ascontiguousarray(x, np.float32).reshape(-1, in_f)
        ids = np.ascontiguousarray(ids, np.uint32).ravel()
        y = np.empty((x.shape[0], out_f), np.float32)
        self.h.orc_k4_linear(_p(x), _p(ids), x.shape[0], _p(np.ascontiguousarray(packed)), k, in_f, out_f, side,
                             _p(np.ascontiguousarray(in_scale, np.uint16)), _p(np.ascontiguousarray(out_scale, np.uint16)), _p(y))
        return y

    def mxfp4_linear(self, x, ids, codes, scales, K, N):
        x = np.ascontiguousarray(x, np.float32).reshape(-1, K)
        ids = np.ascontiguousarray(ids, np.uint32).ravel()
        y = np.empty((x.shape[0], N), np.float32)
        self.h.orc_mxfp4_linear(_p(x), _p(ids), x.shape[0], _p(np.ascontiguousarray(codes)), _p(np.ascontiguousarray(scales)), K, N, _p(y))
        return y

    def mx_quantize(self, v):
        """rows of float32 values [..., n] (n % 32 == 0) -> (codes uint8 [..., n/2], scales uint8 [..., n/32])"""
        v = np.ascontiguousarray(v, np.float32)
        n = v.shape[-1]
        flat = v.reshape(-1, n)
        codes = np.empty((flat.shape[0], n // 2), np.uint8)
        scales = np.empty((flat.shape[0], n // 32), np.uint8)
        for r in range(flat.shape[0]):
            self.h.orc_mx_quantize_row(_p(flat[r]), n, _p(codes[r]), _p(scales[r]))
        return codes.reshape(*v.shape[:-1], n // 2), scales.reshape(*v.shape[:-1], n // 32)

    def k4_to_mxfp4(self, packed, in_f, out_f, side, experts, in_scale, unit, codes, scales, row_offset):
        """fills codes [E, out_rows, in/2] / scales [E, out_rows, in/32] (uint8, C-contiguous) in place"""
        assert codes.flags.c_contiguous and scales.flags.c_contiguous
        ins = None if in_scale is None else np.ascontiguousarray(in_scale, np.uint16)
        un = None if unit is None else np.ascontiguousarray(unit, np.uint16)
        self.h.orc_k4_to_mxfp4(_p(np.ascontiguousarray(packed)), in_f, out_f, side, experts,
                               None if ins is None else _p(ins), None if un is None else _p(un),
                               _p(codes), _p(scales), codes.shape[1], row_offset)

    def k4_moe(self, x, idx9, scores8, residual, h, m, pg, pu, pd, in_g, out_g, in_u, out_u, in_d, out_d, want_values=False,
               k=4):
        x = np.ascontiguousarray(x, np.uint16).reshape(-1, h)
        rows = x.shape[0]
        out = np.empty((rows, h), np.uint16)
        values = np.empty((rows, 9, h), np.uint16) if want_values else None
        c = lambda a, t: np.ascontiguousarray(a, t)
        self.h.orc_trellis_moe(k, _p(x), _p(c(idx9, np.uint32)), _p(c(scores8, np.float32)), _p(c(residual, np.uint16)),
                               rows, h, m, _p(c(pg, np.uint8)), _p(c(pu, np.uint8)), _p(c(pd, np.uint8)),
                               *[_p(c(a, np.uint16)) for a in (in_g, out_g, in_u, out_u, in_d, out_d)], _p(out), _p(values))
        return (out, values) if want_values else out

    def mxfp4_moe(self, x, idx9, scores8, residual, h, m, gu_codes, gu_scales, d_codes, d_scales, unit, out_g, out_u, in_d, out_d,
                  want_values=False):
        x = np.ascontiguousarray(x, np.uint16).reshape(-1, h)
        rows = x.shape[0]
        out = np.empty((rows, h), np.uint16)
        values = np.empty((rows, 9, h), np.uint16) if want_values else None
        c = lambda a, t: np.ascontiguousarray(a, t)
        self.h.orc_mxfp4_moe(_p(x), _p(c(idx9, np.uint32)), _p(c(scores8, np.float32)), _p(c(residual, np.uint16)), rows, h, m,
                             _p(c(gu_codes, np.uint8)), _p(c(gu_scales, np.uint8)), _p(c(d_codes, np.uint8)), _p(c(d_scales, np.uint8)),
                             *[_p(c(a, np.uint16)) for a in (unit, out_g, out_u, in_d, out_d)], _p(out), _p(values))
        return (out, values) if want_values else out

    def residual_rmsnorm(self, x, r, w, eps=1e-5):
        x = np.ascontiguousarray(x, np.uint16)
        n = w.size
        rows = x.size // n
        h_out = np.empty((rows, n), np.uint16)
        out = np.empty((rows, n), np.uint16)
        self.h.orc_residual_rmsnorm(_p(x), _p(np.ascontiguousarray(r, np.uint16)) if r is not None else None,
                                    _p(np.ascontiguousarray(w, np.uint16)), rows, n, eps, _p(h_out), _p(out))
        return h_out, out

    def segment_table(self, ids, experts, block_rows):
        ids = np.ascontiguousarray(ids, np.uint32).ravel()
        n = ids.size
        order = np.empty(n, np.int32)
        counts = np.empty(experts, np.int32)
        starts = np.empty(experts, np.int32)
        cap = n // block_rows + experts + 1
        be, bf, bl = (np.empty(cap, np.int32) for _ in range(3))
        nb = self.h.orc_segment_table(_p(ids), n, experts, block_rows, _p(order), _p(counts), _p(starts), _p(be), _p(bf), _p(bl))
        return order, counts, starts, np.stack([be[:nb], bf[:nb], bl[:nb]])

    def num_threads(self):
        return self.h.orc_num_threads()


def lib():
    global _lib
    if _lib is None:
        build()
        _lib = _Oracle(ctypes.CDLL(str(SO)))
    return _lib


def native_f32(out_dir):
    """The CPU baseline build (fp32 accumulation, -march=native for this host) compiled into
    `out_dir` and loaded; None when it cannot be built here."""
    out = Path(out_dir)
    out.mkdir(parents=True, exist_ok=True)
    r = subprocess.run(["make", "-s", "-f", str(HERE / "Makefile"), "native", f"OUT={out}"], cwd=HERE,
                       capture_output=True, text=True)
    so = out / "libmoe_oracle_f32.so"
    if r.returncode != 0 or not so.exists():
        return None
    return _Oracle(ctypes.CDLL(str(so)))
