"""The C-ABI library loads on a CPU-only host and exports every symbol include/moe_mi355x.h declares.
No compute is launched here (there is no GPU in the CPU test tier)."""
import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def _declared():
    text = (ROOT / "include" / "moe_mi355x.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(moe_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def so():
    from mlxlr8_amd._lib import LIB_PATH
    if not LIB_PATH.exists():
        pytest.fail("libmoe_mi355x.so is not built: run python -m mlxlr8_amd.build")
    return ctypes.CDLL(str(LIB_PATH))


def test_every_declared_symbol_is_exported(so):
    names = _declared()
    assert len(names) >= 10
    for name in names:
        assert hasattr(so, name), name


def test_python_binding_covers_header():
    from mlxlr8_amd._lib import exported_symbols
    assert set(_declared()) <= set(exported_symbols())


def test_version_and_workspace(so):
    so.moe_version.restype = ctypes.c_char_p
    assert b"gfx950" in so.moe_version()
    so.moe_workspace_bytes.restype = ctypes.c_size_t
    assert so.moe_workspace_bytes(6144, 2048) > 32 * 1024 * 1024


def test_argument_errors_without_device():
    from mlxlr8_amd._lib import lib
    L = lib()
    assert L.moe_route_f32(None, None, 1, None, None, None) == -1
    assert b"null" in L.moe_last_error()
    assert L.moe_trellis_decode_f16(ctypes.c_void_p(16), 128 * 128 // 2, 5, 128, 128, 1, 0, ctypes.c_void_p(16), None) == -1
    assert b"2, 3, or 4" in L.moe_last_error()
    assert L.moe_trellis_decode_f16(ctypes.c_void_p(16), 128 * 128 // 2, 3, 128, 128, 1, 0, ctypes.c_void_p(16), None) == -1
    assert b"byte count" in L.moe_last_error()
    assert L.moe_trellis_decode_f16(ctypes.c_void_p(16), 5, 4, 128, 128, 1, 0, ctypes.c_void_p(16), None) == -1
    assert b"byte count" in L.moe_last_error()


def test_host_validation_messages():
    import torch
    from mlxlr8_amd.trellis import _check_format
    with pytest.raises(ValueError, match="byte count"):
        _check_format(torch.zeros(5, dtype=torch.uint8), 4, 128, 128, 1)
    with pytest.raises(ValueError, match="multiples of 128"):
        _check_format(torch.zeros(64, dtype=torch.uint8), 4, 100, 128, 1)
    with pytest.raises(ValueError, match="width"):
        _check_format(torch.zeros(64, dtype=torch.uint8), 5, 128, 128, 1)
    assert _check_format(torch.zeros(3 * 128 * 128 // 2, dtype=torch.uint8), 4, 128, 128, 1) == 3


def test_product_never_imports_oracle():
    for path in (ROOT / "mlxlr8_amd").rglob("*.py"):
        text = path.read_text()
        assert "import oracle" not in text and "from oracle" not in text, path


def test_encode_and_grouped_argument_errors_without_device():
    from mlxlr8_amd._lib import lib
    L = lib()
    p = ctypes.c_void_p(256)
    # moe_k4_to_mxfp4: in_scale and unit come together; rows must fit; codes aligned; whole experts
    assert L.moe_k4_to_mxfp4(p, 128 * 128 // 2, 128, 128, 1, p, None, p, p, 256, 0, p, 1 << 20, None) == -1
    assert b"together" in L.moe_last_error()
    assert L.moe_k4_to_mxfp4(p, 128 * 128 // 2, 128, 128, 1, None, None, p, p, 128, 64, p, 1 << 20, None) == -1
    assert b"destination" in L.moe_last_error()
    assert L.moe_k4_to_mxfp4(p, 100, 128, 128, 2, None, None, p, p, 128, 0, p, 1 << 20, None) == -1
    assert b"whole number" in L.moe_last_error()
    assert L.moe_k4_to_mxfp4(p, 128 * 128 // 2, 128, 128, 2, None, None, p, p, 128, 0, p, 16, None) == -3
    assert b"workspace" in L.moe_last_error()
    assert L.moe_k4_to_mxfp4_workspace_bytes(6144, 2048) == 6144 * 2048 * 2
    # moe_k4_grouped_mlp: widths, whole experts, workspace
    args = [p, p, 4, 9, p, p, p, 128 * 128 // 2] + [p] * 6
    assert L.moe_k4_grouped_mlp(*args[:7], 128 * 128 // 2, *args[8:], 100, 128, p, p, 1 << 30, None) == -1
    assert b"multiples of 128" in L.moe_last_error()
    assert L.moe_k4_grouped_mlp(*args[:7], 1000, *args[8:], 128, 128, p, p, 1 << 30, None) == -1
    assert b"whole number" in L.moe_last_error()
    assert L.moe_k4_grouped_mlp(*args, 128, 128, p, p, 16, None) == -3
    assert b"workspace" in L.moe_last_error()
    assert L.moe_k4_grouped_mlp_workspace_bytes(512, 9, 6144, 2048, 257) > 0


def test_k4_decode_rejects_misaligned_rows_without_device():
    """The fused K4 decode block reads x and side-vector rows 8 bytes at a time: a misaligned row
    pointer is refused before anything is launched."""
    from mlxlr8_amd._lib import lib
    L = lib()
    p = ctypes.c_void_p(256)
    bytes_ = 3 * 128 * 128 // 2   # three K4 experts of 128 x 128
    args = lambda x, in_g: [x, p, 1, 9, p, p, p, bytes_, in_g, p, p, p, p, p, 128, 128, p, p, 1 << 30, None]
    assert L.moe_k4_mlp(*args(ctypes.c_void_p(258), p)) == -1
    assert b"aligned" in L.moe_last_error()
    assert L.moe_k4_mlp(*args(p, ctypes.c_void_p(260))) == -1
    assert b"aligned" in L.moe_last_error()


def test_trellis_grouped_and_combine_argument_errors_without_device():
    from mlxlr8_amd._lib import lib
    L = lib()
    p = ctypes.c_void_p(256)
    k3 = 128 * 128 * 3 // 8
    args = [p, p, 4, 9, p, p, p, k3] + [p] * 6
    assert L.moe_trellis_grouped_mlp(5, *args, 128, 128, p, p, 1 << 30, None) == -1
    assert b"2, 3, or 4" in L.moe_last_error()
    # K4 byte count is not a whole number of K3 experts
    assert L.moe_trellis_grouped_mlp(3, *args[:7], 128 * 128 // 2, *args[8:], 128, 128, p, p, 1 << 30, None) == -1
    assert b"K3 experts" in L.moe_last_error()
    assert L.moe_trellis_grouped_mlp(3, *args, 128, 128, p, p, 16, None) == -3
    lin = [p, 0, p, 4, 9, p, k3, p, p]
    assert L.moe_trellis_grouped_linear(3, *lin, 128, 128, 3, p, p, 1 << 30, None) == -1
    assert b"sharded_side" in L.moe_last_error()
    assert L.moe_trellis_grouped_linear(3, *lin, 128, 100, 1, p, p, 1 << 30, None) == -1
    assert b"multiples of 128" in L.moe_last_error()
    assert L.moe_trellis_grouped_linear(3, *lin, 128, 128, 1, p, p, 16, None) == -3
    need = L.moe_trellis_grouped_linear_workspace_bytes(4, 9, 6144, 2048, 257)
    assert 0 < need < L.moe_k4_grouped_mlp_workspace_bytes(4, 9, 6144, 2048, 257)
    assert L.moe_combine_values(p, p, p, 0, 128, p, None) == -1
    assert b"rows" in L.moe_last_error()
    assert L.moe_combine_values(ctypes.c_void_p(258), p, p, 1, 128, p, None) == -1
    assert b"aligned" in L.moe_last_error()


def test_status_and_wait_bound_argument_errors_without_device():
    from mlxlr8_amd._lib import lib
    L = lib()
    n = ctypes.c_int32(7)
    assert L.moe_set_wait_bound(-1) == -1
    assert b"wait bound" in L.moe_last_error()
    assert L.moe_decode_status(None, 0, 6144, 2048, ctypes.byref(n), None) == -1
    assert b"workspace" in L.moe_last_error()
    assert L.moe_decode_status(ctypes.c_void_p(256), 5, 6144, 2048, ctypes.byref(n), None) == -1
    assert b"kind" in L.moe_last_error()
    assert L.moe_decode_status(ctypes.c_void_p(256), 0, 0, 2048, None, None) == -1
    assert b"NULL" in L.moe_last_error()
    assert n.value == 7
