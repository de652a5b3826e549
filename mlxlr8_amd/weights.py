"""Safetensors reads of single tensors and byte ranges (mirrors the reference ``exlr8/weights.py``).

The header is parsed once; tensor bytes are read on request with ``numpy.fromfile`` (no pickle,
no framework loader), so one expert's byte range can be read without touching the rest.
"""
from __future__ import annotations

import json
import struct
from pathlib import Path

import numpy as np

_DTYPES = {
    "U8": "u1", "I8": "i1", "U16": "<u2", "I16": "<i2", "U32": "<u4", "I32": "<i4", "U64": "<u8",
    "I64": "<i8", "F16": "<f2", "BF16": "<u2", "F32": "<f4", "F64": "<f8", "BOOL": "?",
}


class SafeTensorFile:
    """``header``/``metadata``/``tensors`` of one file; ``raw`` reads a tensor or a byte range."""

    def __init__(self, path):
        self.path = Path(path)
        with self.path.open("rb") as handle:
            size = struct.unpack("<Q", handle.read(8))[0]
            self.header = json.loads(handle.read(size))
        self.data_offset = 8 + size
        self.metadata = self.header.get("__metadata__", {})
        self.tensors = {k: v for k, v in self.header.items() if k != "__metadata__"}

    def raw(self, name, start_bytes=0, byte_count=None):
        """The tensor with its shape, or a flat range of it (BF16 as uint16 bit patterns)."""
        info = self.tensors[name]
        begin, end = info["data_offsets"]
        dtype = np.dtype(_DTYPES[info["dtype"]])
        whole = start_bytes == 0 and byte_count is None
        if byte_count is None:
            byte_count = end - begin - start_bytes
        if (start_bytes < 0 or byte_count < 0 or start_bytes + byte_count > end - begin
                or start_bytes % dtype.itemsize or byte_count % dtype.itemsize):
            raise ValueError(f"invalid byte range for {name}: {start_bytes}, {byte_count}")
        out = np.fromfile(self.path, dtype=dtype, count=byte_count // dtype.itemsize,
                          offset=self.data_offset + begin + start_bytes)
        if out.nbytes != byte_count:
            raise ValueError(f"truncated tensor {name} in {self.path}")
        return out.reshape(info["shape"]) if whole else out

    def load(self, name, device=None):
        """The tensor as a torch tensor (BF16 as bfloat16) on ``device``."""
        import torch
        array = self.raw(name)
        tensor = torch.from_numpy(np.ascontiguousarray(array))
        if self.tensors[name]["dtype"] == "BF16":
            tensor = tensor.view(torch.bfloat16)
        return tensor.to(device) if device is not None else tensor
