"""Memory-mapped safetensors reader for expert checkpoints.

The format: an 8-byte little-endian header length N, N bytes of JSON mapping each tensor name to
``{"dtype", "shape", "data_offsets": [begin, end]}`` (offsets relative to the data section, which
starts right after the header) plus an optional ``"__metadata__"`` string map, then the data.
The file is mapped read-only once; a tensor, or a byte span of it (one expert of a packed
projection), is a zero-copy numpy view of the mapping until it is copied to the device.  Nothing
in the file is executed: the header is JSON and tensor bytes are reinterpreted, never unpickled.

Used by ``experts.layer_arrays`` the way the reference's loader uses ``exlr8/weights.py``.
"""
from __future__ import annotations

import json
import mmap
from pathlib import Path

import numpy as np

# safetensors dtype tags -> numpy dtypes (BF16 is kept as its uint16 bit pattern)
DTYPES = {
    "BOOL": np.dtype(np.bool_), "U8": np.dtype(np.uint8), "I8": np.dtype(np.int8),
    "U16": np.dtype("<u2"), "I16": np.dtype("<i2"), "F16": np.dtype("<f2"), "BF16": np.dtype("<u2"),
    "U32": np.dtype("<u4"), "I32": np.dtype("<i4"), "F32": np.dtype("<f4"),
    "U64": np.dtype("<u8"), "I64": np.dtype("<i8"), "F64": np.dtype("<f8"),
}
MAX_HEADER = 100 << 20


class SafetensorsFile:
    """One safetensors file: ``names``, ``metadata``, ``dtype(name)``, ``shape(name)``,
    ``array(name)`` (the whole tensor, shaped) and ``span(name, offset, nbytes)`` (a flat range)."""

    def __init__(self, path):
        self.path = Path(path)
        with self.path.open("rb") as f:
            self._map = mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ)
        size = len(self._map)
        if size < 8:
            raise ValueError(f"{self.path}: not a safetensors file (shorter than its length prefix)")
        n = int.from_bytes(self._map[:8], "little")
        if n > min(MAX_HEADER, size - 8):
            raise ValueError(f"{self.path}: header length {n} does not fit the file")
        header = json.loads(bytes(self._map[8:8 + n]).decode("utf-8"))
        if not isinstance(header, dict):
            raise ValueError(f"{self.path}: the header is not a JSON object")
        self.metadata = header.pop("__metadata__", None) or {}
        self._base = 8 + n
        data = size - self._base
        self._entries = {}
        spans = []
        for name, entry in header.items():
            tag = entry.get("dtype")
            dt = DTYPES.get(tag)
            shape = entry.get("shape")
            offsets = entry.get("data_offsets")
            if dt is None or not isinstance(shape, list) or not isinstance(offsets, list) or len(offsets) != 2:
                raise ValueError(f"{self.path}: malformed header entry for {name!r}")
            begin, end = int(offsets[0]), int(offsets[1])
            count = int(np.prod(shape, dtype=np.int64)) if shape else 1
            if any(int(d) < 0 for d in shape) or not 0 <= begin <= end <= data or end - begin != count * dt.itemsize:
                raise ValueError(f"{self.path}: tensor {name!r} does not match its byte range")
            self._entries[name] = (dt, tuple(int(d) for d in shape), begin, end, tag)
            spans.append((begin, end, name))
        spans.sort()
        for (b0, e0, n0), (b1, _, n1) in zip(spans, spans[1:]):
            if b1 < e0:
                raise ValueError(f"{self.path}: tensors {n0!r} and {n1!r} overlap")

    @property
    def names(self):
        return list(self._entries)

    def _entry(self, name):
        try:
            return self._entries[name]
        except KeyError:
            raise KeyError(f"{self.path}: no tensor {name!r}") from None

    def dtype(self, name):
        return self._entry(name)[0]

    def shape(self, name):
        return self._entry(name)[1]

    def array(self, name):
        """The whole tensor as a read-only numpy view with its shape."""
        dt, shape, begin, end, _ = self._entry(name)
        return np.frombuffer(self._map, dtype=dt, count=(end - begin) // dt.itemsize,
                             offset=self._base + begin).reshape(shape)

    def span(self, name, offset, nbytes):
        """Bytes [offset, offset + nbytes) of a tensor as a flat view of its element type."""
        dt, _, begin, end, _ = self._entry(name)
        if offset < 0 or nbytes < 0 or offset + nbytes > end - begin or (offset | nbytes) % dt.itemsize:
            raise ValueError(f"{self.path}: span ({offset}, {nbytes}) is outside tensor {name!r} or splits an element")
        return np.frombuffer(self._map, dtype=dt, count=nbytes // dt.itemsize, offset=self._base + begin + offset)

    def tensor(self, name, device=None):
        """The tensor as a torch tensor (BF16 as bfloat16), copied out of the mapping."""
        import torch
        out = torch.from_numpy(np.array(self.array(name)))
        if self._entry(name)[4] == "BF16":
            out = out.view(torch.bfloat16)
        return out.to(device) if device is not None else out
