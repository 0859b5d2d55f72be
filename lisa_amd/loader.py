"""safetensors shard reader with the reference's header validation, and
upload of MLX packed quantized tensors to device memory.

Mirrors ``Shard::open`` / ``get_tensor`` of
crates/lisa-engine/src/core/loader.rs:57-157, 496-507: the 8-byte little-endian
header length, a JSON object header (``__metadata__`` skipped), dtypes
BF16/F32/F16/I64/I32/U32/U8/BOOL, a byte size that matches the shape, and
offsets inside the payload; a name is also looked up with the
``language_model.`` prefix.  The file is memory-mapped; tensors are copied
to the device on request (host -> HBM once, at load time).
"""
from __future__ import annotations

import json
import mmap
import os
import struct
from dataclasses import dataclass
from typing import Dict, Iterable, List, Tuple

import numpy as np

_DTYPES = {
    "BF16": (2, np.uint16),
    "F32": (4, np.float32),
    "F16": (2, np.float16),
    "I64": (8, np.int64),
    "I32": (4, np.int32),
    "U32": (4, np.uint32),
    "U8": (1, np.uint8),
    "BOOL": (1, np.bool_),
}
MAX_HEADER = 64 * 1024 * 1024


class ShardError(ValueError):
    """A malformed shard (the reference's ``bail!``/``ensure!`` failures)."""


@dataclass
class TensorInfo:
    dtype: str
    shape: Tuple[int, ...]
    start: int  # absolute byte offset in the file
    end: int


class Shard:
    def __init__(self, path: str):
        self.path = path
        f = open(path, "rb")
        try:
            size = os.fstat(f.fileno()).st_size
            if size < 8:
                raise ShardError(f"shard {path} too small")
            self._map = mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ)
        finally:
            f.close()
        n = len(self._map)
        (header_len,) = struct.unpack("<Q", self._map[:8])
        payload_start = header_len + 8
        if payload_start > n or header_len > MAX_HEADER:
            raise ShardError(f"shard {path} has an invalid or oversized header")
        try:
            header = json.loads(bytes(self._map[8:payload_start]))
        except json.JSONDecodeError as e:
            raise ShardError(f"parsing shard header {path}: {e}") from None
        if not isinstance(header, dict):
            raise ShardError("safetensors header must be an object")
        self.tensors: Dict[str, TensorInfo] = {}
        for name, info in header.items():
            if name == "__metadata__":
                continue
            if not isinstance(info, dict):
                raise ShardError(f"bad record for {name}")
            dt = info.get("dtype")
            if dt not in _DTYPES:
                raise ShardError(f"unsupported dtype {dt} for {name}")
            shape = info.get("shape")
            if not isinstance(shape, list):
                raise ShardError(f"missing shape for {name}")
            dims = []
            for d in shape:
                if not isinstance(d, int) or isinstance(d, bool) or d < 0 or d > 2**31 - 1:
                    raise ShardError(f"invalid dimension for {name}: {d}")
                dims.append(d)
            expected = _DTYPES[dt][0] * int(np.prod(dims, dtype=np.int64)) if dims else _DTYPES[dt][0]
            rng = info.get("data_offsets")
            if not isinstance(rng, list):
                raise ShardError(f"missing data_offsets for {name}")
            if len(rng) != 2:
                raise ShardError(f"data_offsets must have two entries for {name}")
            for v in rng:
                if not isinstance(v, int) or isinstance(v, bool) or v < 0:
                    raise ShardError(f"invalid data offset for {name}: {v}")
            start, end = rng
            if not (start <= end and end <= n - payload_start):
                raise ShardError(f"tensor {name} exceeds shard payload bounds")
            if end - start != expected:
                raise ShardError(f"tensor byte size differs from shape for {name}")
            self.tensors[name] = TensorInfo(dt, tuple(dims), payload_start + start, payload_start + end)

    def names(self) -> Iterable[str]:
        return self.tensors.keys()

    def _resolve(self, name: str) -> str:
        for cand in (name, f"language_model.{name}"):
            if cand in self.tensors:
                return cand
        raise KeyError(f"tensor {name} not found in shard")

    def numpy(self, name: str) -> np.ndarray:
        """Host view of a tensor (bf16 as uint16 bit patterns)."""
        info = self.tensors[self._resolve(name)]
        arr = np.frombuffer(self._map, dtype=_DTYPES[info.dtype][1], count=(info.end - info.start) // _DTYPES[info.dtype][0],
                            offset=info.start)
        return arr.reshape(info.shape)

    def to_device(self, name: str, device):
        """Copy one tensor to device memory as a torch tensor (bf16 stays bf16,
        U32 packed codes become int32 storage of the same bits)."""
        import torch

        info = self.tensors[self._resolve(name)]
        a = self.numpy(name)
        if info.dtype == "BF16":
            t = torch.from_numpy(a.view(np.int16).copy()).view(torch.bfloat16)
        elif info.dtype == "U32":
            t = torch.from_numpy(a.view(np.int32).copy())
        else:
            t = torch.from_numpy(a.copy())
        return t.to(device)

    def close(self):
        self._map.close()


def write_safetensors(path: str, tensors: Dict[str, Tuple[str, np.ndarray]], metadata=None) -> None:
    """Minimal writer (tests and tools): {name: (dtype, array)} with arrays in that dtype's layout."""
    header = {}
    off = 0
    blobs: List[bytes] = []
    for name, (dt, arr) in tensors.items():
        b = np.ascontiguousarray(arr).tobytes()
        header[name] = {"dtype": dt, "shape": list(arr.shape), "data_offsets": [off, off + len(b)]}
        off += len(b)
        blobs.append(b)
    if metadata:
        header["__metadata__"] = metadata
    hb = json.dumps(header).encode()
    hb += b" " * ((8 - len(hb) % 8) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(hb)))
        f.write(hb)
        for b in blobs:
            f.write(b)
