"""Engine-side quantized layers (crates/lisa-engine/src/core/quant.rs).

``QuantizedLinear`` holds the MLX packed triple on the device and runs
``quantized_matmul`` from liblisaq; ``QuantizedEmbedding`` dequantizes only
the gathered rows.  Loading validates the packed layout through the C ABI
(``lisaq_check_layout``) and re-derives the group size from the shapes as
``detect_group_size`` does (quant.rs:273-287, 400-428).
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch

from . import _lib, ops
from .loader import Shard

GROUP_SIZE = 64  # fallback group size when the shapes do not fix one
BITS = 4


def check_layout(w_shape, s_shape, b_shape, bits: int):
    """Validate an (N, Kq) / (N, G) / (N, G) packed triple; returns (K, group_size)."""
    K = ctypes.c_int64()
    gs = ctypes.c_int()
    lib = _lib.load()
    rc = lib.lisaq_check_layout(w_shape[0], w_shape[1], s_shape[0], s_shape[1], b_shape[0], b_shape[1], bits,
                                ctypes.byref(K), ctypes.byref(gs))
    _lib.check(rc)
    return K.value, gs.value


@dataclass
class QuantizedLinear:
    weight: torch.Tensor  # int32 storage of u32 [N, K*bits/32]
    scales: torch.Tensor  # bf16 [N, K/group_size]
    biases: torch.Tensor  # bf16 [N, K/group_size]
    group_size: int = GROUP_SIZE
    bits: int = BITS

    @classmethod
    def load(cls, shard: Shard, prefix: str, key: str = "", device="cuda", bits: int = BITS):
        """``{prefix}.{key}.weight/.scales/.biases`` (key may be empty), quant.rs:408-428."""
        path = (lambda s: f"{prefix}.{s}") if not key else (lambda s: f"{prefix}.{key}.{s}")
        ws, ss, bs = (shard.tensors[shard._resolve(path(s))].shape for s in ("weight", "scales", "biases"))
        _, gs = check_layout(ws, ss, bs, bits)
        return cls(shard.to_device(path("weight"), device), shard.to_device(path("scales"), device),
                   shard.to_device(path("biases"), device), gs, bits)

    def set_quant(self, group_size: int, bits: int):
        """quant.rs:400-404: re-derive the group size for ``bits``; ``group_size`` is the fallback."""
        self.bits = bits
        g = ops.detect_group_size(self.weight.shape[1], self.scales.shape[1], bits)
        self.group_size = g if g is not None else group_size

    def dims_out(self) -> int:
        return self.weight.shape[0]

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        """[..., K] -> [..., N] (flattened to 2-D for the matmul, quant.rs:306-321)."""
        lead = x.shape[:-1]
        flat = x.reshape(-1, x.shape[-1])
        y = ops.quantized_matmul(flat, self.weight, self.scales, self.biases, True, self.group_size, self.bits)
        return y.reshape(*lead, self.dims_out())

    __call__ = forward

    def forward_serial_rows(self, x: torch.Tensor) -> torch.Tensor:
        """quant.rs:381-394: [B, 1, K] decode rows with the one-row arithmetic."""
        if x.dim() != 3 or x.shape[0] <= 1 or x.shape[1] != 1:
            return self.forward(x)
        return ops.quantized_matmul_serial_rows(x, self.weight, self.scales, self.biases, True, self.group_size,
                                                self.bits)


@dataclass
class QuantizedEmbedding:
    weight: torch.Tensor  # u32 [V, K*bits/32]
    scales: torch.Tensor
    biases: torch.Tensor
    group_size: int = GROUP_SIZE
    bits: int = BITS

    def forward(self, ids: torch.Tensor) -> torch.Tensor:
        """Dequantize the rows of ``ids`` only -> bf16 [..., K] (quant.rs:449-467)."""
        flat = ids.reshape(-1).to(torch.int32).contiguous()
        # gather the packed rows with the library's row gather (u32 rows moved as bf16 pairs)
        w = ops.gather_rows(self.weight.view(torch.bfloat16), flat).view(torch.int32)
        s = ops.gather_rows(self.scales, flat)
        b = ops.gather_rows(self.biases, flat)
        out = ops.dequantize(w, s, b, self.group_size, self.bits)
        return out.reshape(*ids.shape, out.shape[-1])

    def as_linear(self) -> QuantizedLinear:
        """Tied output head: the same packed table as a linear layer."""
        return QuantizedLinear(self.weight, self.scales, self.biases, self.group_size, self.bits)
