"""Routed expert block of the generic MoE path (SwitchGLU of
crates/lisa-engine/src/models/qwen4/moe.rs:12-38, 335-449).

``SwitchGlu.forward(x, logits, top_k)``: top-k routing with softmax over the
selected logits, the stable gather permutation, gate/up gather_qmm, bf16
SwiGLU, down gather_qmm and the sorted combine -- one call into
``lisaq_moe_forward``.  The router logits are an input (the f32 router
matmul and the shared expert are outside this path).
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from . import ops
from .loader import Shard
from .quant import check_layout


@dataclass
class ExpertStack:
    weight: torch.Tensor  # u32 [E, N, K*bits/32]
    scales: torch.Tensor  # bf16 [E, N, K/gs]
    biases: torch.Tensor

    def triple(self):
        return self.weight, self.scales, self.biases


@dataclass
class SwitchGlu:
    gate: ExpertStack  # [E, I, H*bits/32]
    up: ExpertStack
    down: ExpertStack  # [E, H, I*bits/32]
    group_size: int = 64
    bits: int = 4

    @classmethod
    def load(cls, shard: Shard, prefix: str, device="cuda", bits: int = 4):
        """``{prefix}.{gate,up,down}_proj.{weight,scales,biases}`` (moe.rs:25-37)."""
        stacks = {}
        gs = None
        for key in ("gate_proj", "up_proj", "down_proj"):
            names = [f"{prefix}.{key}.{s}" for s in ("weight", "scales", "biases")]
            shapes = [shard.tensors[shard._resolve(n)].shape for n in names]
            E = shapes[0][0]
            flat = [(E * sh[1], sh[2]) for sh in shapes]
            _, g = check_layout(*flat, bits)
            if gs is not None and g != gs:
                raise ValueError(f"{key}: group size {g} differs from {gs}")
            gs = g
            stacks[key] = ExpertStack(*(shard.to_device(n, device) for n in names))
        return cls(stacks["gate_proj"], stacks["up_proj"], stacks["down_proj"], gs, bits)

    def forward(self, x: torch.Tensor, logits: torch.Tensor, top_k: int, return_routing: bool = False):
        """x [..., H] bf16, logits [..., E] f32 -> [..., H] bf16."""
        lead = x.shape[:-1]
        H = x.shape[-1]
        res = ops.moe_forward(x.reshape(-1, H), logits.reshape(-1, logits.shape[-1]), self.gate.triple(),
                              self.up.triple(), self.down.triple(), top_k, self.group_size, self.bits,
                              return_routing=return_routing)
        if return_routing:
            out, idx, wts = res
            return out.reshape(*lead, H), idx, wts
        return res.reshape(*lead, H)

    __call__ = forward
