"""Seeded synthetic inputs with the distributions of the benchmark configurations.

x ~ N(0,1) bf16; packed codes uniform (uniform random u32 words give uniform
codes in 0..2^bits-1); scales |N(0, s_std)| (+ an optional floor); biases
N(0, b_std).  numpy generators feed the CPU oracle in tests; the torch
generators build large weight sets directly on the GPU for the benchmark.
"""
from __future__ import annotations

import numpy as np


def f32_to_bf16_bits(a: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even f32 -> bf16 bit patterns (uint16)."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def np_linear(rng: np.random.Generator, N: int, K: int, bits: int = 4, gs: int = 64,
              s_std: float = 0.02, b_std: float = 0.01, s_floor: float = 0.0):
    """(w uint32 [N, K*bits/32], scales bf16-bits [N, K/gs], biases bf16-bits [N, K/gs])."""
    w = rng.integers(0, 2**32, size=(N, K * bits // 32), dtype=np.uint64).astype(np.uint32)
    s = np.abs(rng.standard_normal((N, K // gs)).astype(np.float32)) * np.float32(s_std) + np.float32(s_floor)
    b = rng.standard_normal((N, K // gs)).astype(np.float32) * np.float32(b_std)
    return w, f32_to_bf16_bits(s), f32_to_bf16_bits(b)


def np_x(rng: np.random.Generator, M: int, K: int) -> np.ndarray:
    return f32_to_bf16_bits(rng.standard_normal((M, K)).astype(np.float32))


def lcg_stream(seed: int):
    """The reference tests' LCG (array_ops.rs:658-662): values in [-1, 1)."""
    state = seed & (2**64 - 1)
    while True:
        state = (state * 6364136223846793005 + 1) & (2**64 - 1)
        yield float(np.float32(state >> 40) / np.float32(8388608.0)) - 1.0


def lcg_array(seed: int, n: int) -> np.ndarray:
    g = lcg_stream(seed)
    return np.array([next(g) for _ in range(n)], dtype=np.float32)


# ---- torch (device) generators ------------------------------------------------
def torch_linear(N: int, K: int, bits: int = 4, gs: int = 64, s_std: float = 0.02, b_std: float = 0.01,
                 s_floor: float = 0.0, device="cuda", generator=None, experts: int | None = None):
    import torch

    lead = () if experts is None else (experts,)
    w = torch.randint(-(2**31), 2**31, lead + (N, K * bits // 32), dtype=torch.int32, device=device,
                      generator=generator)
    s = (torch.randn(lead + (N, K // gs), device=device, generator=generator).abs() * s_std + s_floor)
    b = torch.randn(lead + (N, K // gs), device=device, generator=generator) * b_std
    return w, s.to(torch.bfloat16), b.to(torch.bfloat16)


def torch_x(M: int, K: int, device="cuda", generator=None):
    import torch

    return torch.randn(M, K, device=device, generator=generator).to(torch.bfloat16)
