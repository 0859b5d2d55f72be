"""Writes the small golden fixtures under tests/golden/ from the CPU oracle.

The reference keeps no stored vectors for this path (its tests generate data
in-test with an LCG and assert relations), so these fixtures are produced
by the oracle after it has been pinned by tests/test_oracle.py.  They freeze
the oracle's outputs (so a later change to it is caught) and give the GPU
tests fixed cases.  Inputs use the reference tests' LCG
(crates/lisa-mlx/src/ops/array_ops.rs:658-662) or seeded numpy draws.

Run: python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from lisa_amd.synth import f32_to_bf16_bits, lcg_array, np_linear, np_x  # noqa: E402
from oracle import oracle as O  # noqa: E402


def main():
    O.build()
    out = {}
    # quantize: the reference test's data (K=512, N=64, group 64), bits 2/4/8
    w = lcg_array(0x2F1D4A73, 64 * 512).reshape(64, 512)
    for bits in (2, 4, 8):
        wq, s, b = O.quantize_f32(w, 64, bits)
        out[f"quant{bits}_w"] = w if bits == 2 else np.zeros(0, np.float32)
        out[f"quant{bits}_wq"] = wq
        out[f"quant{bits}_scales"] = s
        out[f"quant{bits}_biases"] = b
    # unpack of fixed words
    words = np.array([[0x76543210, 0xFEDCBA98, 0x12345678, 0x9ABCDEF0]], np.uint32)
    for bits in (2, 4, 8):
        out[f"unpack{bits}_words"] = words
        out[f"unpack{bits}_codes"] = O.unpack(words, 4 * 32 // bits, bits)
    # matvec / matmul cases: (name, M, N, K, bits, gs)
    rng = np.random.default_rng(0x5EED)
    for name, M, N, K, bits, gs in [("qmv4", 1, 64, 1024, 4, 64), ("qmv2", 1, 64, 1024, 2, 64),
                                    ("qmv4m3", 3, 64, 512, 4, 64), ("qmv4gs32", 2, 48, 256, 4, 32),
                                    ("qmm4", 40, 96, 512, 4, 64), ("qmm2", 36, 64, 1024, 2, 128)]:
        wq, s, b = np_linear(rng, N, K, bits, gs, s_std=0.02 if bits == 4 else 0.05,
                             b_std=0.01 if bits == 4 else 0.02)
        x = np_x(rng, M, K)
        fn = O.qmm if name.startswith("qmm") else O.qmv
        y = fn(x, wq, s, b, gs, bits)
        out.update({f"{name}_x": x, f"{name}_w": wq, f"{name}_s": s, f"{name}_b": b,
                    f"{name}_y": y, f"{name}_meta": np.array([M, N, K, bits, gs], np.int64)})
        deq = O.dequantize(wq, s, b, gs, bits)
        out[f"{name}_deq"] = O.f32_to_bf16(deq)
    # MoE routing / sort / combine: T=16 tokens, E=8 experts, k=2
    T, E, k, H = 16, 8, 2, 32
    lg = rng.standard_normal((T, E)).astype(np.float32)
    lg[3, :] = 0.5  # all tied
    idx, wts = O.topk_route(lg, k)
    srt, order, rows, inv, offs = O.moe_sort(idx.reshape(-1), E, k)
    down = f32_to_bf16_bits(rng.standard_normal((T * k, H)).astype(np.float32))
    comb = O.moe_combine(down, wts, inv, T, k)
    g = f32_to_bf16_bits(rng.standard_normal(256).astype(np.float32) * 3)
    u = f32_to_bf16_bits(rng.standard_normal(256).astype(np.float32))
    out.update({"moe_logits": lg, "moe_idx": idx, "moe_wts": wts, "moe_sorted": srt, "moe_order": order,
                "moe_rows": rows, "moe_inv": inv, "moe_offs": offs, "moe_down": down, "moe_comb": comb,
                "swiglu_g": g, "swiglu_u": u, "swiglu_act": O.swiglu(g, u)})
    path = os.path.join(HERE, "fixtures.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path} ({os.path.getsize(path)} bytes, {len(out)} arrays)")


if __name__ == "__main__":
    main()
