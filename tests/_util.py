"""Helpers shared by the tests: tolerance check and host<->device bf16 moves."""
import numpy as np


def assert_close_bf16(got_bits: np.ndarray, ref_f32: np.ndarray, atol=2e-2, rtol=1e-2, what=""):
    """|got - ref| <= atol + rtol*|ref| with got in bf16 and ref the f32 oracle value.

    This is the tolerance the north star states (max-abs 2e-2, relative 1e-2),
    applied per element as a combined bound: a bare 2e-2 bound would fail on a
    single bf16 rounding step wherever |y| > 8 (bf16 ulp 0.0625)."""
    from lisa_amd.synth import bf16_bits_to_f32

    got = bf16_bits_to_f32(got_bits).astype(np.float64)
    ref = ref_f32.astype(np.float64)
    err = np.abs(got - ref)
    bound = atol + rtol * np.abs(ref)
    bad = err > bound
    if bad.any():
        i = np.unravel_index(np.argmax(err - bound), err.shape)
        raise AssertionError(
            f"{what}: {int(bad.sum())}/{bad.size} outside |d| <= {atol} + {rtol}|ref|; worst at {i}: "
            f"got {got[i]:.6g} ref {ref[i]:.6g} (max |d| {err.max():.4g})")


def to_dev_bf16(bits, device):
    import torch

    return torch.from_numpy(np.ascontiguousarray(bits, np.uint16).view(np.int16)).view(torch.bfloat16).to(device)


def to_dev_u32(w, device):
    import torch

    return torch.from_numpy(np.ascontiguousarray(w, np.uint32).view(np.int32)).to(device)


def to_dev(a, device):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).to(device)


def from_dev_bf16(t) -> np.ndarray:
    import torch

    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)
