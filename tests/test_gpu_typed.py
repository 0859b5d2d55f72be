"""GPU parity of quantized_matmul for the compute dtypes and code widths
outside the bf16 2/4-bit kernels (lisaq_quantized_matmul_typed): f16 and f32
with 2/4/8-bit codes, bf16 with 8-bit codes, on both sides of the matvec /
matmul split, against the oracle's typed restatements (oracle.qmv_typed,
oracle.qmm_typed).  Tolerances are per output dtype: one rounding of the
output plus f32 summation-order differences."""
import numpy as np
import pytest

from lisa_amd import ops
from lisa_amd.synth import bf16_bits_to_f32, np_linear
from tests._util import to_dev_u32

pytestmark = pytest.mark.gpu

# (atol, rtol) per output dtype
TOL = {"bf16": (2e-2, 1e-2), "f16": (2e-3, 2e-3), "f32": (1e-4, 1e-5)}


def _tensor(a, dtype, dev):
    import torch

    t = torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(dev)
    return t.to({"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}[dtype])


def _close(got, ref, dtype, what):
    atol, rtol = TOL[dtype]
    err = np.abs(got - ref)
    bound = atol + rtol * np.abs(ref)
    assert (err <= bound).all(), f"{what}: {int((err > bound).sum())} outside, max err {err.max():.3g}"


@pytest.mark.parametrize("dtype,bits", [("f16", 2), ("f16", 4), ("f16", 8), ("f32", 2), ("f32", 4), ("f32", 8),
                                        ("bf16", 8)])
@pytest.mark.parametrize("gs", [32, 64, 128])
@pytest.mark.parametrize("M", [1, 5, 40, 130])
def test_quantized_matmul_typed(dev, oracle, dtype, bits, gs, M):
    import torch

    rng = np.random.default_rng(M * 100 + bits * 10 + gs)
    N, K = 200, 384
    w, s, b = np_linear(rng, N, K, bits, gs, s_std=0.02 if bits < 8 else 0.002)
    # values of the compute dtype: round once through it on the host
    sf = oracle._round_to(bf16_bits_to_f32(s), dtype)
    bf = oracle._round_to(bf16_bits_to_f32(b), dtype)
    xf = oracle._round_to(rng.standard_normal((M, K)).astype(np.float32), dtype)
    y = ops.quantized_matmul(_tensor(xf, dtype, dev), to_dev_u32(w, dev), _tensor(sf, dtype, dev),
                             _tensor(bf, dtype, dev), True, gs, bits)
    assert y.dtype == _tensor(xf, dtype, dev).dtype
    got = y.float().cpu().numpy()
    if M < ops.qmv_batch_limit(K, N):
        ref = oracle.qmv_typed(xf, w, sf, bf, gs, bits)
    else:
        ref = oracle.qmm_typed(xf, w, sf, bf, gs, bits, dtype)
    _close(got, ref, dtype, f"{dtype} bits={bits} gs={gs} M={M}")
    torch.cuda.synchronize()


def test_promotion_bf16_x_f32_scales(dev, oracle):
    """x in bf16 with f32 scales/biases computes in f32 (AO:398-404) and
    returns f32."""
    import torch

    rng = np.random.default_rng(3)
    N, K, gs, bits = 64, 256, 64, 4
    w, s, b = np_linear(rng, N, K, bits, gs)
    x = oracle._round_to(rng.standard_normal((2, K)).astype(np.float32), "bf16")
    sf, bf = bf16_bits_to_f32(s), bf16_bits_to_f32(b)
    y = ops.quantized_matmul(_tensor(x, "bf16", dev), to_dev_u32(w, dev), _tensor(sf, "f32", dev),
                             _tensor(bf, "f32", dev), True, gs, bits)
    assert y.dtype == torch.float32
    _close(y.cpu().numpy(), oracle.qmv_typed(x, w, sf, bf, gs, bits), "f32", "promoted")


@pytest.mark.parametrize("dtype", ["f16", "f32"])
@pytest.mark.parametrize("M", [1, 3, 64])
def test_quantized_matmul_typed_long_k(dev, oracle, dtype, M):
    """K = 5120: the matvec's lanes take several 32-code chunks each (K/32 =
    160 chunks over 64 lanes; f16 with three rows: the dot-instruction
    matvec) and the matmul's K loop runs 80 steps over 16 column tiles."""
    import torch

    rng = np.random.default_rng(5120 + M)
    N, K, gs, bits = 1000, 5120, 64, 4
    w, s, b = np_linear(rng, N, K, bits, gs)
    sf = oracle._round_to(bf16_bits_to_f32(s), dtype)
    bf = oracle._round_to(bf16_bits_to_f32(b), dtype)
    xf = oracle._round_to(rng.standard_normal((M, K)).astype(np.float32), dtype)
    y = ops.quantized_matmul(_tensor(xf, dtype, dev), to_dev_u32(w, dev), _tensor(sf, dtype, dev),
                             _tensor(bf, dtype, dev), True, gs, bits)
    got = y.float().cpu().numpy()
    assert (M < ops.qmv_batch_limit(K, N)) == (M < 64)  # both sides of the split
    if M < 64:
        ref = oracle.qmv_typed(xf, w, sf, bf, gs, bits)
    else:
        ref = oracle.qmm_typed(xf, w, sf, bf, gs, bits, dtype)
    _close(got, ref, dtype, f"{dtype} K={K} M={M}")
    torch.cuda.synchronize()


@pytest.mark.parametrize("dtype,bits", [("f16", 4), ("bf16", 8), ("f16", 2)])
def test_quantized_matmul_typed_wide_tiles(dev, oracle, dtype, bits):
    """M, N ragged and large enough for the matrix-core matmul's 128 x 128 tiles (at least 512 of
    them: 16 x 33 here), against the oracle's matmul semantics."""
    import torch

    rng = np.random.default_rng(2000 + bits)
    M, N, K, gs = 2000, 4200, 256, 64
    w, s, b = np_linear(rng, N, K, bits, gs, s_std=0.02 if bits < 8 else 0.002)
    sf = oracle._round_to(bf16_bits_to_f32(s), dtype)
    bf = oracle._round_to(bf16_bits_to_f32(b), dtype)
    xf = oracle._round_to(rng.standard_normal((M, K)).astype(np.float32), dtype)
    y = ops._mm_typed(_tensor(xf, dtype, dev), to_dev_u32(w, dev), _tensor(sf, dtype, dev), _tensor(bf, dtype, dev),
                      True, gs, bits, _tensor(xf[:1], dtype, dev).dtype)
    got = y.float().cpu().numpy()
    _close(got, oracle.qmm_typed(xf, w, sf, bf, gs, bits, dtype), dtype, f"{dtype} bits={bits} wide tiles")
    torch.cuda.synchronize()
