"""Golden fixtures (tests/golden/fixtures.npz, written by make_golden.py):
the CPU oracle must still reproduce them exactly, and the HIP path through
the C ABI must match them (bit-exact for integer work and dequantize,
north-star tolerance for matmul outputs)."""
import os

import numpy as np
import pytest

from tests._util import assert_close_bf16, from_dev_bf16, to_dev, to_dev_bf16, to_dev_u32

FIX = os.path.join(os.path.dirname(__file__), "golden", "fixtures.npz")
CASES = ["qmv4", "qmv2", "qmv4m3", "qmv4gs32", "qmm4", "qmm2"]


@pytest.fixture(scope="module")
def fx():
    with np.load(FIX, allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def test_oracle_reproduces_fixtures(fx, oracle):
    from lisa_amd.synth import lcg_array

    w = lcg_array(0x2F1D4A73, 64 * 512).reshape(64, 512)
    assert np.array_equal(w, fx["quant2_w"])
    for bits in (2, 4, 8):
        wq, s, b = oracle.quantize_f32(w, 64, bits)
        assert np.array_equal(wq, fx[f"quant{bits}_wq"])
        assert np.array_equal(s, fx[f"quant{bits}_scales"]) and np.array_equal(b, fx[f"quant{bits}_biases"])
        assert np.array_equal(oracle.unpack(fx[f"unpack{bits}_words"], 4 * 32 // bits, bits), fx[f"unpack{bits}_codes"])
    for c in CASES:
        M, N, K, bits, gs = fx[f"{c}_meta"].tolist()
        fn = oracle.qmm if c.startswith("qmm") else oracle.qmv
        y = fn(fx[f"{c}_x"], fx[f"{c}_w"], fx[f"{c}_s"], fx[f"{c}_b"], gs, bits)
        assert np.array_equal(y, fx[f"{c}_y"]), c
    idx, wts = oracle.topk_route(fx["moe_logits"], 2)
    assert np.array_equal(idx, fx["moe_idx"]) and np.array_equal(wts, fx["moe_wts"])
    got = oracle.moe_sort(idx.reshape(-1), 8, 2)
    for g, name in zip(got, ["moe_sorted", "moe_order", "moe_rows", "moe_inv", "moe_offs"]):
        assert np.array_equal(g, fx[name]), name
    assert np.array_equal(oracle.moe_combine(fx["moe_down"], fx["moe_wts"], fx["moe_inv"], 16, 2), fx["moe_comb"])
    assert np.array_equal(oracle.swiglu(fx["swiglu_g"], fx["swiglu_u"]), fx["swiglu_act"])


def test_fixture_codes_follow_layout_law(fx):
    # little-end-first: word 0x76543210 holds codes 0..7 (4-bit)
    assert fx["unpack4_codes"][0, :8].tolist() == list(range(8))
    assert fx["unpack8_codes"][0, :4].tolist() == [0x10, 0x32, 0x54, 0x76]


@pytest.mark.gpu
@pytest.mark.parametrize("case", CASES)
def test_gpu_matches_fixtures(dev, fx, case):
    from lisa_amd import ops

    M, N, K, bits, gs = fx[f"{case}_meta"].tolist()
    x, w, s, b = (to_dev_bf16(fx[f"{case}_x"], dev), to_dev_u32(fx[f"{case}_w"], dev),
                  to_dev_bf16(fx[f"{case}_s"], dev), to_dev_bf16(fx[f"{case}_b"], dev))
    fn = ops.qmm if case.startswith("qmm") else ops.qmv
    assert_close_bf16(from_dev_bf16(fn(x, w, s, b, gs, bits)), fx[f"{case}_y"], what=case)
    assert np.array_equal(from_dev_bf16(ops.dequantize(w, s, b, gs, bits)), fx[f"{case}_deq"])


@pytest.mark.gpu
def test_gpu_moe_fixtures(dev, fx):
    from lisa_amd import ops

    idx, wts = ops.moe_route(to_dev(fx["moe_logits"], dev), 2)
    assert np.array_equal(idx.cpu().numpy(), fx["moe_idx"])
    assert np.allclose(wts.cpu().numpy(), fx["moe_wts"], rtol=2e-6, atol=1e-7)
    got = ops.moe_sort(to_dev(fx["moe_idx"].reshape(-1), dev), 8, 2)
    for g, name in zip(got, ["moe_sorted", "moe_order", "moe_rows", "moe_inv", "moe_offs"]):
        assert np.array_equal(g.cpu().numpy(), fx[name]), name
    comb = ops.moe_combine(to_dev_bf16(fx["moe_down"], dev), to_dev(fx["moe_wts"], dev), to_dev(fx["moe_inv"], dev), 16, 2)
    assert np.array_equal(from_dev_bf16(comb), fx["moe_comb"])
