"""GPU parity of quantized_matmul (matvec and matmul paths), dequantize and
quantize against the CPU oracle, through the C ABI (lisa_amd.ops -> liblisaq).

Tolerance for outputs: |got - ref| <= 2e-2 + 1e-2*|ref| per element (the
north-star bound; see tests/_util.py).  Integer work (codes, quantize output,
dequantize bits) is compared bit-exactly."""
import numpy as np
import pytest

from lisa_amd import ops
from lisa_amd.synth import bf16_bits_to_f32, np_linear, np_x
from tests._util import assert_close_bf16, from_dev_bf16, to_dev, to_dev_bf16, to_dev_u32

pytestmark = pytest.mark.gpu


def _run(fn, dev, x, w, s, b, gs, bits):
    y = fn(to_dev_bf16(x, dev), to_dev_u32(w, dev), to_dev_bf16(s, dev), to_dev_bf16(b, dev),
           group_size=gs, bits=bits)
    return from_dev_bf16(y)


QMV_CASES = [
    # (M, N, K, bits, gs)
    (1, 3072, 1024, 4, 64),      # configs[0]
    (1, 256, 512, 4, 64),
    (3, 64, 512, 4, 64),         # array_ops.rs:650-710 shape
    (1, 100, 512, 4, 64),        # N tail (not a multiple of 32)
    (5, 77, 320, 4, 64),         # K/gs = 5 groups (U = 1 path), N tail
    (1, 9728, 2560, 4, 64),      # configs[1] up
    (2, 9728, 2560, 4, 64),
    (4, 9728, 2560, 4, 64),
    (8, 9728, 2560, 4, 64),
    (1, 2560, 9728, 4, 64),      # configs[1] down
    (2, 2560, 9728, 4, 64),
    (8, 2560, 9728, 4, 64),      # (split over K)
    (4, 2560, 9728, 4, 64),
    (1, 512, 1024, 2, 64),
    (8, 640, 2048, 2, 64),
    (1, 256, 1024, 4, 32),
    (3, 256, 1024, 4, 128),
    (1, 256, 1024, 2, 32),
    (2, 256, 1024, 2, 128),
    (12, 1024, 1024, 4, 64),     # MQ = 2
    (20, 512, 2048, 4, 64),      # MQ = 3
    (32, 512, 1024, 4, 64),      # MQ = 4 (forced qmv)
]


@pytest.mark.parametrize("M,N,K,bits,gs", QMV_CASES)
def test_qmv_parity(dev, oracle, M, N, K, bits, gs):
    rng = np.random.default_rng(M * 7 + N + K + bits + gs)
    w, s, b = np_linear(rng, N, K, bits, gs, s_std=0.02 if bits == 4 else 0.05,
                        b_std=0.01 if bits == 4 else 0.02)
    x = np_x(rng, M, K)
    ref = oracle.qmv(x, w, s, b, gs, bits)
    got = _run(ops.qmv, dev, x, w, s, b, gs, bits)
    assert_close_bf16(got, ref, what=f"qmv M={M} N={N} K={K} bits={bits} gs={gs}")
    if M < ops.qmv_batch_limit(K, N):
        got2 = _run(ops.quantized_matmul, dev, x, w, s, b, gs, bits)
        assert np.array_equal(got, got2)


@pytest.mark.parametrize("kernel", ["w", "p", "s", "d", "t", "16", "32"])
@pytest.mark.parametrize("M,N,K,bits,gs", [
    (1, 100, 1024, 4, 64),      # fewer rows than waves (persistent kernel), J = 1
    (1, 4099, 2560, 4, 64),     # J = 2, N tail
    (1, 17408, 5120, 4, 64),    # north star, J = 3
    (1, 3000, 5120, 2, 64),
    (1, 1000, 4096, 4, 32),
    (1, 1000, 6144, 4, 128),
    (1, 777, 2048, 2, 128),
    (2, 3001, 5120, 4, 64),
    (2, 640, 2048, 2, 64),
    (2, 4097, 2560, 4, 32),     # four rows a step (K = 2560), ragged last step, two rows of x
    (1, 1001, 5120, 4, 128),    # two rows a step (K = 5120), odd N
])
def test_qmv_every_kernel(dev, oracle, force_path, kernel, M, N, K, bits, gs):
    """Each matvec kernel (forced through LISAQ_QMV_KERNEL; a shape it does not
    take falls through to the next one) against the oracle."""
    force_path("LISAQ_QMV_KERNEL", kernel)
    rng = np.random.default_rng(N * 3 + K + bits + gs + M)
    w, s, b = np_linear(rng, N, K, bits, gs, s_std=0.02 if bits == 4 else 0.05,
                        b_std=0.01 if bits == 4 else 0.02)
    x = np_x(rng, M, K)
    ref = oracle.qmv(x, w, s, b, gs, bits)
    got = _run(ops.qmv, dev, x, w, s, b, gs, bits)
    assert_close_bf16(got, ref, what=f"qmv[{kernel}] M={M} N={N} K={K} bits={bits} gs={gs}")


@pytest.mark.parametrize("M,N,K,bits,gs", [
    (33, 256, 512, 4, 64), (64, 256, 1024, 4, 64), (130, 300, 512, 4, 64), (128, 512, 2048, 2, 64),
    (96, 256, 1024, 4, 32), (50, 256, 1024, 4, 128), (200, 1024, 768, 4, 64), (13, 256, 4096, 2, 128),
])
def test_qmm_parity(dev, oracle, M, N, K, bits, gs):
    rng = np.random.default_rng(M + N + K + bits * 3 + gs)
    w, s, b = np_linear(rng, N, K, bits, gs)
    x = np_x(rng, M, K)
    ref = oracle.qmm(x, w, s, b, gs, bits)
    got = _run(ops.qmm, dev, x, w, s, b, gs, bits)
    assert_close_bf16(got, ref, what=f"qmm M={M} N={N} K={K} bits={bits} gs={gs}")
    if M >= ops.qmv_batch_limit(K, N):
        got2 = _run(ops.quantized_matmul, dev, x, w, s, b, gs, bits)
        assert np.array_equal(got, got2)


@pytest.mark.parametrize("split", ["1", "2", "3", "7"])
def test_qmm_split_k(dev, oracle, force_path, split):
    """The matmul split over K (f32 partials in the workspace, summed in split
    order): every split count against the oracle, and the same bits on a repeat."""
    force_path("LISAQ_QMM_SPLIT", split)
    rng = np.random.default_rng(77)
    M, N, K = 70, 300, 1024
    w, s, b = np_linear(rng, N, K, 4, 64)
    x = np_x(rng, M, K)
    ref = oracle.qmm(x, w, s, b, 64, 4)
    got = _run(ops.qmm, dev, x, w, s, b, 64, 4)
    assert_close_bf16(got, ref, what=f"qmm split={split}")
    assert np.array_equal(_run(ops.qmm, dev, x, w, s, b, 64, 4), got)


@pytest.mark.parametrize("M,N,K,bits", [(128, 17408, 5120, 4), (128, 5120, 17408, 4), (512, 17408, 5120, 4),
                                        (512, 5120, 17408, 4), (2048, 17408, 5120, 4), (2048, 5120, 17408, 4),
                                        (512, 17408, 5120, 2), (512, 5120, 17408, 2)])
def test_qmm_prefill_shapes_sampled_rows(dev, oracle, M, N, K, bits):
    """configs[2]/[3] prefill shapes; the oracle checks 8 sampled rows (every column)."""
    import torch

    rng = np.random.default_rng(M + N)
    w, s, b = np_linear(rng, N, K, bits, 64, s_std=0.02 if bits == 4 else 0.05, b_std=0.01 if bits == 4 else 0.02)
    x = np_x(rng, M, K)
    y = ops.quantized_matmul(to_dev_bf16(x, dev), to_dev_u32(w, dev), to_dev_bf16(s, dev), to_dev_bf16(b, dev),
                             group_size=64, bits=bits)
    torch.cuda.synchronize()
    rows = np.sort(rng.choice(M, 8, replace=False))
    rows[0], rows[-1] = 0, M - 1
    ref = oracle.qmm(x[rows], w, s, b, 64, bits)
    got = from_dev_bf16(y)[rows]
    assert_close_bf16(got, ref, what=f"prefill M={M} N={N} K={K}")


@pytest.mark.parametrize("M", [4, 8])
def test_qmv_split_k_and_its_fallback(dev, oracle, force_path, M):
    """Few row tiles (N = 2560): the streaming matvec splits K over workgroups when the workspace holds
    the parts; given none, the same call runs unsplit. Both against the oracle, and close to each other."""
    import torch

    force_path("LISAQ_QMV_KERNEL", "t")

    from lisa_amd import _lib

    N, K, gs, bits = 2560, 9728, 64, 4
    rng = np.random.default_rng(2560 + M)
    w, s, b = np_linear(rng, N, K, bits, gs)
    x = np_x(rng, M, K)
    ref = oracle.qmv(x, w, s, b, gs, bits)
    lib = _lib.load()
    need = lib.lisaq_quantized_matmul_workspace(M, N, K, gs, bits)
    assert need > 0  # the split is on for this shape
    xd, wd, sd, bd = to_dev_bf16(x, dev), to_dev_u32(w, dev), to_dev_bf16(s, dev), to_dev_bf16(b, dev)
    outs = []
    for with_ws in (True, False):
        y = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
        ws = ops.workspace(dev, need) if with_ws else None
        _lib.call("lisaq_quantized_matmul", torch.cuda.current_stream().cuda_stream, xd.data_ptr(), wd.data_ptr(),
                  sd.data_ptr(), bd.data_ptr(), y.data_ptr(), M, N, K, 1, gs, bits,
                  ws.data_ptr() if with_ws else None, need if with_ws else 0)
        got = from_dev_bf16(y)
        assert_close_bf16(got, ref, what=f"qmv M={M} {'split' if with_ws else 'unsplit (no workspace)'}")
        if with_ws:  # parts summed in part order: the same bits on a repeat
            y2 = torch.empty_like(y)
            _lib.call("lisaq_quantized_matmul", torch.cuda.current_stream().cuda_stream, xd.data_ptr(),
                      wd.data_ptr(), sd.data_ptr(), bd.data_ptr(), y2.data_ptr(), M, N, K, 1, gs, bits,
                      ws.data_ptr(), need)
            assert np.array_equal(from_dev_bf16(y2), got)
        outs.append(bf16_bits_to_f32(got))
    # same tolerance between the two as against the oracle (they differ in summation order only)
    assert (np.abs(outs[0] - outs[1]) <= 2e-2 + 1e-2 * np.abs(outs[1])).all()


@pytest.mark.parametrize("bits", [2, 4])
def test_north_star_qmv_shape(dev, oracle, bits):
    rng = np.random.default_rng(17408 + bits)
    N, K = 17408, 5120
    w, s, b = np_linear(rng, N, K, bits, 64, s_std=0.02 if bits == 4 else 0.05, b_std=0.01 if bits == 4 else 0.02)
    for M in (1, 5, 8):  # 5 and 8: two 16-row tiles per workgroup share the staged x
        x = np_x(rng, M, K)
        ref = oracle.qmv(x, w, s, b, 64, bits)
        got = _run(ops.quantized_matmul, dev, x, w, s, b, 64, bits)
        assert_close_bf16(got, ref, what=f"north-star qmv M={M} bits={bits}")
        assert np.array_equal(_run(ops.quantized_matmul, dev, x, w, s, b, 64, bits), got)


@pytest.mark.parametrize("bits", [2, 4])
def test_down_shape_qmv(dev, oracle, bits):
    """configs[3] (2-bit) and configs[2] (4-bit) down shape at decode: N = 5120, K = 17408 (272 groups a
    row), M = 1 over every row, with the config's scale/bias distributions."""
    rng = np.random.default_rng(5120 + bits)
    N, K = 5120, 17408
    w, s, b = np_linear(rng, N, K, bits, 64, s_std=0.02 if bits == 4 else 0.05, b_std=0.01 if bits == 4 else 0.02)
    for M in (1, 4):
        x = np_x(rng, M, K)
        ref = oracle.qmv(x, w, s, b, 64, bits)
        got = _run(ops.quantized_matmul, dev, x, w, s, b, 64, bits)
        assert_close_bf16(got, ref, what=f"down-shape qmv M={M} bits={bits}")


@pytest.mark.parametrize("N,K,gs", [(17408, 5120, 64), (9728, 2560, 64), (2560, 9728, 64), (5120, 17408, 64), (5120, 17408, 128), (1000, 1024, 64),
                                    (777, 2048, 128), (5, 512, 64)])
def test_one_stream_rows_bitwise(dev, oracle, force_path, N, K, gs):
    """The one-stream matvec (1..8 rows of x on one pass over W): every row of an M-row call is bitwise
    equal to the same kernel's one-row call (the matrix-core column of a row never mixes other rows), for
    every M; every row within tolerance of the oracle.  Eight rows at K = 9728 and four at K = 17408
    stage x in two passes over K, eight at K = 17408 in four (all of it does not fit the LDS): bitwise
    equal to the one-pass one-row call as well."""
    force_path("LISAQ_QMV_KERNEL", "w")
    rng = np.random.default_rng(N + K + gs)
    w, s, b = np_linear(rng, N, K, 4, gs)
    x = np_x(rng, 8, K)
    ref = oracle.qmv(x, w, s, b, gs, 4)
    ones = np.concatenate([_run(ops.qmv, dev, x[r:r + 1], w, s, b, gs, 4) for r in range(8)])
    assert_close_bf16(ones, ref, what=f"one-stream M=1 N={N} K={K}")
    for M in range(2, 9):
        got = _run(ops.qmv, dev, x[:M], w, s, b, gs, 4)
        assert_close_bf16(got, ref[:M], what=f"one-stream M={M} N={N} K={K}")
        if _one_stream_fits(M, N, K):
            assert np.array_equal(got, ones[:M]), (N, K, M)


def _one_stream_fits(M, N, K):
    """LDS bytes of the one-stream matvec at its default grid (256 workgroups) within 160 KB, with x
    staged in one pass over K, or (four or eight staged rows) two or four: staged rows of x (each padded by
    256 bytes), block sums, per-unit partials (qmvw.hip, qmvw_lds)."""
    MP = 1 if M == 1 else 2 if M == 2 else 4 if M <= 4 else 8
    RP = min(MP, 4)
    T = (-(-N // 256) + 15) // 16
    segs = K // 512
    for passes in ((1, 2, 4) if MP >= 4 else (1,)):
        KP = -(-segs // passes) * 512
        if MP * (2 * KP + 256) + (K // 64) * MP * 4 + T * segs * 64 * RP * 4 <= 160 * 1024:
            return True
    return False


@pytest.mark.parametrize("bits", [2, 4])
@pytest.mark.parametrize("M", [2, 3, 4, 5, 6, 8])
def test_serial_rows_bitwise_equal_to_single_rows(dev, force_path, bits, M):
    """array_ops.rs:650-710 / jit::affine_verify_qmm (matmul.rs:579-664): batched rows == independent
    M=1 calls, bitwise.  Eight or four rows at a time run on one weight stream (fours where eight rows
    of x do not fit the LDS: K = 9728), the rest in a pair and/or a single row; long rows (K = 17408) in
    pairs; the pair path forced for comparison."""
    rng = np.random.default_rng(99 + bits + 10 * M)
    for N, K in ((64, 512), (2560, 9728), (9728, 2560), (17408, 5120), (1000, 17408), (77, 2048)):
        w, s, b = np_linear(rng, N, K, bits, 64)
        x = np_x(rng, M, K)
        batched = _run(ops.quantized_matmul_serial_rows, dev, x, w, s, b, 64, bits)
        for r in range(M):
            one = _run(ops.quantized_matmul, dev, x[r:r + 1], w, s, b, 64, bits)
            assert np.array_equal(batched[r:r + 1], one), (N, K, M, r)
        force_path("LISAQ_SERIAL_ROWS", "0")
        assert np.array_equal(_run(ops.quantized_matmul_serial_rows, dev, x, w, s, b, 64, bits), batched), (N, K, M)
        force_path("LISAQ_SERIAL_ROWS", None)


def test_repeated_calls_deterministic(dev):
    """Split-K partials are summed in slab order: identical bits every call."""
    rng = np.random.default_rng(5)
    w, s, b = np_linear(rng, 2560, 9728)
    x = np_x(rng, 4, 9728)
    first = _run(ops.quantized_matmul, dev, x, w, s, b, 64, 4)
    for _ in range(3):
        assert np.array_equal(_run(ops.quantized_matmul, dev, x, w, s, b, 64, 4), first)


@pytest.mark.parametrize("bits,gs", [(4, 64), (2, 64), (4, 32), (2, 128), (8, 64)])
def test_dequantize_bit_exact(dev, oracle, bits, gs):
    rng = np.random.default_rng(bits * gs)
    N, K = 300, 1024
    w, s, b = np_linear(rng, N, K, bits, gs)
    got = from_dev_bf16(ops.dequantize(to_dev_u32(w, dev), to_dev_bf16(s, dev), to_dev_bf16(b, dev), gs, bits))
    ref = oracle.f32_to_bf16(oracle.dequantize(w, s, b, gs, bits))
    assert np.array_equal(got, ref)


@pytest.mark.parametrize("bits", [2, 4, 8])
def test_quantize_bit_exact_f32(dev, oracle, bits):
    import torch

    from lisa_amd.synth import lcg_array

    N, K, gs = 64, 512, 64
    wf = lcg_array(0x2F1D4A73, N * K).reshape(N, K)
    wf[0, :64] = 0.0  # all-zero group
    wf[1, :64] = -np.abs(wf[1, :64]) - 0.1  # all-negative group
    wq, sc, bi = ops.quantize(to_dev(wf, dev), gs, bits)
    rq, rs, rb = oracle.quantize_f32(wf, gs, bits)
    assert np.array_equal(wq.cpu().numpy().view(np.uint32), rq)
    assert np.array_equal(sc.cpu().numpy(), rs) and np.array_equal(bi.cpu().numpy(), rb)
    # bf16 input: scales/biases rounded to bf16 like to_dtype(wdt)
    wb = torch.from_numpy(wf).to(torch.bfloat16)
    wbf = wb.float().numpy()
    wq2, sc2, bi2 = ops.quantize(wb.to(dev), gs, bits)
    rq2, rs2, rb2 = oracle.quantize_f32(wbf, gs, bits)
    assert np.array_equal(wq2.cpu().numpy().view(np.uint32), rq2)
    assert np.array_equal(from_dev_bf16(sc2), oracle.f32_to_bf16(rs2))
    assert np.array_equal(from_dev_bf16(bi2), oracle.f32_to_bf16(rb2))


def test_quantize_then_matmul_smoke(dev):
    """smoke.rs:19-40 with our ops: quantize -> quantized_matmul vs dequantize -> matmul (max |d| < 0.1)."""
    import torch

    from lisa_amd.synth import lcg_array

    w = torch.from_numpy(lcg_array(42, 64 * 256).reshape(64, 256)).to(dev)
    x = torch.from_numpy(lcg_array(7, 256).reshape(1, 256)).to(dev).to(torch.bfloat16)
    wq, sc, bi = ops.quantize(w, 32, 4)
    y1 = ops.quantized_matmul(x, wq, sc.to(torch.bfloat16), bi.to(torch.bfloat16), True, 32, 4)
    wd = ops.dequantize(wq, sc.to(torch.bfloat16), bi.to(torch.bfloat16), 32, 4)
    y2 = (x.float() @ wd.float().T)
    assert (y1.float() - y2).abs().max().item() < 0.1


def test_rejections_raise(dev):
    rng = np.random.default_rng(0)
    w, s, b = np_linear(rng, 64, 128)
    x = np_x(rng, 1, 128)
    with pytest.raises(ops.LisaqError, match="biases"):
        ops.quantized_matmul(to_dev_bf16(x, dev), to_dev_u32(w, dev), to_dev_bf16(s, dev), None)
    with pytest.raises(ops.LisaqError, match="transpose"):
        ops.quantized_matmul(to_dev_bf16(x, dev), to_dev_u32(w, dev), to_dev_bf16(s, dev), to_dev_bf16(b, dev),
                             transpose=False)
    import torch
    with pytest.raises(ops.LisaqError, match="dtype"):  # (f16/f32 are supported; f64 is not)
        ops.quantized_matmul(torch.zeros(1, 128, device=dev, dtype=torch.float64), to_dev_u32(w, dev),
                             to_dev_bf16(s, dev), to_dev_bf16(b, dev))


@pytest.mark.parametrize("N,K", [(264, 5120), (1000, 9728), (17408, 5120), (16384, 4608), (5120, 5120)])
def test_qmv_addnorm(dev, oracle, N, K):
    """Residual add + RMSNorm + matvec (jit::affine_qmv_fast_addnorm, matmul.rs:315-443): the sum row
    bit-exact; the normed row within one bf16 step of the oracle (the f32 sum of squares may differ in
    its last bit from the float64 one); y bitwise equal to the matvec on the kernel's own normed row and
    within tolerance of the oracle's matvec on the oracle's normed row.  Every shape here is one launch: the
    persistent matvec (N >= 16384, K <= 6144) or the wave-rows matvec, each with the add + RMSNorm folded in."""
    import torch

    rng = np.random.default_rng(N + K)
    w, s, b = np_linear(rng, N, K, 4, 64)
    x = np_x(rng, 1, K)
    r = np_x(rng, 1, K)
    from lisa_amd.synth import f32_to_bf16_bits
    nw = f32_to_bf16_bits((1.0 + 0.1 * rng.standard_normal(K)).astype(np.float32))
    dw = (to_dev_u32(w, dev), to_dev_bf16(s, dev), to_dev_bf16(b, dev))
    y, sm, nm = ops.qmv_addnorm(to_dev_bf16(x, dev), to_dev_bf16(r, dev), to_dev_bf16(nw, dev), *dw, 1e-6)
    torch.cuda.synchronize()
    s_ref, n_ref = oracle.add_rms_norm(x, r, nw, 1e-6)
    assert np.array_equal(from_dev_bf16(sm), s_ref)
    got_n = bf16_bits_to_f32(from_dev_bf16(nm))
    ref_n = bf16_bits_to_f32(n_ref)
    step = np.abs(ref_n) * 2.0**-7 + 1e-30
    assert (np.abs(got_n - ref_n) <= step).all()
    assert (got_n != ref_n).mean() < 0.01
    chain = from_dev_bf16(ops.quantized_matmul(nm, *dw, True, 64, 4))
    assert np.array_equal(from_dev_bf16(y), chain)
    assert_close_bf16(from_dev_bf16(y), oracle.qmv(n_ref, w, s, b, 64, 4), what=f"qmv_addnorm N={N} K={K}")
    _, _, none = ops.qmv_addnorm(to_dev_bf16(x, dev), to_dev_bf16(r, dev), to_dev_bf16(nw, dev), *dw, 1e-6,
                                 write_norm=False)
    assert none is None


@pytest.mark.parametrize("M,N,K,bits", [(1, 17408, 5120, 4), (2, 17408, 5120, 4), (1, 9728, 2560, 4), (1, 2560, 9728, 4),
                                        (8, 2560, 9728, 4), (1, 17408, 5120, 2)])
def test_null_workspace_when_none_needed(dev, M, N, K, bits):
    """A caller that passes NULL/0 where lisaq_quantized_matmul_workspace() is 0 gets the same bits as
    one that passes a workspace (the header's contract)."""
    import torch

    from lisa_amd import _lib

    lib = _lib.load()
    if lib.lisaq_quantized_matmul_workspace(M, N, K, 64, bits) != 0:
        pytest.skip("this shape uses a workspace")
    rng = np.random.default_rng(N + K + M)
    w, s, b = np_linear(rng, N, K, bits, 64)
    x = np_x(rng, M, K)
    xd, wd, sd, bd = to_dev_bf16(x, dev), to_dev_u32(w, dev), to_dev_bf16(s, dev), to_dev_bf16(b, dev)
    y = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
    _lib.call("lisaq_quantized_matmul", torch.cuda.current_stream().cuda_stream, xd.data_ptr(), wd.data_ptr(),
              sd.data_ptr(), bd.data_ptr(), y.data_ptr(), M, N, K, 1, 64, bits, None, 0)
    ref = ops.quantized_matmul(xd, wd, sd, bd, True, 64, bits)
    assert torch.equal(y.view(torch.int16), ref.view(torch.int16))



@pytest.mark.parametrize("M,N,K,bits", [(1, 17408, 5120, 4), (1, 3000, 5120, 2), (2, 3001, 5120, 4), (1, 9728, 2560, 4),
                                        (2, 640, 2048, 2), (1, 100, 1024, 4), (2, 777, 6144, 4)])
def test_wave_rows_equal_persistent(dev, force_path, M, N, K, bits):
    """The wave-rows matvec and the persistent matvec share the one-row arithmetic (lane l chains the chunks
    l, l+64, ... and the same 64-lane sum): every shape both take gives bitwise equal rows, so
    serial_rows may pair rows in either kernel."""
    rng = np.random.default_rng(N * 5 + K + M + bits)
    w, s, b = np_linear(rng, N, K, bits, 64)
    x = np_x(rng, M, K)
    force_path("LISAQ_QMV_KERNEL", "s")
    got_s = _run(ops.qmv, dev, x, w, s, b, 64, bits)
    force_path("LISAQ_QMV_KERNEL", "p")
    got_p = _run(ops.qmv, dev, x, w, s, b, 64, bits)
    assert np.array_equal(got_s, got_p)


@pytest.mark.parametrize("N,K", [(264, 5120), (2000, 6144)])
def test_addnorm_folded_kernels_agree(dev, force_path, N, K):
    """The add + RMSNorm prologue folded into the wave-rows matvec and into the persistent matvec: the same
    sum row, normed row and outputs bit for bit (same sum-of-squares order, same matvec arithmetic)."""
    import torch

    rng = np.random.default_rng(N + 7 * K)
    w, s, b = np_linear(rng, N, K, 4, 64)
    from lisa_amd.synth import f32_to_bf16_bits
    x, r = np_x(rng, 1, K), np_x(rng, 1, K)
    nw = f32_to_bf16_bits((1.0 + 0.1 * rng.standard_normal(K)).astype(np.float32))
    dw = (to_dev_u32(w, dev), to_dev_bf16(s, dev), to_dev_bf16(b, dev))
    outs = []
    for k in ("s", "p"):
        force_path("LISAQ_QMV_KERNEL", k)
        y, sm, nm = ops.qmv_addnorm(to_dev_bf16(x, dev), to_dev_bf16(r, dev), to_dev_bf16(nw, dev), *dw, 1e-6)
        torch.cuda.synchronize()
        outs.append([from_dev_bf16(t) for t in (y, sm, nm)])
    for a, c in zip(*outs):
        assert np.array_equal(a, c)
