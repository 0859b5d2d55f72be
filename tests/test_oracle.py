"""Pins the CPU oracle (oracle/lisaq_oracle.c) against checks that do not
restate its code: brute-force bit extraction, float64 numpy formulations,
closed forms, textbook library routines (numpy stable argsort) and the
invariants of the reference's own tests.  CPU only."""
import numpy as np
import pytest

from lisa_amd.synth import bf16_bits_to_f32, f32_to_bf16_bits, lcg_array, np_linear, np_x


def np_unpack(w, K, bits):
    """Brute force: one code at a time with Python ints."""
    pack = 32 // bits
    rows = w.shape[0]
    out = np.zeros((rows, K), np.uint8)
    for r in range(rows):
        for k in range(K):
            word = int(w[r, k // pack])
            out[r, k] = (word >> (bits * (k % pack))) & ((1 << bits) - 1)
    return out


@pytest.mark.parametrize("bits", [2, 4, 8])
def test_unpack_brute_force(oracle, bits):
    rng = np.random.default_rng(bits)
    K = 64
    w = rng.integers(0, 2**32, size=(5, K * bits // 32), dtype=np.uint64).astype(np.uint32)
    assert np.array_equal(oracle.unpack(w, K, bits), np_unpack(w, K, bits))


def test_unpack_little_end_first(oracle):
    # code k of a word sits at bits [bits*k, bits*k+bits): 0x76543210 -> 0,1,..,7
    w = np.array([[0x76543210, 0xFEDCBA98]], np.uint32)
    assert oracle.unpack(w, 16, 4).tolist() == [list(range(16))]
    w2 = np.array([[0b11100100 | (0b11100100 << 8) | (0b11100100 << 16) | (0b11100100 << 24)]], np.uint32)
    assert oracle.unpack(w2, 16, 2).tolist() == [[0, 1, 2, 3] * 4]


def bf16_round(a):
    return bf16_bits_to_f32(f32_to_bf16_bits(a))


def test_bf16_rounding_matches_numpy_formulation(oracle):
    rng = np.random.default_rng(0)
    a = rng.standard_normal(10000).astype(np.float32) * 100
    a[:4] = [0.0, -0.0, np.inf, -np.inf]
    # ties: values exactly halfway between two bf16 numbers round to even
    a[4] = np.float32(1.0 + 2**-8)  # halfway between 1 and 1+2^-7 -> 1 (even)
    a[5] = np.float32(1.0 + 3 * 2**-8)  # halfway -> 1+2^-6 (even)
    assert np.array_equal(oracle.f32_to_bf16(a), f32_to_bf16_bits(a))
    assert bf16_round(a[4:5])[0] == 1.0 and bf16_round(a[5:6])[0] == np.float32(1.0 + 2**-6)


# ---- quantize (array_ops.rs:218-290) -----------------------------------------
def deq_f32(wq, s, b, K, bits, gs, oracle):
    codes = oracle.unpack(wq, K, bits).astype(np.float64)
    return codes * np.repeat(s.astype(np.float64), gs, axis=-1) + np.repeat(b.astype(np.float64), gs, axis=-1)


@pytest.mark.parametrize("bits", [2, 4, 8])
def test_quantize_invariants_lcg(oracle, bits):
    # data as in the reference test array_ops.rs:650-710 (LCG, K=512, N=64)
    K, N, gs = 512, 64, 64
    w = lcg_array(0x2F1D4A73, N * K).reshape(N, K)
    wq, s, b = oracle.quantize_f32(w, gs, bits)
    assert wq.shape == (N, K * bits // 32) and s.shape == (N, K // gs)
    codes = oracle.unpack(wq, K, bits)
    maxq = 2**bits - 1
    assert codes.max() <= maxq
    deq = deq_f32(wq, s, b, K, bits, gs, oracle)
    err = np.abs(deq - w)
    srep = np.repeat(np.abs(s).astype(np.float64), gs, axis=-1)
    clipped = codes == maxq
    # unclipped codes are the nearest grid point
    assert (err[~clipped] <= srep[~clipped] * (0.5 + 1e-5)).all()
    # the edge of every group is reproduced exactly (its code is 0, its value the bias)
    for r in range(N):
        for g in range(K // gs):
            grp = w[r, g * gs:(g + 1) * gs]
            side = abs(min(grp.min(), 3.4e38)) > abs(max(grp.max(), 0.0))
            edge = grp.min() if side else max(grp.max(), 0.0)
            if b[r, g] != 0.0:
                assert b[r, g] == np.float32(edge)


def test_quantize_closed_forms(oracle):
    gs, bits = 64, 4
    # all zero -> scale = -1e-7 (flipped eps), bias 0, codes 0
    wq, s, b = oracle.quantize_f32(np.zeros((1, gs), np.float32), gs, bits)
    assert s[0, 0] == np.float32(-1e-7) and b[0, 0] == 0.0 and (wq == 0).all()
    # all negative: w_max is seeded with 0, so max = 0 and min side wins
    grp = -np.linspace(1.0, 2.0, gs, dtype=np.float32)
    wq, s, b = oracle.quantize_f32(grp[None], gs, bits)
    scale0 = np.float32((np.float32(0.0) - np.float32(-2.0)) / np.float32(15.0))
    q0 = np.round(np.float32(-2.0) / scale0)
    assert b[0, 0] == np.float32(-2.0)
    assert s[0, 0] == np.float32(np.float32(-2.0) / np.float32(q0))
    # positive group: max side, negative scale
    grp = np.linspace(1.0, 2.0, gs, dtype=np.float32)
    wq, s, b = oracle.quantize_f32(grp[None], gs, bits)
    assert s[0, 0] < 0 and b[0, 0] == np.float32(2.0)
    codes = oracle.unpack(wq, gs, bits)[0]
    assert codes[-1] == 0  # the edge (2.0) has code 0


def test_quantize_rejects_bad_group(oracle):
    with pytest.raises(ValueError):
        oracle.quantize_f32(np.zeros((1, 96), np.float32), 64, 4)


# ---- dequantize / qmv / qmm ---------------------------------------------------
@pytest.mark.parametrize("bits,gs", [(4, 64), (2, 64), (4, 32), (2, 128), (8, 64)])
def test_dequantize_closed_form(oracle, bits, gs):
    rng = np.random.default_rng(1)
    N, K = 7, 256
    w, s, b = np_linear(rng, N, K, bits, gs)
    got = oracle.dequantize(w, s, b, gs, bits)
    ref = deq_f32(w, bf16_bits_to_f32(s), bf16_bits_to_f32(b), K, bits, gs, oracle)
    assert np.array_equal(got, ref.astype(np.float32))  # s*q is exact, one rounding of the add


def np_matmul_f64(x_bits, w, s, b, gs, bits, oracle, round_w=False):
    K = x_bits.shape[1]
    wd = deq_f32(w, bf16_bits_to_f32(s), bf16_bits_to_f32(b), K, bits, gs, oracle)
    if round_w:
        wd = bf16_round(wd.astype(np.float32)).astype(np.float64)
    return bf16_bits_to_f32(x_bits).astype(np.float64) @ wd.T


@pytest.mark.parametrize("bits,gs", [(4, 64), (2, 64), (4, 32), (4, 128)])
def test_qmv_qmm_vs_float64(oracle, bits, gs):
    rng = np.random.default_rng(2)
    M, N, K = 3, 40, 1024
    w, s, b = np_linear(rng, N, K, bits, gs)
    x = np_x(rng, M, K)
    ref = np_matmul_f64(x, w, s, b, gs, bits, oracle)
    y = oracle.qmv(x, w, s, b, gs, bits)
    assert np.allclose(y, ref, rtol=1e-5, atol=1e-4)
    refr = np_matmul_f64(x, w, s, b, gs, bits, oracle, round_w=True)
    ym = oracle.qmm(x, w, s, b, gs, bits)
    assert np.allclose(ym, refr, rtol=1e-5, atol=1e-4)
    # and the two semantics really differ (qmm rounds the weights)
    assert not np.allclose(y, ym, rtol=0, atol=1e-6)


def test_qmv_closed_forms(oracle):
    rng = np.random.default_rng(3)
    N, K, gs, bits = 4, 256, 64, 4
    _, s, b = np_linear(rng, N, K, bits, gs)
    x = np_x(rng, 1, K)
    xf = bf16_bits_to_f32(x)[0].astype(np.float64)
    sf, bf = bf16_bits_to_f32(s).astype(np.float64), bf16_bits_to_f32(b).astype(np.float64)
    # every code = 9: y = sum_g (9 s_g + b_g) * sum_{k in g} x_k
    w = np.full((N, K // 8), 0x99999999, np.uint32)
    y = oracle.qmv(x, w, s, b, gs, bits)[0]
    xs = xf.reshape(-1, gs).sum(1)
    assert np.allclose(y, (9 * sf + bf) @ xs, rtol=1e-5, atol=1e-5)
    # one-hot x at k=70 (group 1, code 6 of word 8): y = s*q + b exactly
    w = rng.integers(0, 2**32, size=(N, K // 8), dtype=np.uint64).astype(np.uint32)
    xo = f32_to_bf16_bits(np.eye(1, K, 70, dtype=np.float32))
    y = oracle.qmv(xo, w, s, b, gs, bits)[0]
    q = (w[:, 8] >> 24) & 0xF
    assert np.array_equal(y, (q * bf16_bits_to_f32(s)[:, 1] + bf16_bits_to_f32(b)[:, 1]).astype(np.float32))


# ---- MoE routing ----------------------------------------------------------------
def test_topk_route_vs_numpy(oracle):
    rng = np.random.default_rng(4)
    T, E, k = 33, 128, 8
    lg = rng.standard_normal((T, E)).astype(np.float32)
    lg[0, :] = 0.5  # all tied: experts 0..7 in order
    lg[1, [3, 9, 77]] = 5.0  # tie among the top
    idx, wts = oracle.topk_route(lg, k)
    ref = np.argsort(-lg, axis=-1, kind="stable")[:, :k]
    assert np.array_equal(idx, ref)
    assert idx[0].tolist() == list(range(8)) and idx[1, :3].tolist() == [3, 9, 77]
    sel = np.take_along_axis(lg, ref, -1).astype(np.float64)
    e = np.exp(sel - sel.max(-1, keepdims=True))
    assert np.allclose(wts, e / e.sum(-1, keepdims=True), rtol=1e-6, atol=1e-7)


@pytest.mark.parametrize("R,E,k", [(8, 128, 8), (1000, 16, 4), (4096 * 8, 128, 8), (7, 1, 1)])
def test_moe_sort_vs_numpy(oracle, R, E, k):
    rng = np.random.default_rng(R)
    ids = rng.integers(0, E, R).astype(np.int32)
    srt, order, rows, inv, offs = oracle.moe_sort(ids, E, k)
    ref_order = np.argsort(ids, kind="stable")
    assert np.array_equal(order, ref_order)
    assert np.array_equal(srt, ids[ref_order])
    assert np.array_equal(rows, ref_order // k)
    assert np.array_equal(inv, np.argsort(ref_order, kind="stable"))
    assert np.array_equal(order[inv], np.arange(R))  # inverse permutation
    assert np.array_equal(offs, np.concatenate([[0], np.cumsum(np.bincount(ids, minlength=E))]))
    assert (np.diff(srt) >= 0).all()


def test_moe_sort_rejects_out_of_range(oracle):
    with pytest.raises(ValueError):
        oracle.moe_sort(np.array([0, 5], np.int32), 4, 1)


def test_swiglu_float64(oracle):
    rng = np.random.default_rng(5)
    g = f32_to_bf16_bits(rng.standard_normal(5000).astype(np.float32) * 4)
    u = f32_to_bf16_bits(rng.standard_normal(5000).astype(np.float32))
    got = bf16_bits_to_f32(oracle.swiglu(g, u)).astype(np.float64)
    gf, uf = bf16_bits_to_f32(g).astype(np.float64), bf16_bits_to_f32(u).astype(np.float64)
    ref = gf / (1 + np.exp(-gf)) * uf
    # three bf16 roundings in the chain: within 4 bf16 ulps (2^-6 relative)
    assert np.all(np.abs(got - ref) <= 2**-6 * np.abs(ref) + 1e-30)


@pytest.mark.parametrize("k", [1, 2, 8, 10, 16])
def test_moe_combine_chain_order(oracle, k):
    rng = np.random.default_rng(k)
    T, H = 5, 33
    R = T * k
    down = f32_to_bf16_bits(rng.standard_normal((R, H)).astype(np.float32))
    w = rng.random(R).astype(np.float32)
    inv = rng.permutation(R).astype(np.int32)
    got = oracle.moe_combine(down, w, inv, T, k)
    d = bf16_bits_to_f32(down)
    TY = min(k, 8)
    ref = np.zeros((T, H), np.float32)
    for t in range(T):
        prod = [d[inv[t * k + j]] * w[t * k + j] for j in range(k)]  # f32 products
        parts = []
        for y in range(TY):
            acc = np.zeros(H, np.float32)
            for rr in range(y, k, TY):
                acc = (prod[rr] + acc).astype(np.float32)
            parts.append(acc)
        tot = parts[0]
        for j in range(1, TY):
            tot = (parts[j] + tot).astype(np.float32)
        ref[t] = tot
    assert np.array_equal(got, f32_to_bf16_bits(ref))


def test_moe_combine_known_answer(oracle):
    """colsum_small<K> (exact_header.metal:12-24) by hand, k = 10 (8 partial sums; slots 8 and 9 join
    partials 0 and 1), weights 1: products p0 = 2^24, p1 = -2^24, p8 = p9 = 1, the rest 0.
    t0 = p8 + (p0 + 0) = 1 + 2^24 -> 2^24 (f32 tie to even); t1 = p9 + (p1 + 0) = -16777215 (exact);
    total = t1 + t0 = 1, then + 0 six times: 1.0.  Summing the slots in order gives 2.0, summing the
    partials the other way round also 1.0 but t0 first absorbing p8 is what loses the 1."""
    k, T, H = 10, 1, 2
    vals = np.zeros((k, H), np.float32)
    vals[0, 0], vals[1, 0], vals[8, 0], vals[9, 0] = 2.0**24, -(2.0**24), 1.0, 1.0
    vals[:, 1] = 0.5  # ten halves: 5.0 in any order
    down = f32_to_bf16_bits(vals)
    w = np.ones(k, np.float32)
    inv = np.arange(k, dtype=np.int32)
    got = bf16_bits_to_f32(oracle.moe_combine(down, w, inv, T, k))
    assert got.tolist() == [[1.0, 5.0]]
    assert float(np.float32(sum(np.float32(v) for v in vals[:, 0]))) == 2.0  # the slot-order sum differs


def test_qmv_threads_matches_single(oracle):
    rng = np.random.default_rng(6)
    N, K = 300, 512
    w, s, b = np_linear(rng, N, K)
    x = np_x(rng, 2, K)
    assert np.array_equal(oracle.qmv_threads(x, w, s, b, 64, 4, 7), oracle.qmv(x, w, s, b, 64, 4))


def test_add_rms_norm_known_answer(oracle):
    """norm_qmv.metal:383-400 by hand: s alternating 3, 4 (mean square 12.5, eps 0), norm weight 1.5.
    3/sqrt(12.5) = 0.84853 rounds to bf16 0.84765625, times 1.5 = 1.271484375 -> 1.2734375;
    4/sqrt(12.5) = 1.13137 rounds to 1.1328125, times 1.5 = 1.69921875, a tie -> 1.703125 (even).
    Without the inner rounding the 4 would give 1.6953125: the double rounding is pinned."""
    K = 8
    x = f32_to_bf16_bits(np.array([[1, 3] * (K // 2)], np.float32))
    r = f32_to_bf16_bits(np.array([[2, 1] * (K // 2)], np.float32))
    nw = f32_to_bf16_bits(np.full(K, 1.5, np.float32))
    s, normed = oracle.add_rms_norm(x, r, nw, 0.0)
    assert np.array_equal(bf16_bits_to_f32(s), np.array([[3, 4] * (K // 2)], np.float32))
    assert np.array_equal(bf16_bits_to_f32(normed), np.array([[1.2734375, 1.703125] * (K // 2)], np.float32))
    # eps enters the mean: a zero row gives zeros, not NaN
    s0, n0 = oracle.add_rms_norm(np.zeros((1, K), np.uint16), np.zeros((1, K), np.uint16), nw, 1e-6)
    assert not np.isnan(bf16_bits_to_f32(n0)).any() and (bf16_bits_to_f32(n0) == 0).all()


def test_add_rms_norm_unit_rms(oracle):
    """With unit norm weight the normed row has mean square ~1 (float64 check of the formula's scale)."""
    rng = np.random.default_rng(4)
    x = np_x(rng, 3, 6144)
    r = np_x(rng, 3, 6144)
    nw = f32_to_bf16_bits(np.ones(6144, np.float32))
    _, normed = oracle.add_rms_norm(x, r, nw, 1e-6)
    ms = (bf16_bits_to_f32(normed).astype(np.float64) ** 2).mean(axis=-1)
    assert np.allclose(ms, 1.0, atol=1e-2)


# ---- the typed (any dtype, 2/4/8-bit) restatements ----------------------------

@pytest.mark.parametrize("bits", [2, 4])
def test_typed_restatements_match_the_bf16_oracle(oracle, bits):
    """On bf16 values the typed numpy restatements agree with the C oracle's
    qmv and qmm (f32 sums there, float64 here: agreement to f32 precision)."""
    rng = np.random.default_rng(40 + bits)
    M, N, K, gs = 3, 17, 256, 64
    w, s, b = np_linear(rng, N, K, bits, gs)
    x = np_x(rng, M, K)
    xf, sf, bf = (bf16_bits_to_f32(a) for a in (x, s, b))
    mv = oracle.qmv_typed(xf, w, sf, bf, gs, bits)
    mm = oracle.qmm_typed(xf, w, sf, bf, gs, bits, "bf16")
    scale = np.abs(mv).max()
    assert np.abs(mv - oracle.qmv(x, w, s, b, gs, bits)).max() <= 1e-5 * scale
    assert np.abs(mm - oracle.qmm(x, w, s, b, gs, bits)).max() <= 1e-5 * scale


@pytest.mark.parametrize("dtype", ["bf16", "f16", "f32"])
def test_typed_closed_form_constant_codes(oracle, dtype):
    """8-bit codes all equal to c and x all ones: every weight of group g is
    s_g*c + b_g, so y = sum_g gs * (s_g*c + b_g) (matvec, exact weights) and
    y = sum_g gs * T(s_g*c + b_g) (matmul, weights rounded to T)."""
    gs, K, N, c = 32, 128, 3, 201
    word = c | (c << 8) | (c << 16) | (c << 24)
    w = np.full((N, K // 4), word, np.uint32)
    rng = np.random.default_rng(7)
    s = rng.uniform(0.001, 0.01, (N, K // gs)).astype(np.float32)
    b = rng.uniform(-0.5, 0.5, (N, K // gs)).astype(np.float32)
    x = np.ones((2, K), np.float32)
    exact = (gs * (s.astype(np.float64) * c + b)).sum(1)
    assert np.allclose(oracle.qmv_typed(x, w, s, b, gs, 8), exact[None], rtol=1e-12)
    wt = oracle._round_to((s.astype(np.float64) * c + b).astype(np.float32), dtype).astype(np.float64)
    assert np.allclose(oracle.qmm_typed(x, w, s, b, gs, 8, dtype), (gs * wt).sum(1)[None], rtol=1e-12)
    if dtype != "f32":  # the rounding to T is really applied
        assert not np.allclose(wt, s * c + b, rtol=1e-7, atol=0)
