"""GPU parity of the MoE path (route, sort, gather, gather_qmm, SwiGLU,
combine, whole routed SwitchGLU) against the CPU oracle through the C ABI.
Routing indices, sort permutation, token rows and inverse are bit-exact; the
combine is bit-exact for identical inputs; matmul outputs use the north-star
tolerance."""
import numpy as np
import pytest

from lisa_amd import ops
from lisa_amd.synth import bf16_bits_to_f32, f32_to_bf16_bits, np_linear, np_x
from tests._util import assert_close_bf16, from_dev_bf16, to_dev, to_dev_bf16, to_dev_u32

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("T,E,k", [(1, 128, 8), (4096, 128, 8), (37, 64, 4), (5, 512, 10), (3, 1024, 32)])
def test_route_bit_exact(dev, oracle, T, E, k):
    rng = np.random.default_rng(T + E)
    lg = rng.standard_normal((T, E)).astype(np.float32)
    if T > 2:
        lg[0, :] = 0.25  # fully tied row
        lg[1, 5:40] = lg[1].max() + 1  # ties at the top
    idx, wts = ops.moe_route(to_dev(lg, dev), k)
    ridx, rw = oracle.topk_route(lg, k)
    assert np.array_equal(idx.cpu().numpy(), ridx)
    assert np.allclose(wts.cpu().numpy(), rw, rtol=2e-6, atol=1e-7)


@pytest.mark.parametrize("R,E,k", [(8, 128, 8), (32768, 128, 8), (1000, 16, 4), (5, 1, 1), (4099, 1024, 3)])
def test_sort_bit_exact(dev, oracle, R, E, k):
    rng = np.random.default_rng(R)
    ids = rng.integers(0, E, R).astype(np.int32)
    got = ops.moe_sort(to_dev(ids, dev), E, k)
    ref = oracle.moe_sort(ids, E, k)
    for g, r, name in zip(got, ref, ["sorted_idx", "order", "token_rows", "inverse", "offsets"]):
        assert np.array_equal(g.cpu().numpy(), r), name


def test_gather_rows_and_swiglu(dev, oracle):
    rng = np.random.default_rng(3)
    x = np_x(rng, 50, 2048)
    rows = rng.integers(0, 50, 400).astype(np.int32)
    got = from_dev_bf16(ops.gather_rows(to_dev_bf16(x, dev), to_dev(rows, dev)))
    assert np.array_equal(got, x[rows])
    g = f32_to_bf16_bits(rng.standard_normal(10000).astype(np.float32) * 3)
    u = f32_to_bf16_bits(rng.standard_normal(10000).astype(np.float32))
    act = from_dev_bf16(ops.swiglu(to_dev_bf16(g, dev), to_dev_bf16(u, dev)))
    ref = oracle.swiglu(g, u)
    # exp differs in the last ulp between libm and the device: allow one bf16 ulp
    diff = np.abs(act.astype(np.int32) - ref.astype(np.int32))
    assert diff.max() <= 1 and (diff == 0).mean() > 0.99


@pytest.mark.parametrize("T,k,H", [(1, 8, 2048), (4096, 8, 2048), (9, 10, 100), (3, 16, 64)])
def test_combine_bit_exact(dev, oracle, T, k, H):
    rng = np.random.default_rng(T * k)
    R = T * k
    down = f32_to_bf16_bits(rng.standard_normal((R, H)).astype(np.float32))
    w = rng.random(R).astype(np.float32)
    inv = rng.permutation(R).astype(np.int32)
    got = from_dev_bf16(ops.moe_combine(to_dev_bf16(down, dev), to_dev(w, dev), to_dev(inv, dev), T, k))
    assert np.array_equal(got, oracle.moe_combine(down, w, inv, T, k))


def test_combine_known_answer(dev):
    """The combine's association on the GPU (the case of the oracle's known-answer test, H = 8 for the
    vector kernel and H = 3 for the scalar one): slots 8 and 9 fold into partials 0 and 1, so
    2^24 - 2^24 + 1 + 1 over ten slots gives 1.0, not the slot-order 2.0."""
    k = 10
    for H in (8, 3):
        vals = np.zeros((k, H), np.float32)
        vals[0, :], vals[1, :], vals[8, :], vals[9, :] = 2.0**24, -(2.0**24), 1.0, 1.0
        got = ops.moe_combine(to_dev_bf16(f32_to_bf16_bits(vals), dev), to_dev(np.ones(k, np.float32), dev),
                              to_dev(np.arange(k, dtype=np.int32), dev), 1, k)
        assert np.array_equal(bf16_bits_to_f32(from_dev_bf16(got)), np.ones((1, H), np.float32)), H


def _expert_stack(rng, E, N, K, bits=4):
    ws, ss, bs = [], [], []
    for _ in range(E):
        w, s, b = np_linear(rng, N, K, bits, 64)
        ws.append(w), ss.append(s), bs.append(b)
    return np.stack(ws), np.stack(ss), np.stack(bs)


def _gather_ref(oracle, x, W, S, B, ids, limit):
    """The reference's non-NAX gather (array_ops.rs:591-630): per contiguous run
    of one expert, quantized_matmul of the run (matvec math below the batch
    limit, matmul math above)."""
    R = x.shape[0]
    out = np.zeros((R, W.shape[1]), np.float32)
    s = 0
    while s < R:
        e = s + 1
        while e < R and ids[e] == ids[s]:
            e += 1
        fn = oracle.qmv if (e - s) < limit else oracle.qmm
        out[s:e] = fn(x[s:e], W[ids[s]], S[ids[s]], B[ids[s]], 64, 4)
        s = e
    return out


@pytest.mark.parametrize("R,E,N,K", [(8, 16, 768, 2048), (300, 8, 256, 512), (64, 4, 2048, 768),
                                     (1000, 32, 160, 256)])
def test_gather_qmm_parity(dev, oracle, R, E, N, K):
    rng = np.random.default_rng(R + E)
    W, S, B = _expert_stack(rng, E, N, K)
    ids = np.sort(rng.integers(0, E, R)).astype(np.int32)
    if R >= 300:
        ids[: R // 3] = ids[0]  # one long run (matmul path) among short ones
        ids = np.sort(ids)
    x = np_x(rng, R, K)
    y = ops.gather_qmm(to_dev_bf16(x, dev), to_dev_u32(W, dev), to_dev_bf16(S, dev), to_dev_bf16(B, dev),
                       rhs_indices=to_dev(ids, dev), group_size=64, bits=4)
    ref = _gather_ref(oracle, x, W, S, B, ids, ops.qmv_batch_limit(K, N))
    assert_close_bf16(from_dev_bf16(y), ref, what=f"gather R={R} E={E} N={N} K={K}")


@pytest.mark.parametrize("kernel", ["d", "t"])
@pytest.mark.parametrize("R,E,N,K", [(1, 4, 768, 2048), (2, 4, 768, 2048), (2, 2, 2048, 768), (2, 1, 300, 512)])
def test_gather_qmm_short_runs(dev, oracle, force_path, kernel, R, E, N, K):
    """Runs of one or two rows (decode MoE) through each tile-capable matvec
    kernel (forced with LISAQ_QMV_KERNEL)."""
    force_path("LISAQ_QMV_KERNEL", kernel)
    rng = np.random.default_rng(R * 11 + E + N)
    W, S, B = _expert_stack(rng, E, N, K)
    ids = np.sort(rng.integers(0, E, R)).astype(np.int32)
    x = np_x(rng, R, K)
    y = ops.gather_qmm(to_dev_bf16(x, dev), to_dev_u32(W, dev), to_dev_bf16(S, dev), to_dev_bf16(B, dev),
                       rhs_indices=to_dev(ids, dev), group_size=64, bits=4)
    ref = _gather_ref(oracle, x, W, S, B, ids, ops.qmv_batch_limit(K, N))
    assert_close_bf16(from_dev_bf16(y), ref, what=f"gather[{kernel}] R={R} E={E} N={N} K={K}")


@pytest.mark.parametrize("kernel", [None, "t"])
def test_gather_qmm_walking_grid(dev, oracle, force_path, kernel):
    """Long runs with a dozen short ones among them: R >= 4 x the matvec limit x E, so the matvec's
    tile-table launch is a short grid whose blocks walk the table (1,536 matvec tiles over 1,024
    blocks: some blocks take two)."""
    if kernel:
        force_path("LISAQ_QMV_KERNEL", kernel)
    E, N, K = 16, 2048, 512
    limit = ops.qmv_batch_limit(K, N)
    rng = np.random.default_rng(2024)
    W, S, B = _expert_stack(rng, E, N, K)
    lens = [int(v) for v in rng.integers(1, limit, 12)] + [600, 700, 650, 555]
    assert sum(lens) >= 4 * limit * E
    ids = np.concatenate([np.full(n, e, np.int32) for e, n in enumerate(lens)])
    x = np_x(rng, ids.size, K)
    y = ops.gather_qmm(to_dev_bf16(x, dev), to_dev_u32(W, dev), to_dev_bf16(S, dev), to_dev_bf16(B, dev),
                       rhs_indices=to_dev(ids, dev), group_size=64, bits=4)
    ref = _gather_ref(oracle, x, W, S, B, ids, limit)
    assert_close_bf16(from_dev_bf16(y), ref, what=f"gather walking grid [{kernel}]")


@pytest.mark.parametrize("N,K", [(768, 2048), (2048, 768)])
def test_gather_qmm_folded_runs(dev, oracle, N, K):
    """Short runs on average (4 rows here: the tile tables use the 8-row matvec class and put longer
    runs below the limit in pieces of 8 rows into it, with no launch for a longer class) with runs of
    17, 25 and 32 rows among them, and one run at the matvec limit (matmul arithmetic)."""
    E = 40
    limit = ops.qmv_batch_limit(K, N)
    rng = np.random.default_rng(N + K)
    W, S, B = _expert_stack(rng, E, N, K)
    lens = [int(v) for v in rng.integers(1, 4, E - 4)] + [17, 25, 32, limit]
    assert sum(lens) <= 8 * E and max(lens[:-1]) < limit
    ids = np.concatenate([np.full(n, e, np.int32) for e, n in enumerate(lens)])
    x = np_x(rng, ids.size, K)
    y = ops.gather_qmm(to_dev_bf16(x, dev), to_dev_u32(W, dev), to_dev_bf16(S, dev), to_dev_bf16(B, dev),
                       rhs_indices=to_dev(ids, dev), group_size=64, bits=4)
    ref = _gather_ref(oracle, x, W, S, B, ids, limit)
    assert_close_bf16(from_dev_bf16(y), ref, what=f"gather folded runs N={N} K={K}")


@pytest.mark.parametrize("T", [1, 4, 64])
def test_moe_forward_parity(dev, oracle, T):
    """Whole routed SwitchGLU vs the oracle chain, with the reference shapes
    (E=128, k=8, H=2048, I=768).  Routing is compared bit-exactly; the down
    projection input is taken from the device's own SwiGLU output so the
    combine step can be checked on identical inputs."""
    rng = np.random.default_rng(T)
    E, k, H, I = 128, 8, 2048, 768
    G = _expert_stack(rng, E, I, H)
    U = _expert_stack(rng, E, I, H)
    D = _expert_stack(rng, E, H, I)
    x = np_x(rng, T, H)
    lg = rng.standard_normal((T, E)).astype(np.float32)
    dv = [tuple(to_dev_u32(a, dev) if i == 0 else to_dev_bf16(a, dev) for i, a in enumerate(st)) for st in (G, U, D)]
    out, idx, wts = ops.moe_forward(to_dev_bf16(x, dev), to_dev(lg, dev), dv[0], dv[1], dv[2], k,
                                    return_routing=True)
    ridx, rw = oracle.topk_route(lg, k)
    assert np.array_equal(idx.cpu().numpy(), ridx)
    srt, order, rows, inv, offs = oracle.moe_sort(ridx.reshape(-1), E, k)
    xs = x[rows]
    lim_gu = ops.qmv_batch_limit(H, I)
    g = _gather_ref(oracle, xs, *G, srt, lim_gu)
    u = _gather_ref(oracle, xs, *U, srt, lim_gu)
    # device pieces for the later stages (inputs identical to the oracle's)
    import torch

    xs_d = to_dev_bf16(xs, dev)
    sid = to_dev(srt, dev)
    gd = ops.gather_qmm(xs_d, *dv[0], rhs_indices=sid)
    ud = ops.gather_qmm(xs_d, *dv[1], rhs_indices=sid)
    assert_close_bf16(from_dev_bf16(gd), g, what="gate")
    assert_close_bf16(from_dev_bf16(ud), u, what="up")
    act = ops.swiglu(gd, ud)
    dd = ops.gather_qmm(act, *dv[2], rhs_indices=sid)
    dref = _gather_ref(oracle, from_dev_bf16(act), *D, srt, ops.qmv_batch_limit(I, H))
    assert_close_bf16(from_dev_bf16(dd), dref, what="down")
    comb = ops.moe_combine(dd, wts.reshape(-1), to_dev(inv, dev), T, k)
    # the fused entry point may pick other matvec kernels (it knows that a run
    # is at most T rows): same result within the output tolerance
    from lisa_amd.synth import bf16_bits_to_f32

    assert_close_bf16(from_dev_bf16(out), bf16_bits_to_f32(from_dev_bf16(comb)), what="moe_forward vs step by step")
    assert np.array_equal(from_dev_bf16(comb), oracle.moe_combine(from_dev_bf16(dd), wts.cpu().numpy(), inv, T, k))
    torch.cuda.synchronize()


@pytest.mark.parametrize("T,E,k,H,I,bits,gs,skew", [(16, 128, 8, 2048, 768, 4, 64, False),
                                                    (64, 128, 8, 2048, 768, 4, 64, False),
                                                    (64, 128, 8, 2048, 768, 4, 64, True),
                                                    (200, 128, 8, 2048, 768, 4, 64, True),
                                                    (40, 16, 2, 512, 320, 2, 64, True),
                                                    (9, 8, 3, 256, 256, 4, 128, False),
                                                    (24, 16, 4, 256, 192, 4, 32, True)])
def test_moe_forward_gate_up_matvec(dev, force_path, T, E, k, H, I, bits, gs, skew):
    """Between the decode window and the gate|up matmul path (9 <= T, T*k < 20E): gate|up + SwiGLU in
    the gate|up streaming matvec (and the gate|up matmul for runs at or above the matvec limit; skewed
    routing makes such runs), x read through the row map -- bitwise equal to the same block with gate,
    up and SwiGLU as separate launches over gathered rows (LISAQ_MOE_GU_MV=0)."""
    import torch

    rng = np.random.default_rng(T * 7 + E + bits)
    st = lambda n, kk: tuple(a.reshape(E, n, -1) for a in np_linear(rng, E * n, kk, bits, gs))
    G, U, D = st(I, H), st(I, H), st(H, I)
    x = np_x(rng, T, H)
    lg = rng.standard_normal((T, E)).astype(np.float32)
    if skew:  # a few experts picked by most tokens: runs of up to T rows
        lg[:, :3] += 4.0
    dv = [tuple(to_dev_u32(a, dev) if i == 0 else to_dev_bf16(a, dev) for i, a in enumerate(s_)) for s_ in (G, U, D)]
    xd, lgd = to_dev_bf16(x, dev), to_dev(lg, dev)
    fused = from_dev_bf16(ops.moe_forward(xd, lgd, dv[0], dv[1], dv[2], k, group_size=gs, bits=bits))
    force_path("LISAQ_MOE_GU_MV", "0")
    steps = from_dev_bf16(ops.moe_forward(xd, lgd, dv[0], dv[1], dv[2], k, group_size=gs, bits=bits))
    torch.cuda.synchronize()
    assert np.array_equal(fused, steps)


def _run_ref(oracle, xr, W, S, B, e, limit):
    """One run of expert e as the reference's per-run loop computes it (array_ops.rs:591-630)."""
    fn = oracle.qmv if xr.shape[0] < limit else oracle.qmm
    return fn(xr, W[e], S[e], B[e], 64, 4)


def test_moe_forward_baseline_shape(dev, oracle):
    """BASELINE configs[4] at T=4096 (E=128, k=8, H=2048, I=768; 32768 routed rows, ~256-row expert runs
    through the matmul tiles): routing bit-exact; the gate, up and down gather_qmm of four sampled experts'
    whole runs (all columns) against the per-run oracle; moe_forward bitwise equal to its steps composed
    from the public entry points; 64 sampled tokens of the combine bit-exact against the oracle's combine."""
    import torch

    rng = np.random.default_rng(4096)
    T, E, k, H, I = 4096, 128, 8, 2048, 768
    G, U, D = _expert_stack(rng, E, I, H), _expert_stack(rng, E, I, H), _expert_stack(rng, E, H, I)
    x = np_x(rng, T, H)
    lg = rng.standard_normal((T, E)).astype(np.float32)
    dv = [tuple(to_dev_u32(a, dev) if i == 0 else to_dev_bf16(a, dev) for i, a in enumerate(st)) for st in (G, U, D)]
    xd, lgd = to_dev_bf16(x, dev), to_dev(lg, dev)
    out, idx, wts = ops.moe_forward(xd, lgd, dv[0], dv[1], dv[2], k, return_routing=True)
    ridx, rw = oracle.topk_route(lg, k)
    assert np.array_equal(idx.cpu().numpy(), ridx)
    assert np.allclose(wts.cpu().numpy(), rw, rtol=2e-6, atol=1e-7)
    srt, order, rows, inv, offs = oracle.moe_sort(ridx.reshape(-1), E, k)
    # device pieces (public entry points) on the same sorted rows
    sid = to_dev(srt, dev)
    xs_d = ops.gather_rows(xd, to_dev(rows, dev))
    gd = ops.gather_qmm(xs_d, *dv[0], rhs_indices=sid)
    ud = ops.gather_qmm(xs_d, *dv[1], rhs_indices=sid)
    act = ops.swiglu(gd, ud)
    dd = ops.gather_qmm(act, *dv[2], rhs_indices=sid)
    comb = ops.moe_combine(dd, wts.reshape(-1), to_dev(inv, dev), T, k)
    assert torch.equal(out.view(torch.int16), comb.view(torch.int16))
    xs, g_h, u_h, a_h, d_h = (from_dev_bf16(t) for t in (xs_d, gd, ud, act, dd))
    assert np.array_equal(xs, x[rows])
    lim_gu, lim_d = ops.qmv_batch_limit(H, I), ops.qmv_batch_limit(I, H)
    sizes = np.diff(offs)
    picks = [int(np.argmax(sizes)), int(np.argmin(np.where(sizes > 0, sizes, 1 << 30))), 0, E - 1]
    for e in picks:
        a, b = offs[e], offs[e + 1]
        if a == b:
            continue
        assert_close_bf16(g_h[a:b], _run_ref(oracle, xs[a:b], *G, e, lim_gu), what=f"gate expert {e} ({b - a} rows)")
        assert_close_bf16(u_h[a:b], _run_ref(oracle, xs[a:b], *U, e, lim_gu), what=f"up expert {e}")
        assert_close_bf16(d_h[a:b], _run_ref(oracle, a_h[a:b], *D, e, lim_d), what=f"down expert {e}")
    tok = np.sort(rng.choice(T, 64, replace=False))
    ref = oracle.moe_combine(d_h, wts.cpu().numpy(), inv, T, k)
    assert np.array_equal(from_dev_bf16(out)[tok], ref[tok])


@pytest.mark.parametrize("T,E,k,H,I,bits,gs", [(1, 128, 8, 2048, 768, 4, 64), (3, 16, 4, 512, 256, 4, 32),
                                             (8, 32, 2, 1024, 384, 4, 128), (2, 64, 8, 256, 768, 2, 64),
                                             (5, 32, 16, 128, 1024, 2, 128), (1, 4, 1, 4096, 64, 4, 64)])
def test_moe_fused_decode_vs_generic(dev, force_path, T, E, k, H, I, bits, gs):
    """The fused decode path (T <= 8: gate|up+SwiGLU and down+combine kernels)
    against the generic path (sort, gather_qmm, SwiGLU, combine) on the same
    inputs: identical routing, outputs within the output tolerance (the two
    differ only in the order of the matvec sums)."""
    from lisa_amd import _lib

    rng = np.random.default_rng(T * 1000 + k)
    stk = lambda n, kk: tuple(a.reshape(E, n, -1) for a in np_linear(rng, E * n, kk, bits, gs))
    G, U, D = stk(I, H), stk(I, H), stk(H, I)
    x = np_x(rng, T, H)
    lg = rng.standard_normal((T, E)).astype(np.float32)
    dv = [tuple(to_dev_u32(a, dev) if i == 0 else to_dev_bf16(a, dev) for i, a in enumerate(st)) for st in (G, U, D)]
    assert _lib.load().lisaq_moe_decode_supported(T, H, I, E, k, gs, bits) == 1
    outs = {}
    for fused in ("2", "1", "0"):
        force_path("LISAQ_MOE_FUSED", fused)
        o, idx, w = ops.moe_forward(to_dev_bf16(x, dev), to_dev(lg, dev), dv[0], dv[1], dv[2], k, gs, bits,
                                    return_routing=True)
        outs[fused] = (from_dev_bf16(o), idx.cpu().numpy(), w.cpu().numpy())
    from lisa_amd.synth import bf16_bits_to_f32

    assert np.array_equal(outs["1"][1], outs["0"][1]) and np.array_equal(outs["1"][2], outs["0"][2])
    assert_close_bf16(outs["1"][0], bf16_bits_to_f32(outs["0"][0]), what=f"fused vs generic T={T} k={k} bits={bits}")
    # one launch: the two-launch kernels' arithmetic, bit for bit
    for a, b in zip(outs["2"], outs["1"]):
        assert np.array_equal(a, b), f"one launch vs two T={T} k={k} bits={bits}"
    _assert_sync_clear(dev)


def _assert_sync_clear(dev):
    """No wait of the one-launch decode gave up (the give-up word, first in
    the MoE workspace, is still zero)."""
    import torch

    torch.cuda.synchronize()
    word = ops.workspace(dev, 256, "moe_forward")[:4].view(torch.int32).item()
    assert word == 0, "a one-launch wait gave up"


@pytest.mark.parametrize("T,k", [(1, 8), (1, 4), (1, 2), (4, 8)])
def test_moe_one_launch_repeated(dev, force_path, T, k):
    """Eight one-launch decode calls in a row on one stream (T = 1; T = 4
    takes two launches either way), each with new router logits and x (flags
    of one call must not satisfy the next call's waits), every output bitwise
    equal to the two-launch path's; then the
    same eight calls captured in a HIP graph and replayed three times (each
    replay a new dispatch, so a new tag), every replay checked."""
    import torch

    E, H, I, bits, gs = 64, 1024, 512, 4, 64
    rng = np.random.default_rng(77 + T + k)
    stk = lambda n, kk: tuple(a.reshape(E, n, -1) for a in np_linear(rng, E * n, kk, bits, gs))
    G, U, D = stk(I, H), stk(I, H), stk(H, I)
    dv = [tuple(to_dev_u32(a, dev) if i == 0 else to_dev_bf16(a, dev) for i, a in enumerate(st)) for st in (G, U, D)]
    xs = [to_dev_bf16(np_x(rng, T, H), dev) for _ in range(8)]
    lgs = [to_dev(rng.standard_normal((T, E)).astype(np.float32), dev) for _ in range(8)]
    run = lambda i: ops.moe_forward(xs[i], lgs[i], dv[0], dv[1], dv[2], k, gs, bits)
    force_path("LISAQ_MOE_FUSED", "1")
    ref = [run(i).view(torch.int16).clone() for i in range(8)]
    force_path("LISAQ_MOE_FUSED", "2")
    got = [run(i).view(torch.int16).clone() for i in range(8)]
    for i in range(8):
        assert torch.equal(got[i], ref[i]), f"call {i}"
    _assert_sync_clear(dev)
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        run(0)  # workspace sized before capture
    torch.cuda.current_stream().wait_stream(st)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = [run(i) for i in range(8)]
    for rep in range(3):
        for o in outs:
            o.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for i in range(8):
            assert torch.equal(outs[i].view(torch.int16), ref[i]), f"replay {rep} call {i}"
        _assert_sync_clear(dev)


@pytest.mark.parametrize("T,E,k,H,I", [(600, 64, 8, 128, 64), (300, 1024, 4, 256, 128), (600, 1023, 2, 256, 128),
                                       (2100, 1024, 4, 256, 128)])
def test_moe_forward_generic_equals_composition(dev, force_path, T, E, k, H, I):
    """moe_forward's generic path (multi-workgroup counting sort, tile tables
    built from the expert offsets) against the same steps composed from the
    public entry points (one-workgroup sort, tile tables from the sorted ids):
    bit-identical, at a size where the sort spans several workgroups
    (T=600, k=8: 4800 ids), and at E = 1024 / 1023 experts (the sort's scan
    with one thread per expert row, and with a wave per row at 17 blocks)."""
    import torch

    force_path("LISAQ_MOE_FUSED", "0")
    rng = np.random.default_rng(T + E)
    G, U, D = _expert_stack(rng, E, I, H), _expert_stack(rng, E, I, H), _expert_stack(rng, E, H, I)
    x = to_dev_bf16(np_x(rng, T, H), dev)
    lg = to_dev(rng.standard_normal((T, E)).astype(np.float32), dev)
    dv = [tuple(to_dev_u32(a, dev) if i == 0 else to_dev_bf16(a, dev) for i, a in enumerate(st)) for st in (G, U, D)]
    out, idx, wts = ops.moe_forward(x, lg, dv[0], dv[1], dv[2], k, return_routing=True)
    ridx, rw = ops.moe_route(lg, k)
    assert torch.equal(ridx, idx) and torch.equal(rw, wts)
    srt, order, rows, inv, offs = ops.moe_sort(ridx.reshape(-1), E, k)
    xs = ops.gather_rows(x, rows)
    g = ops.gather_qmm(xs, *dv[0], rhs_indices=srt)
    u = ops.gather_qmm(xs, *dv[1], rhs_indices=srt)
    d = ops.gather_qmm(ops.swiglu(g, u), *dv[2], rhs_indices=srt)
    ref = ops.moe_combine(d, rw.reshape(-1), inv, T, k)
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))


@pytest.mark.parametrize("I", [200, 72])
def test_gather_qmm_swiglu_partial_column_block(dev, oracle, I):
    """I not a multiple of 64: the gate|up tile's last 64-column block ends
    partway (the epilogue's column clamp and its gate/up exchange on a partial
    block).  Every run against the oracle's matmul arithmetic (gate and up
    rounded to bf16, then the bf16 SwiGLU: bound 2e-2 + 2e-2|ref|)."""
    import torch

    T, E, k, H, gs, bits = 256, 8, 2, 256, 64, 4
    rng = np.random.default_rng(I)
    stk = lambda n, kk: tuple(a.reshape(E, n, -1) for a in np_linear(rng, E * n, kk, bits, gs))
    G, U = stk(I, H), stk(I, H)
    x = np_x(rng, T, H)
    lg = rng.standard_normal((T, E)).astype(np.float32)
    dv = [tuple(to_dev_u32(a, dev) if i == 0 else to_dev_bf16(a, dev) for i, a in enumerate(st)) for st in (G, U)]
    xd = to_dev_bf16(x, dev)
    ridx, _ = ops.moe_route(to_dev(lg, dev), k)
    srt, order, rows, inv, offs = ops.moe_sort(ridx.reshape(-1), E, k)
    act = from_dev_bf16(ops.gather_qmm_swiglu(xd, rows, dv[0], dv[1], srt, gs, bits))
    torch.cuda.synchronize()
    offs_h, rows_h = offs.cpu().numpy(), rows.cpu().numpy()
    assert act.shape == (T * k, I)
    for e in range(E):
        a, b = offs_h[e], offs_h[e + 1]
        if b == a:
            continue
        xr = x[rows_h[a:b]]
        g = oracle.f32_to_bf16(oracle.qmm(xr, G[0][e], G[1][e], G[2][e], gs, bits))
        u = oracle.f32_to_bf16(oracle.qmm(xr, U[0][e], U[1][e], U[2][e], gs, bits))
        ref = bf16_bits_to_f32(oracle.swiglu(g, u))
        assert_close_bf16(act[a:b], ref, rtol=2e-2, what=f"I={I} expert {e} ({b - a} rows)")


@pytest.mark.parametrize("T,E,k,H,I,bits,gs", [(512, 16, 4, 512, 320, 4, 64), (300, 8, 2, 256, 192, 2, 32),
                                             (1024, 32, 8, 1024, 768, 4, 128), (640, 16, 2, 128, 64, 4, 64),
                                             (1024, 16, 4, 256, 128, 2, 64)])
def test_gather_qmm_swiglu(dev, oracle, force_path, T, E, k, H, I, bits, gs):
    """The fused gate|up + SwiGLU matmul (x rows read through the sort's row
    map) with skewed routing, so that long runs and a run shorter than the
    matvec limit (5 rows) occur: runs at or above the limit bitwise equal to
    swiglu(gather_qmm(gate), gather_qmm(up)) on the gathered rows (the same
    matmul arithmetic); the short run against the oracle's matmul arithmetic
    (gate and up rounded to bf16, then the bf16 SwiGLU: two roundings deep,
    so the bound is 2e-2 + 2e-2|ref|); and moe_forward, which takes this path
    for T*k >= 20*E, bitwise equal to its steps composed from the public entry
    points (route, sort, gather_qmm_swiglu, gather_qmm(down), combine) and
    identical in routing to the three-step path (LISAQ_MOE_GU=0).  Runs averaging >= 192 rows
    (T=1024, E=32, k=8 and the 2-bit T=1024, E=16, k=4) take the 288-row tiles."""
    import torch

    rng = np.random.default_rng(T + 7 * E + bits)
    stk = lambda n, kk: tuple(a.reshape(E, n, -1) for a in np_linear(rng, E * n, kk, bits, gs))
    G, U, D = stk(I, H), stk(I, H), stk(H, I)
    x = np_x(rng, T, H)
    lg = rng.standard_normal((T, E)).astype(np.float32)
    lg[:, 0] += 2.5  # a popular expert
    lg[:, E - 1] = -50.0  # a rare one: picked by 5 tokens only
    lg[:5, E - 1] = 50.0
    dv = [tuple(to_dev_u32(a, dev) if i == 0 else to_dev_bf16(a, dev) for i, a in enumerate(st)) for st in (G, U, D)]
    xd, lgd = to_dev_bf16(x, dev), to_dev(lg, dev)
    ridx, rw = ops.moe_route(lgd, k)
    srt, order, rows, inv, offs = ops.moe_sort(ridx.reshape(-1), E, k)
    act = ops.gather_qmm_swiglu(xd, rows, dv[0], dv[1], srt, gs, bits)
    xs = ops.gather_rows(xd, rows)
    comp = ops.swiglu(ops.gather_qmm(xs, *dv[0], rhs_indices=srt, group_size=gs, bits=bits),
                      ops.gather_qmm(xs, *dv[1], rhs_indices=srt, group_size=gs, bits=bits))
    a_h, c_h, offs_h, rows_h = from_dev_bf16(act), from_dev_bf16(comp), offs.cpu().numpy(), rows.cpu().numpy()
    sizes = np.diff(offs_h)
    lim = ops.qmv_batch_limit(H, I)
    assert sizes.max() >= lim and sizes[E - 1] == 5, sizes
    for e in range(E):
        a, b = offs_h[e], offs_h[e + 1]
        if b - a >= lim:
            assert np.array_equal(a_h[a:b], c_h[a:b]), f"expert {e} ({b - a} rows)"
        elif b > a:
            xr = x[rows_h[a:b]]
            g = oracle.f32_to_bf16(oracle.qmm(xr, G[0][e], G[1][e], G[2][e], gs, bits))
            u = oracle.f32_to_bf16(oracle.qmm(xr, U[0][e], U[1][e], U[2][e], gs, bits))
            ref = bf16_bits_to_f32(oracle.swiglu(g, u))
            assert_close_bf16(a_h[a:b], ref, rtol=2e-2, what=f"short run of expert {e} ({b - a} rows)")
    # the whole block: fused path bitwise equal to its composition; routing as the three-step path
    assert T * k >= 20 * E and H % 64 == 0 and I % 64 == 0
    out, idx, w = ops.moe_forward(xd, lgd, dv[0], dv[1], dv[2], k, gs, bits, return_routing=True)
    d = ops.gather_qmm(act, *dv[2], rhs_indices=srt, group_size=gs, bits=bits)
    ref = ops.moe_combine(d, rw.reshape(-1), inv, T, k)
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
    force_path("LISAQ_MOE_GU", "0")
    out0, idx0, w0 = ops.moe_forward(xd, lgd, dv[0], dv[1], dv[2], k, gs, bits, return_routing=True)
    assert torch.equal(idx, idx0) and torch.equal(w, w0)
    long_tok = np.all(sizes[idx.cpu().numpy()] >= lim, axis=1)
    assert long_tok.any()
    assert np.array_equal(from_dev_bf16(out)[long_tok], from_dev_bf16(out0)[long_tok])
    torch.cuda.synchronize()


@pytest.mark.parametrize("runs", [(300, 64, 65, 256, 320, 1, 40, 129, 0, 513),
                                  (200, 33, 100, 64, 128, 190, 16, 255)])
def test_gather_short_last_tiles(dev, oracle, force_path, runs):
    """A run's last matmul tile of at most 64 rows goes to the short-tile kernel: gather_qmm and
    gather_qmm_swiglu bitwise equal to the same calls with every tile in the tall kernel
    (LISAQ_GATHER_SHORT=0), and gather_qmm's runs against the per-run oracle."""
    import torch

    rng = np.random.default_rng(sum(runs))
    E, N, K = len(runs), 256, 512
    W, S, B = _expert_stack(rng, E, N, K)
    ids = np.repeat(np.arange(E, dtype=np.int32), runs)
    R = ids.size
    x = np_x(rng, R, K)
    args = (to_dev_bf16(x, dev), to_dev_u32(W, dev), to_dev_bf16(S, dev), to_dev_bf16(B, dev))
    sid = to_dev(ids, dev)
    T = 700
    xt = np_x(rng, T, K)
    xrows = to_dev(rng.integers(0, T, R).astype(np.int32), dev)
    U = _expert_stack(rng, E, N, K)
    gate, up = tuple(args[1:]), (to_dev_u32(U[0], dev), to_dev_bf16(U[1], dev), to_dev_bf16(U[2], dev))

    def both():
        y = from_dev_bf16(ops.gather_qmm(*args, rhs_indices=sid))
        a = from_dev_bf16(ops.gather_qmm_swiglu(to_dev_bf16(xt, dev), xrows, gate, up, sid))
        torch.cuda.synchronize()
        return y, a

    y, a = both()
    force_path("LISAQ_GATHER_SHORT", "0")
    y0, a0 = both()
    assert np.array_equal(y, y0)
    assert np.array_equal(a, a0)
    ref = _gather_ref(oracle, x, W, S, B, ids, ops.qmv_batch_limit(K, N))
    assert_close_bf16(y, ref)
