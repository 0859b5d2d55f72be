"""CPU emulation of the matmul launch's index math (lisa_amd/csrc/qmm_kernel.h,
qmm.hip): the workgroup -> (tile, K split, partial unit) mapping of plain,
per-part split and hybrid split launches, the K-step range of every part, the
partial-store and reduction addresses, checked against the workspace size the
host reserves and the x / W / y extents -- for every tile height (128/192/256
rows), split count and hybrid choice at the BASELINE prefill and expert shapes,
including combinations the dispatcher never picks.  No GPU: the formulas below
restate the kernel's and host's integer arithmetic, and every property is an
invariant (coverage exactly once, bounds), not a number copied from the code."""
import itertools

import numpy as np
import pytest

from lisa_amd import _lib

SHAPES = [(128, 17408, 5120), (128, 5120, 17408), (512, 17408, 5120), (512, 5120, 17408),
          (2048, 17408, 5120), (2048, 5120, 17408), (256, 768, 2048), (256, 2048, 768), (70, 300, 1024)]
BK, BN = 64, 256


def normalize_splits(nk_all, S):
    """Host rule: every split non-empty (qmm.hip, S = ceil(nk / ceil(nk / S)))."""
    per = -(-nk_all // S)
    return -(-nk_all // per)


def blocks(M, N, K, MT, S, full_tiles):
    """Yield (kind, tile, split, unit, m0, nt0, kb, nk) per workgroup, as the kernel derives them."""
    BM = 32 * MT
    gn = -(-N // BN)
    T = gn * -(-M // BM)
    nk_all = K // BK
    grid = (full_tiles + (T - full_tiles) * S) if (S > 1 and full_tiles > 0) else T * S
    for bx in range(grid):
        ksplit, unit, whole = S, -1, S == 1
        if S > 1 and full_tiles > 0:
            if bx < full_tiles:
                tile, split, whole, ksplit = bx, 0, True, 1
            else:
                unit = bx - full_tiles
                tile, split = full_tiles + unit // S, unit % S
        else:
            tile, split = bx % T, bx // T
        per = -(-nk_all // ksplit)
        kb = split * per
        nk = min(nk_all - kb, per)
        yield ("whole" if whole else ("unit" if unit >= 0 else "part")), tile, split, unit, \
            (tile // gn) * BM, (tile % gn) * BN, kb, nk


@pytest.mark.parametrize("M,N,K", SHAPES)
def test_every_split_layout_stays_in_bounds_and_covers_once(M, N, K):
    nk_all = K // BK
    for MT, S0 in itertools.product((4, 6, 8), range(1, 17)):
        S = normalize_splits(nk_all, S0) if S0 > 1 else 1
        BM = 32 * MT
        gn = -(-N // BN)
        T = gn * -(-M // BM)
        fulls = [0] + ([T // 256 * 256] if S > 1 and T >= 256 and T % 256 and (T - T // 256 * 256) * S <= 256 else [])
        for full in fulls:
            ws_floats = (T - full) * S * BM * BN if full else (S * M * N if S > 1 else 0)
            steps = np.zeros(T, np.int64)          # K-steps accumulated per tile
            writers = np.zeros(T, np.int64)        # parts per tile
            for kind, tile, split, unit, m0, nt0, kb, nk in blocks(M, N, K, MT, S, full):
                assert 0 <= tile < T
                assert nk >= 1 and 0 <= kb and kb + nk <= nk_all, (MT, S, full, tile, split)
                steps[tile] += nk
                writers[tile] += 1
                # loads: x rows clamped to M - 1, W rows clamped to N - 1, K steps inside [0, K)
                assert m0 < M and nt0 < N
                m_hi = min(m0 + BM, M) - 1
                n_hi = min(nt0 + BN, N) - 1
                if kind == "unit":
                    assert unit * BM * BN + (m_hi - m0) * BN + (n_hi - nt0) < ws_floats
                elif kind == "part":
                    assert split * M * N + m_hi * N + n_hi < ws_floats
                else:
                    assert m_hi * N + n_hi < M * N
            assert (steps == nk_all).all(), (MT, S, full)  # every K step of every tile exactly once
            assert (writers[:full] == 1).all() if full else True
            # reductions read only what the parts wrote
            if full:
                R = T - full
                tsz = BM * BN
                last = (R * tsz // 4 - 1) * 4
                r, e = divmod(last, tsz)
                assert r * S * tsz + e + (S - 1) * tsz + 3 < ws_floats
            elif S > 1:
                assert (S - 1) * M * N + M * N - 1 < ws_floats


@pytest.mark.parametrize("M,N,K", SHAPES)
def test_dispatched_workspace_covers_its_layout(M, N, K):
    """The library's workspace size for the dispatched configuration is at least what one of the layouts
    above needs (per-part with 128-row tiles, or hybrid with 256-row tiles)."""
    lib = _lib.load()
    got = lib.lisaq_qmm_workspace(M, N, K, 64, 4)
    nk_all = K // BK
    if got == 0:
        return
    options = []
    for S0 in range(2, 17):
        S = normalize_splits(nk_all, S0)
        options.append(S * M * N * 4)                       # per-part, 128-row tiles
        T8 = -(-N // BN) * -(-M // 256)
        if T8 >= 256 and T8 % 256:
            options.append((T8 - T8 // 256 * 256) * S * 256 * BN * 4)   # hybrid, 256-row tiles
    assert got in options, (M, N, K, got)
