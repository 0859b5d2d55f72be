"""The C ABI library loads, exports every symbol include/lisaq.h declares, and
its host-side checks (validation before any device work) behave like the
reference's rejections.  CPU only: no call here reaches a kernel launch."""
import ctypes
import os
import re

import pytest

from lisa_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    text = open(os.path.join(ROOT, "include", "lisaq.h")).read()
    return sorted(set(re.findall(r"LISAQ_API\s+[\w\s\*]+?\b(lisaq_\w+)\s*\(", text)))


def test_every_declared_symbol_is_exported():
    lib = _lib.load()
    syms = declared_symbols()
    assert len(syms) >= 20
    for s in syms:
        assert hasattr(lib, s), s
    assert set(syms) == set(_lib.SIGNATURES), set(syms) ^ set(_lib.SIGNATURES)


def test_version_and_error_string():
    lib = _lib.load()
    assert lib.lisaq_version() >= 100
    assert isinstance(lib.lisaq_last_error(), bytes)


def test_qmv_batch_limit_matches_reference():
    # jit/matmul.rs:1873-1881
    lim = _lib.load().lisaq_qmv_batch_limit
    assert lim(2048, 2048) == 33 and lim(2048, 768) == 33
    assert lim(4096, 4096) == 25 and lim(2560, 4096) == 25
    assert lim(5120, 17408) == 13 and lim(2560, 9728) == 13 and lim(768, 4096) == 25 and lim(768, 4097) == 13


def test_detect_group_size_matches_reference():
    # core/quant.rs:273-287
    d = _lib.load().lisaq_detect_group_size
    assert d(640, 80, 4) == 64  # 17408x5120 4-bit gs64
    assert d(320, 80, 2) == 64
    assert d(32, 8, 4) == 32  # smoke.rs: K=256, gs 32
    assert d(640, 3, 4) == -1  # does not divide
    assert d(0, 80, 4) == -1 and d(640, 0, 4) == -1 and d(640, 80, 3) == -1
    assert d(1, 1, 4) == 8
    assert d(4096 * 2, 1, 4) == -1  # group above 4096


def test_check_layout():
    lib = _lib.load()
    K = ctypes.c_int64()
    gs = ctypes.c_int()
    assert lib.lisaq_check_layout(17408, 640, 17408, 80, 17408, 80, 4, ctypes.byref(K), ctypes.byref(gs)) == 0
    assert (K.value, gs.value) == (5120, 64)
    assert lib.lisaq_check_layout(17408, 640, 17408, 80, 17407, 80, 4, None, None) == _lib.EINVAL_SHAPE
    assert b"rows" in lib.lisaq_last_error()
    assert lib.lisaq_check_layout(10, 640, 10, 80, 10, 79, 4, None, None) == _lib.EINVAL_SHAPE
    assert lib.lisaq_check_layout(10, 641, 10, 7, 10, 7, 4, None, None) == _lib.EINVAL_SHAPE


FAKE = 0x10000  # aligned, never dereferenced: every call below fails validation first


@pytest.mark.parametrize("kwargs,code,msg", [
    (dict(transpose=0), _lib.EINVAL_LAYOUT, b"transpose"),
    (dict(b=None), _lib.EINVAL_LAYOUT, b"biases"),
    (dict(bits=3), _lib.EUNSUPPORTED, b"bits"),
    (dict(gs=48), _lib.EUNSUPPORTED, b"group_size"),
    (dict(K=96), _lib.EINVAL_SHAPE, b"incompatible"),
    (dict(M=-1), _lib.EINVAL_SHAPE, b"negative"),
    (dict(x=FAKE + 2), _lib.EINVAL_LAYOUT, b"aligned"),
    (dict(x=None), _lib.EINVAL_LAYOUT, b"null"),
])
def test_quantized_matmul_rejections(kwargs, code, msg):
    lib = _lib.load()
    a = dict(x=FAKE, w=FAKE, s=FAKE, b=FAKE, y=FAKE, M=1, N=64, K=128, transpose=1, gs=64, bits=4)
    a.update(kwargs)
    rc = lib.lisaq_quantized_matmul(None, a["x"], a["w"], a["s"], a["b"], a["y"], a["M"], a["N"], a["K"],
                                    a["transpose"], a["gs"], a["bits"], None, 0)
    assert rc == code
    assert msg in lib.lisaq_last_error()


def test_empty_problem_is_a_no_op():
    lib = _lib.load()
    # M = 0 and N = 0 enqueue nothing (no device needed)
    assert lib.lisaq_quantized_matmul(None, FAKE, FAKE, FAKE, FAKE, FAKE, 0, 64, 128, 1, 64, 4, None, 0) == 0
    assert lib.lisaq_qmm(None, FAKE, FAKE, FAKE, FAKE, FAKE, 5, 0, 128, 64, 4, None, 0) == 0
    assert lib.lisaq_moe_combine(None, FAKE, FAKE, FAKE, FAKE, 0, 8, 16) == 0


def test_other_rejections():
    lib = _lib.load()
    # x of 2^32 elements: refused before anything is enqueued
    assert lib.lisaq_qmm(None, FAKE, FAKE, FAKE, FAKE, FAKE, 1 << 20, 256, 4096, 64, 4, None, 0) == _lib.EINVAL_SHAPE
    assert b"2^31" in lib.lisaq_last_error()
    assert lib.lisaq_quantized_matmul(None, FAKE, FAKE, FAKE, FAKE, FAKE, 1 << 20, 256, 4096, 1, 64, 4,
                                      None, 0) == _lib.EINVAL_SHAPE
    assert lib.lisaq_qmv(None, FAKE, FAKE, FAKE, FAKE, FAKE, 33, 64, 128, 64, 4, None, 0) == _lib.EINVAL_SHAPE
    assert lib.lisaq_moe_route(None, FAKE, 4, 2000, 8, FAKE, FAKE) == _lib.EINVAL_SHAPE
    assert lib.lisaq_moe_route(None, FAKE, 4, 128, 0, FAKE, FAKE) == _lib.EINVAL_SHAPE
    assert lib.lisaq_moe_combine(None, FAKE, FAKE, FAKE, FAKE, 4, 0, 16) == _lib.EINVAL_SHAPE
    assert lib.lisaq_quantize(None, FAKE, 7, FAKE, FAKE, FAKE, 1, 64, 64, 4) == _lib.EINVAL_DTYPE
    assert lib.lisaq_dequantize(None, FAKE, FAKE, FAKE, FAKE, 1, 96, 64, 4) == _lib.EINVAL_SHAPE
    # gather: rhs required, workspace required
    assert lib.lisaq_gather_qmm(None, FAKE, FAKE, FAKE, FAKE, None, FAKE, 8, 64, 128, 4, 1, 64, 4,
                                None, 0) == _lib.EINVAL_LAYOUT
    assert lib.lisaq_gather_qmm(None, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 8, 64, 128, 4, 1, 64, 4,
                                None, 0) == _lib.EWORKSPACE


def test_qmv_addnorm_rejections():
    """jit::affine_qmv_fast_addnorm's eligibility (matmul.rs:328-347), checked before anything is enqueued."""
    lib = _lib.load()
    call = lambda M, N, K, gs, bits, ptr=FAKE: lib.lisaq_qmv_addnorm(
        None, ptr, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, M, N, K, 1e-6, gs, bits, None, 0)
    assert call(1, 512, 5120, 32, 4) == _lib.EUNSUPPORTED
    assert call(1, 512, 5120, 64, 2) == _lib.EUNSUPPORTED
    assert call(2, 512, 5120, 64, 4) == _lib.EUNSUPPORTED and b"M=1" in lib.lisaq_last_error()
    assert call(1, 512, 4096, 64, 4) == _lib.EUNSUPPORTED and b"ineligible" in lib.lisaq_last_error()
    assert call(1, 500, 5120, 64, 4) == _lib.EUNSUPPORTED
    assert call(1, 512, 5120, 64, 4, None) == _lib.EINVAL_LAYOUT


def test_workspace_queries():
    lib = _lib.load()
    # one row: no workspace; 2-8 rows: the one-stream kernel (eight rows at K = 9728 stage x in two
    # passes), no workspace; 9 rows over few row tiles (N = 2560: 160 tiles of 16 rows): the streaming
    # matvec splits K in four, f32 parts [4][9][2560]
    assert lib.lisaq_quantized_matmul_workspace(1, 17408, 5120, 64, 4) == 0
    assert lib.lisaq_quantized_matmul_workspace(8, 2560, 9728, 64, 4) == 0
    assert lib.lisaq_quantized_matmul_workspace(9, 2560, 9728, 64, 4) == 4 * 9 * 2560 * 4
    assert lib.lisaq_quantized_matmul_workspace(4, 2560, 9728, 64, 4) == 0  # one-stream kernel
    assert lib.lisaq_quantized_matmul_workspace(8, 17408, 5120, 64, 4) == 0
    # matmul at M=2048, N=17408: 68 x 8 = 544 tiles of 256 x 256; the 32 past two full rounds of 256 CUs are
    # split over K into 8 parts with f32 partials: 32 * 8 * 256 * 256 * 4 bytes
    assert lib.lisaq_quantized_matmul_workspace(2048, 17408, 5120, 64, 4) == 32 * 8 * 256 * 256 * 4
    # M=2048, N=5120: 8 x 20 = 160 tiles of 256 rows, fewer than one round: 192-row tiles, no split
    assert lib.lisaq_quantized_matmul_workspace(2048, 5120, 17408, 64, 4) == 0
    assert lib.lisaq_gather_qmm_workspace(32768, 768, 2048, 128, 64, 4) >= 256
    assert lib.lisaq_moe_workspace(4096, 2048, 768, 128, 8, 64, 4) > 32768 * 2048 * 2


def test_qmv_addnorm_rejects_overlapping_outputs():
    """The add+RMSNorm outputs are written while other workgroups still read x and r: an overlap is an
    error (EINVAL_LAYOUT) found before any device work (the pointers here are never dereferenced)."""
    lib = _lib.load()
    K, N = 5120, 17408
    x, r, nw, w, s, b, so, no, y = (0x100000 * (i + 1) for i in range(9))
    rc = lib.lisaq_qmv_addnorm(None, x, r, nw, w, s, b, x + 64, no, y, 1, N, K, ctypes.c_float(1e-6), 64, 4, None, 0)
    assert rc == _lib.EINVAL_LAYOUT and b"overlap" in lib.lisaq_last_error()
    rc = lib.lisaq_qmv_addnorm(None, x, r, nw, w, s, b, so, r, y, 1, N, K, ctypes.c_float(1e-6), 64, 4, None, 0)
    assert rc == _lib.EINVAL_LAYOUT
