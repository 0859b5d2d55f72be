"""numpy/ctypes front of the CPU oracle (``lisaq_oracle.c``).

TEST INFRASTRUCTURE ONLY: imported by ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py``.  The product package
``lisa_amd`` never imports it.

bf16 tensors are carried as ``numpy.uint16`` bit patterns.  Every wrapper
checks shapes and returns freshly allocated numpy arrays.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_SO = os.path.join(_HERE, "liblisaq_oracle.so")
_lib = None


def build(force: bool = False) -> str:
    """Compile the oracle with its Makefile (gcc only)."""
    if force or not os.path.exists(_SO) or os.path.getmtime(_SO) < os.path.getmtime(
        os.path.join(_HERE, "lisaq_oracle.c")
    ):
        subprocess.run(["make", "-s", "-C", _HERE, "-B" if force else "all"], check=True)
    return _SO


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_SO):
            build()
        _lib = ctypes.CDLL(_SO)
    return _lib


def _p(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


i64 = ctypes.c_int64


def f32_to_bf16(a) -> np.ndarray:
    a = _c(a, np.float32)
    out = np.empty(a.shape, np.uint16)
    lib().lo_f32_to_bf16(_p(a), _p(out), i64(a.size))
    return out


def bf16_to_f32(a) -> np.ndarray:
    a = _c(a, np.uint16)
    out = np.empty(a.shape, np.float32)
    lib().lo_bf16_to_f32(_p(a), _p(out), i64(a.size))
    return out


def unpack(w, K: int, bits: int) -> np.ndarray:
    w = _c(w, np.uint32)
    rows = w.size // (K * bits // 32)
    out = np.empty((rows, K), np.uint8)
    lib().lo_unpack(_p(w), i64(rows), i64(K), ctypes.c_int(bits), _p(out))
    return out


def quantize_f32(w, group_size: int = 64, bits: int = 4):
    """Reference ``ops::quantize`` (AO:218-290): returns (wq u32, scales f32, biases f32)."""
    w = _c(w, np.float32)
    K = w.shape[-1]
    rows = w.size // K
    if K % group_size or group_size % (32 // bits):
        raise ValueError(f"quantize: group size {group_size} incompatible with K={K}, bits={bits}")
    wq = np.zeros(w.shape[:-1] + (K * bits // 32,), np.uint32)
    sc = np.empty(w.shape[:-1] + (K // group_size,), np.float32)
    bi = np.empty_like(sc)
    rc = lib().lo_quantize_f32(_p(w), i64(rows), i64(K), ctypes.c_int(group_size), ctypes.c_int(bits),
                               _p(wq), _p(sc), _p(bi))
    if rc != 0:
        raise ValueError("quantize rejected the shape")
    return wq, sc, bi


def dequantize(w, scales, biases, group_size: int, bits: int) -> np.ndarray:
    w = _c(w, np.uint32)
    s = _c(scales, np.uint16)
    b = _c(biases, np.uint16)
    K = w.shape[-1] * 32 // bits
    rows = w.size // w.shape[-1]
    out = np.empty(w.shape[:-1] + (K,), np.float32)
    lib().lo_dequantize(_p(w), _p(s), _p(b), i64(rows), i64(K), ctypes.c_int(group_size),
                        ctypes.c_int(bits), _p(out))
    return out


def _mm(fn, x, w, scales, biases, group_size, bits):
    x = _c(x, np.uint16)
    w = _c(w, np.uint32)
    s = _c(scales, np.uint16)
    b = _c(biases, np.uint16)
    K = x.shape[-1]
    M = x.size // K
    N = w.shape[0]
    assert w.shape == (N, K * bits // 32), (w.shape, N, K)
    assert s.shape == (N, K // group_size) and b.shape == s.shape
    y = np.empty((M, N), np.float32)
    fn(_p(x), _p(w), _p(s), _p(b), i64(M), i64(N), i64(K), ctypes.c_int(group_size),
       ctypes.c_int(bits), _p(y))
    return y


def qmv(x, w, scales, biases, group_size: int = 64, bits: int = 4) -> np.ndarray:
    """qmv/qmv_wide semantics (f32 weights, per-group s*P + b*X); f32 [M,N]."""
    return _mm(lib().lo_qmv, x, w, scales, biases, group_size, bits)


def qmm(x, w, scales, biases, group_size: int = 64, bits: int = 4) -> np.ndarray:
    """qmm semantics (weights rounded to bf16, f32 accumulate); f32 [M,N]."""
    return _mm(lib().lo_qmm, x, w, scales, biases, group_size, bits)


def qmv_threads(x, w, scales, biases, group_size: int, bits: int, nthreads: int) -> np.ndarray:
    x = _c(x, np.uint16)
    K = x.shape[-1]
    M = x.size // K
    N = w.shape[0]
    y = np.empty((M, N), np.float32)
    lib().lo_qmv_threads(_p(x), _p(w), _p(scales), _p(biases), i64(M), i64(N), i64(K),
                         ctypes.c_int(group_size), ctypes.c_int(bits), _p(y), ctypes.c_int(nthreads))
    return y


def add_rms_norm(x, r, norm_w, eps: float):
    """Prologue of affine_qmv_fast_addnorm (norm_qmv.metal:376-400): s = bf16(x + r);
    inv = rsqrt(f32(sum(s^2)/K) + eps) rounded once to f32 (metal::precise::rsqrt, norm_qmv.metal:377);
    normed = bf16(norm_w * bf16(s * inv)).  x, r: bf16 bits
    [M, K]; norm_w: bf16 bits [K].  Returns (s, normed) as bf16 bits.  The sum of squares is taken
    in float64 (the reference's order is Apple's simd_sum tree, not reproducible here)."""
    x = _c(x, np.uint16)
    r = _c(r, np.uint16)
    K = x.shape[-1]
    s = f32_to_bf16(bf16_to_f32(x) + bf16_to_f32(r))
    sf = bf16_to_f32(s).astype(np.float32)
    ss = (sf.astype(np.float64) ** 2).sum(axis=-1, keepdims=True).astype(np.float32)
    a = (ss / np.float32(K) + np.float32(eps)).astype(np.float32)
    inv = (1.0 / np.sqrt(a.astype(np.float64))).astype(np.float32)
    t = bf16_to_f32(f32_to_bf16(sf * inv)).astype(np.float32)
    normed = f32_to_bf16(bf16_to_f32(_c(norm_w, np.uint16)).reshape(1, K).astype(np.float32) * t)
    return s, normed


def topk_route(logits, k: int):
    lg = _c(logits, np.float32)
    T, E = lg.shape
    idx = np.empty((T, k), np.int32)
    wt = np.empty((T, k), np.float32)
    lib().lo_topk_route(_p(lg), i64(T), ctypes.c_int(E), ctypes.c_int(k), _p(idx), _p(wt))
    return idx, wt


def moe_sort(idx_flat, num_experts: int, top_k: int):
    """Returns (sorted_idx, order, token_rows, inverse, expert_offsets[E+1])."""
    idx = _c(idx_flat, np.int32).reshape(-1)
    R = idx.size
    outs = [np.empty(R, np.int32) for _ in range(4)]
    offs = np.empty(num_experts + 1, np.int32)
    rc = lib().lo_moe_sort(_p(idx), i64(R), ctypes.c_int(num_experts), ctypes.c_int(top_k),
                           *[_p(o) for o in outs], _p(offs))
    if rc != 0:
        raise ValueError("expert id out of range")
    return (*outs, offs)


def swiglu(gate, up) -> np.ndarray:
    g = _c(gate, np.uint16)
    u = _c(up, np.uint16)
    assert g.shape == u.shape
    out = np.empty(g.shape, np.uint16)
    lib().lo_swiglu(_p(g), _p(u), _p(out), i64(g.size))
    return out


def moe_combine(down_sorted, weights, inverse, T: int, k: int) -> np.ndarray:
    d = _c(down_sorted, np.uint16)
    H = d.shape[-1]
    w = _c(weights, np.float32).reshape(-1)
    inv = _c(inverse, np.int32).reshape(-1)
    assert w.size == T * k and inv.size == T * k
    out = np.empty((T, H), np.uint16)
    lib().lo_moe_combine(_p(d), _p(w), _p(inv), i64(T), ctypes.c_int(k), i64(H), _p(out))
    return out


# --- signatures -----------------------------------------------------------
def _declare():
    L = lib()
    for name in ["lo_f32_to_bf16", "lo_bf16_to_f32", "lo_unpack", "lo_dequantize", "lo_qmv",
                 "lo_qmm", "lo_topk_route", "lo_swiglu", "lo_moe_combine"]:
        getattr(L, name).restype = None
    for name in ["lo_quantize_f32", "lo_moe_sort", "lo_qmv_threads"]:
        getattr(L, name).restype = ctypes.c_int


try:
    _declare()
except OSError:  # not built yet; build() then lib() will load it
    _lib = None


# ---- every compute dtype and code width (lisaq_quantized_matmul_typed) ----
# x, scales and biases are float arrays holding values of the compute dtype T
# (bf16, f16 or f32), i.e. after the reference's promotion (AO:398-404).

def _round_to(a, dtype: str) -> np.ndarray:
    """float32 values rounded to T (nearest even) and back to float32."""
    a = np.asarray(a, np.float32)
    if dtype == "bf16":
        return bf16_to_f32(f32_to_bf16(a))
    if dtype == "f16":
        return a.astype(np.float16).astype(np.float32)
    return a


def qmv_typed(x, w, scales, biases, group_size: int, bits: int) -> np.ndarray:
    """Matvec semantics for any T (QM:767-830, 996-1088): weights never
    rounded; per group scale*sum(x*q) + bias*sum(x), here in float64; [M, N]
    float64 (the caller rounds to T)."""
    x = np.asarray(x, np.float64)
    K = x.shape[-1]
    q = unpack(w, K, bits).astype(np.float64)               # [N, K]
    N, G = q.shape[0], K // group_size
    xg = x.reshape(x.shape[0], G, group_size)                 # [M, G, gs]
    qg = q.reshape(N, G, group_size)                          # [N, G, gs]
    dots = np.einsum("mgk,ngk->mng", xg, qg)                 # [M, N, G]
    xs = xg.sum(-1)                                           # [M, G]
    s = np.asarray(scales, np.float64).reshape(N, G)
    b = np.asarray(biases, np.float64).reshape(N, G)
    return (dots * s[None] + xs[:, None, :] * b[None]).sum(-1)


def qmm_typed(x, w, scales, biases, group_size: int, bits: int, dtype: str) -> np.ndarray:
    """Matmul semantics for any T (QM:585-703, 1208-1326): each weight is
    T(fma(scale, q, bias)) (the f32 fma rounded once to f32, then to T), then
    x . w^T accumulated here in float64; [M, N] float64."""
    x = np.asarray(x, np.float64)
    K = x.shape[-1]
    q = unpack(w, K, bits).astype(np.float64)
    N, G = q.shape[0], K // group_size
    s = np.repeat(np.asarray(scales, np.float64).reshape(N, G), group_size, axis=1)
    b = np.repeat(np.asarray(biases, np.float64).reshape(N, G), group_size, axis=1)
    wt = _round_to((s * q + b).astype(np.float32), dtype).astype(np.float64)  # s*q exact in f64: one rounding to f32
    return x @ wt.T
