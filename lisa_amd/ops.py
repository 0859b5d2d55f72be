"""Operator surface of the MLX affine quantized linear, on device tensors.

Mirrors ``crates/lisa-mlx/src/ops/array_ops.rs`` of the reference: same
names, same argument meaning (``transpose``, ``group_size``, ``bits``,
optional ``biases``), same rejections (raised as :class:`LisaqError` where
the reference returns ``Err``).  Every op runs the HIP kernels of
``liblisaq.so`` through its C ABI on the current torch stream; PyTorch only
provides device memory and streams.

Tensors: ``x`` bf16 ``[..., K]``; ``w`` uint32 (``torch.int32`` or
``torch.uint32`` storage) ``[N, K*bits/32]``; ``scales``/``biases`` bf16
``[N, K/group_size]``.  Outputs are freshly allocated (as the reference's
ops return new arrays).
"""
from __future__ import annotations

import threading
from typing import Optional, Tuple

import torch

from . import _lib
from ._lib import LisaqError

__all__ = [
    "LisaqError", "quantized_matmul", "quantized_matmul_serial_rows", "qmv", "qmm", "gather_qmm",
    "dequantize", "quantize", "moe_route", "moe_sort", "gather_rows", "swiglu", "gather_qmm_swiglu", "moe_combine",
    "moe_forward", "qmv_batch_limit", "detect_group_size",
]

_ws_lock = threading.Lock()
_ws: dict = {}
_ws_retired: list = []


def workspace(device: torch.device, nbytes: int, kind: str = "linear") -> torch.Tensor:
    """A zero-initialised scratch buffer of at least ``nbytes`` on ``device``.

    ``kind`` "linear" is the quantized-matmul workspace (split-K partials of
    the matmul path), reused by calls ordered on one stream; "moe" is scratch
    for gather_qmm (tile tables, intermediates); "moe_forward" moe_forward's
    (intermediates, the decode path's flags and give-up word).

    A buffer that is outgrown is replaced but never freed: a HIP graph captured
    earlier still holds its address in its kernel arguments, and freeing it
    would let the caching allocator hand that memory to another tensor which a
    later replay of the graph would then overwrite.  Outgrown buffers stay
    alive for the life of the process (at most a few per device and kind)."""
    key = (device.type, device.index, kind)
    nbytes = max(int(nbytes), 256)
    with _ws_lock:
        buf = _ws.get(key)
        if buf is None or buf.numel() < nbytes:
            if buf is not None:
                _ws_retired.append(buf)
            buf = torch.zeros(nbytes, dtype=torch.uint8, device=device)
            _ws[key] = buf
        return buf


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _require(cond: bool, code: int, msg: str) -> None:
    if not cond:
        raise LisaqError(code, msg)


def _bf16(t: torch.Tensor, name: str) -> torch.Tensor:
    _require(t.is_cuda, _lib.EINVAL_LAYOUT, f"{name} must be a device tensor")
    _require(t.dtype == torch.bfloat16, _lib.EINVAL_DTYPE,
             f"{name}: compute dtype {t.dtype} not supported (bfloat16 only)")
    return t.contiguous()


def _u32(t: torch.Tensor, name: str) -> torch.Tensor:
    _require(t.is_cuda, _lib.EINVAL_LAYOUT, f"{name} must be a device tensor")
    _require(t.dtype in (torch.int32, torch.uint32), _lib.EINVAL_DTYPE, f"{name} must be uint32 packed codes")
    return t.contiguous()


def qmv_batch_limit(K: int, N: int) -> int:
    """MLX ``get_qmv_batch_limit`` (jit/matmul.rs:1873-1881)."""
    return _lib.load().lisaq_qmv_batch_limit(K, N)


def detect_group_size(weight_cols: int, scales_cols: int, bits: int) -> Optional[int]:
    """core/quant.rs:273-287."""
    g = _lib.load().lisaq_detect_group_size(weight_cols, scales_cols, bits)
    return None if g < 0 else g


def _mm(entry: str, x, w, scales, biases, transpose, group_size, bits):
    _require(transpose, _lib.EINVAL_LAYOUT, f"{entry}: only transpose=true supported")
    _require(biases is not None, _lib.EINVAL_LAYOUT, f"{entry}: affine biases required")
    x = _bf16(x, "x")
    w = _u32(w, "w")
    scales = _bf16(scales, "scales")
    biases = _bf16(biases, "biases")
    K = x.shape[-1]
    M = x.numel() // K if K else 0
    N = w.shape[0]
    _require(w.dim() == 2 and w.shape[1] * 32 // bits == K, _lib.EINVAL_SHAPE,
             f"{entry}: w {tuple(w.shape)} does not match K={K}, bits={bits}")
    _require(scales.shape == (N, K // group_size) and biases.shape == scales.shape, _lib.EINVAL_SHAPE,
             f"{entry}: scales/biases {tuple(scales.shape)} != ({N}, {K // group_size})")
    y = torch.empty(*x.shape[:-1], N, dtype=torch.bfloat16, device=x.device)
    lib = _lib.load()
    if entry == "lisaq_qmm":
        nbytes = lib.lisaq_qmm_workspace(M, N, K, group_size, bits)
    else:
        nbytes = lib.lisaq_quantized_matmul_workspace(M, N, K, group_size, bits)
    ws = workspace(x.device, nbytes)
    args = [_stream(x), x.data_ptr(), w.data_ptr(), scales.data_ptr(), biases.data_ptr(), y.data_ptr(), M, N, K]
    if entry in ("lisaq_quantized_matmul", "lisaq_quantized_matmul_serial_rows"):
        args.append(1)
    args += [group_size, bits, ws.data_ptr(), ws.numel()]
    _lib.call(entry, *args)
    return y


def quantized_matmul(x, w, scales, biases=None, transpose=True, group_size=64, bits=4):
    """``ops::quantized_matmul`` (array_ops.rs:378-493): ``x . dequant(w)^T``.

    Dispatch as the reference: M < qmv_batch_limit(K, N) -> matvec kernel
    (f32 weights), else the MFMA matmul (weights rounded to bf16).  x,
    scales and biases are promoted to one compute dtype first (bf16, f16 or
    f32, array_ops.rs:398-404); anything but bf16 with 2/4-bit codes goes
    through ``lisaq_quantized_matmul_typed`` (every dtype, 2/4/8 bits)."""
    _require(biases is not None, _lib.EINVAL_LAYOUT, "quantized_matmul: affine biases required")
    dt = torch.promote_types(torch.promote_types(x.dtype, scales.dtype), biases.dtype)
    if dt == torch.bfloat16 and bits in (2, 4):
        return _mm("lisaq_quantized_matmul", x, w, scales, biases, transpose, group_size, bits)
    return _mm_typed(x, w, scales, biases, transpose, group_size, bits, dt)


_DTYPE_CODE = {torch.bfloat16: _lib.DTYPE_BF16, torch.float16: _lib.DTYPE_F16, torch.float32: _lib.DTYPE_F32}


def _mm_typed(x, w, scales, biases, transpose, group_size, bits, dt):
    _require(transpose, _lib.EINVAL_LAYOUT, "quantized_matmul: only transpose=true supported")
    _require(dt in _DTYPE_CODE, _lib.EINVAL_DTYPE, f"quantized_matmul: unsupported compute dtype {dt}")
    for t, name in ((x, "x"), (scales, "scales"), (biases, "biases")):
        _require(t.is_cuda, _lib.EINVAL_LAYOUT, f"{name} must be a device tensor")
    x, scales, biases = (t.to(dt).contiguous() for t in (x, scales, biases))
    w = _u32(w, "w")
    K = x.shape[-1]
    M = x.numel() // K if K else 0
    N = w.shape[0]
    _require(w.dim() == 2 and w.shape[1] * 32 // bits == K, _lib.EINVAL_SHAPE,
             f"quantized_matmul: w {tuple(w.shape)} does not match K={K}, bits={bits}")
    _require(scales.shape == (N, K // group_size) and biases.shape == scales.shape, _lib.EINVAL_SHAPE,
             f"quantized_matmul: scales/biases {tuple(scales.shape)} != ({N}, {K // group_size})")
    y = torch.empty(*x.shape[:-1], N, dtype=dt, device=x.device)
    _lib.call("lisaq_quantized_matmul_typed", _stream(x), x.data_ptr(), w.data_ptr(), scales.data_ptr(),
              biases.data_ptr(), y.data_ptr(), M, N, K, 1, group_size, bits, _DTYPE_CODE[dt], None, 0)
    return y


def quantized_matmul_serial_rows(x, w, scales, biases=None, transpose=True, group_size=64, bits=4):
    """``ops::quantized_matmul_serial_rows`` (array_ops.rs:500-555): rows 2..8
    bitwise equal to independent M=1 calls."""
    return _mm("lisaq_quantized_matmul_serial_rows", x, w, scales, biases, transpose, group_size, bits)


def qmv(x, w, scales, biases, group_size=64, bits=4):
    """Forced matvec path (1 <= M <= 32)."""
    return _mm("lisaq_qmv", x, w, scales, biases, True, group_size, bits)


def qmm(x, w, scales, biases, group_size=64, bits=4):
    """Forced MFMA matmul path (any M)."""
    return _mm("lisaq_qmm", x, w, scales, biases, True, group_size, bits)


def gather_qmm(x, w, scales, biases=None, lhs_indices=None, rhs_indices=None, transpose=True,
               group_size=64, bits=4, sorted_indices=True):
    """``ops::gather_qmm`` (array_ops.rs:561-642), the sorted right-hand path:
    ``x`` ``[R, 1, K]`` (or ``[R, K]``) rows sorted by expert, ``w``
    ``[E, N, K*bits/32]``, ``rhs_indices`` ``[R]`` -> ``[R, 1, N]`` (or ``[R, N]``)."""
    _require(transpose, _lib.EINVAL_LAYOUT, "gather_qmm: only transpose=true supported")
    _require(lhs_indices is None, _lib.EUNSUPPORTED, "gather_qmm: lhs_indices path not ported")
    _require(sorted_indices, _lib.EUNSUPPORTED, "gather_qmm: only sorted_indices=true supported")
    _require(rhs_indices is not None, _lib.EINVAL_LAYOUT, "gather_qmm: rhs_indices required")
    _require(biases is not None, _lib.EINVAL_LAYOUT, "gather_qmm: affine biases required")
    x = _bf16(x, "x")
    w = _u32(w, "w")
    scales = _bf16(scales, "scales")
    biases = _bf16(biases, "biases")
    rhs = rhs_indices.to(torch.int32).contiguous()
    K = x.shape[-1]
    R = x.numel() // K
    _require(w.dim() == 3 and w.shape[2] * 32 // bits == K, _lib.EINVAL_SHAPE,
             f"gather_qmm: w {tuple(w.shape)} does not match K={K}, bits={bits}")
    E, N = w.shape[0], w.shape[1]
    _require(rhs.numel() == R, _lib.EINVAL_SHAPE, f"gather_qmm: {rhs.numel()} indices for {R} rows")
    _require(scales.shape == (E, N, K // group_size) and biases.shape == scales.shape, _lib.EINVAL_SHAPE,
             "gather_qmm: scales/biases shape mismatch")
    y = torch.empty(*x.shape[:-1], N, dtype=torch.bfloat16, device=x.device)
    lib = _lib.load()
    nbytes = lib.lisaq_gather_qmm_workspace(R, N, K, E, group_size, bits)
    ws = workspace(x.device, nbytes, "moe")
    _lib.call("lisaq_gather_qmm", _stream(x), x.data_ptr(), w.data_ptr(), scales.data_ptr(), biases.data_ptr(),
              rhs.data_ptr(), y.data_ptr(), R, N, K, E, 1, group_size, bits, ws.data_ptr(), ws.numel())
    return y


def qmv_addnorm(x, r, norm_weight, w, scales, biases, eps: float, group_size=64, bits=4, write_norm=True):
    """``jit::affine_qmv_fast_addnorm`` (matmul.rs:315-443): residual add + RMSNorm of x [1, K], then the
    decode matvec on the normed row.  Returns ``(y [1, N], sum [1, K], normed [1, K] or None)`` like the
    reference; ``write_norm`` only decides whether ``normed`` is returned."""
    x = _bf16(x, "x")
    r = _bf16(r, "r")
    norm_weight = _bf16(norm_weight, "norm_weight")
    w = _u32(w, "w")
    scales = _bf16(scales, "scales")
    biases = _bf16(biases, "biases")
    _require(x.dim() == 2 and r.shape == x.shape, _lib.EINVAL_SHAPE, f"qmv_addnorm: x {tuple(x.shape)}, r {tuple(r.shape)}")
    M, K = x.shape
    N = w.shape[0]
    _require(norm_weight.numel() == K, _lib.EINVAL_SHAPE, f"qmv_addnorm: norm weight of {norm_weight.numel()} != K={K}")
    _require(w.dim() == 2 and w.shape[1] * 32 // bits == K, _lib.EINVAL_SHAPE,
             f"qmv_addnorm: w {tuple(w.shape)} does not match K={K}, bits={bits}")
    _require(scales.shape == (N, K // group_size) and biases.shape == scales.shape, _lib.EINVAL_SHAPE,
             f"qmv_addnorm: scales/biases {tuple(scales.shape)} != ({N}, {K // group_size})")
    y = torch.empty(M, N, dtype=torch.bfloat16, device=x.device)
    sum_out = torch.empty_like(x)
    norm_out = torch.empty_like(x)
    lib = _lib.load()
    ws = workspace(x.device, lib.lisaq_quantized_matmul_workspace(M, N, K, group_size, bits))
    _lib.call("lisaq_qmv_addnorm", _stream(x), x.data_ptr(), r.data_ptr(), norm_weight.data_ptr(), w.data_ptr(),
              scales.data_ptr(), biases.data_ptr(), sum_out.data_ptr(), norm_out.data_ptr(), y.data_ptr(), M, N, K,
              float(eps), group_size, bits, ws.data_ptr(), ws.numel())
    return y, sum_out, (norm_out if write_norm else None)


def dequantize(w, scales, biases, group_size=64, bits=4):
    """``ops::dequantize`` (array_ops.rs:37-84): bf16 ``[..., K]``."""
    w = _u32(w, "w")
    scales = _bf16(scales, "scales")
    biases = _bf16(biases, "biases")
    K = w.shape[-1] * 32 // bits
    rows = w.numel() // w.shape[-1] if w.shape[-1] else 0
    out = torch.empty(*w.shape[:-1], K, dtype=torch.bfloat16, device=w.device)
    _lib.call("lisaq_dequantize", _stream(w), w.data_ptr(), scales.data_ptr(), biases.data_ptr(),
              out.data_ptr(), rows, K, group_size, bits)
    return out


def quantize(w, group_size=64, bits=4) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """``ops::quantize`` (array_ops.rs:218-290) -> (wq uint32-as-int32, scales, biases)
    with scales/biases in ``w``'s dtype (bf16 or f32)."""
    _require(w.is_cuda, _lib.EINVAL_LAYOUT, "w must be a device tensor")
    _require(w.dtype in (torch.bfloat16, torch.float32), _lib.EINVAL_DTYPE, f"quantize: dtype {w.dtype}")
    w = w.contiguous()
    K = w.shape[-1]
    rows = w.numel() // K if K else 0
    _require(K % group_size == 0 and group_size % (32 // bits) == 0, _lib.EINVAL_SHAPE,
             f"quantize: group size {group_size} incompatible with K={K}, bits={bits}")
    wq = torch.empty(*w.shape[:-1], K * bits // 32, dtype=torch.int32, device=w.device)
    sc = torch.empty(*w.shape[:-1], K // group_size, dtype=w.dtype, device=w.device)
    bi = torch.empty_like(sc)
    dt = _lib.DTYPE_BF16 if w.dtype == torch.bfloat16 else _lib.DTYPE_F32
    _lib.call("lisaq_quantize", _stream(w), w.data_ptr(), dt, wq.data_ptr(), sc.data_ptr(), bi.data_ptr(),
              rows, K, group_size, bits)
    return wq, sc, bi


def moe_route(logits: torch.Tensor, k: int):
    """Top-k (stable, descending) + softmax over the selected (moe.rs:352-359)."""
    _require(logits.dtype == torch.float32, _lib.EINVAL_DTYPE, "moe_route: logits must be float32")
    logits = logits.contiguous()
    E = logits.shape[-1]
    T = logits.numel() // E
    idx = torch.empty(*logits.shape[:-1], k, dtype=torch.int32, device=logits.device)
    wts = torch.empty(*logits.shape[:-1], k, dtype=torch.float32, device=logits.device)
    _lib.call("lisaq_moe_route", _stream(logits), logits.data_ptr(), T, E, k, idx.data_ptr(), wts.data_ptr())
    return idx, wts


def moe_sort(idx_flat: torch.Tensor, num_experts: int, top_k: int):
    """(sorted_idx, order, token_rows, inverse, expert_offsets) of the routed slots (moe.rs:364-374)."""
    ids = idx_flat.reshape(-1).to(torch.int32).contiguous()
    R = ids.numel()
    dev = ids.device
    outs = [torch.empty(R, dtype=torch.int32, device=dev) for _ in range(4)]
    offs = torch.empty(num_experts + 1, dtype=torch.int32, device=dev)
    _lib.call("lisaq_moe_sort", _stream(ids), ids.data_ptr(), R, num_experts, top_k,
              *[o.data_ptr() for o in outs], offs.data_ptr())
    return (*outs, offs)


def gather_rows(x: torch.Tensor, rows: torch.Tensor) -> torch.Tensor:
    x = _bf16(x, "x")
    rows = rows.to(torch.int32).contiguous()
    H = x.shape[-1]
    out = torch.empty(rows.numel(), H, dtype=torch.bfloat16, device=x.device)
    _lib.call("lisaq_gather_rows", _stream(x), x.data_ptr(), rows.data_ptr(), out.data_ptr(), rows.numel(), H)
    return out


def swiglu(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    gate = _bf16(gate, "gate")
    up = _bf16(up, "up")
    _require(gate.shape == up.shape, _lib.EINVAL_SHAPE, "swiglu: shape mismatch")
    out = torch.empty_like(gate)
    _lib.call("lisaq_swiglu", _stream(gate), gate.data_ptr(), up.data_ptr(), out.data_ptr(), gate.numel())
    return out


def gather_qmm_swiglu(x, x_rows, gate, up, rhs_indices, group_size=64, bits=4) -> torch.Tensor:
    """SwiGLU of the gate and up ``gather_qmm`` over expert-sorted rows in one launch (moe.rs:373-413):
    row r is ``x[x_rows[r]]`` (``x`` ``[T, H]``), ``rhs_indices`` ``[R]`` sorted expert ids, ``gate`` /
    ``up`` ``(w, scales, biases)`` stacks ``[E, I, H*bits/32]`` -> act ``[R, I]``.  Every run uses the
    matmul arithmetic (runs of at least ``qmv_batch_limit(H, I)`` rows are bitwise equal to
    ``swiglu(gather_qmm(gate), gather_qmm(up))``)."""
    x = _bf16(x, "x")
    rows = x_rows.to(torch.int32).contiguous()
    rhs = rhs_indices.to(torch.int32).contiguous()
    gw, gsc, gbi = _u32(gate[0], "gate w"), _bf16(gate[1], "gate scales"), _bf16(gate[2], "gate biases")
    uw, usc, ubi = _u32(up[0], "up w"), _bf16(up[1], "up scales"), _bf16(up[2], "up biases")
    _require(x.dim() == 2, _lib.EINVAL_SHAPE, f"gather_qmm_swiglu: x {tuple(x.shape)} must be [T, H]")
    T, H = x.shape
    R = rows.numel()
    _require(rhs.numel() == R, _lib.EINVAL_SHAPE, f"gather_qmm_swiglu: {rhs.numel()} indices for {R} rows")
    _require(gw.dim() == 3 and gw.shape[2] * 32 // bits == H and uw.shape == gw.shape, _lib.EINVAL_SHAPE,
             f"gather_qmm_swiglu: gate {tuple(gw.shape)} / up {tuple(uw.shape)} do not match H={H}, bits={bits}")
    E, I = gw.shape[0], gw.shape[1]
    for t in (gsc, gbi, usc, ubi):
        _require(t.shape == (E, I, H // group_size), _lib.EINVAL_SHAPE, "gather_qmm_swiglu: scales/biases shape mismatch")
    act = torch.empty(R, I, dtype=torch.bfloat16, device=x.device)
    nbytes = _lib.load().lisaq_gather_qmm_swiglu_workspace(R, I, E)
    ws = workspace(x.device, nbytes, "moe")
    _lib.call("lisaq_gather_qmm_swiglu", _stream(x), x.data_ptr(), rows.data_ptr(), rhs.data_ptr(), gw.data_ptr(),
              gsc.data_ptr(), gbi.data_ptr(), uw.data_ptr(), usc.data_ptr(), ubi.data_ptr(), act.data_ptr(), R, T,
              I, H, E, group_size, bits, ws.data_ptr(), ws.numel())
    return act


def moe_combine(down_sorted, weights, inverse, T: int, k: int) -> torch.Tensor:
    down_sorted = _bf16(down_sorted, "down_sorted")
    weights = weights.to(torch.float32).contiguous()
    inverse = inverse.to(torch.int32).contiguous()
    H = down_sorted.shape[-1]
    out = torch.empty(T, H, dtype=torch.bfloat16, device=down_sorted.device)
    _lib.call("lisaq_moe_combine", _stream(down_sorted), down_sorted.data_ptr(), weights.data_ptr(),
              inverse.data_ptr(), out.data_ptr(), T, k, H)
    return out


def moe_forward(x, logits, gate, up, down, top_k: int, group_size=64, bits=4, return_routing=False):
    """Routed SwitchGLU of ``SparseMoeBlock::forward``'s generic path (moe.rs:352-449).

    ``gate``/``up``/``down`` are ``(w, scales, biases)`` expert stacks
    ``[E, I, H*bits/32]`` / ``[E, H, I*bits/32]``."""
    x = _bf16(x, "x")
    H = x.shape[-1]
    T = x.numel() // H
    logits = logits.to(torch.float32).contiguous()
    E = logits.shape[-1]
    gw, gs_, gb = (_u32(gate[0], "gate_w"), _bf16(gate[1], "gate_s"), _bf16(gate[2], "gate_b"))
    uw, us_, ub = (_u32(up[0], "up_w"), _bf16(up[1], "up_s"), _bf16(up[2], "up_b"))
    dw, ds_, db = (_u32(down[0], "down_w"), _bf16(down[1], "down_s"), _bf16(down[2], "down_b"))
    I = gw.shape[1]
    _require(gw.shape == (E, I, H * bits // 32) and uw.shape == gw.shape, _lib.EINVAL_SHAPE,
             "moe_forward: gate/up stack shape")
    _require(dw.shape == (E, H, I * bits // 32), _lib.EINVAL_SHAPE, "moe_forward: down stack shape")
    out = torch.empty(*x.shape, dtype=torch.bfloat16, device=x.device)
    idx = torch.empty(T, top_k, dtype=torch.int32, device=x.device)
    wts = torch.empty(T, top_k, dtype=torch.float32, device=x.device)
    lib = _lib.load()
    # its own buffer: its first word is the fused decode's give-up flag (zero
    # unless a wait gave up), which no other op may write
    ws = workspace(x.device, lib.lisaq_moe_workspace(T, H, I, E, top_k, group_size, bits), "moe_forward")
    _lib.call("lisaq_moe_forward", _stream(x), x.data_ptr(), logits.data_ptr(),
              gw.data_ptr(), gs_.data_ptr(), gb.data_ptr(), uw.data_ptr(), us_.data_ptr(), ub.data_ptr(),
              dw.data_ptr(), ds_.data_ptr(), db.data_ptr(), out.data_ptr(), T, H, I, E, top_k,
              group_size, bits, idx.data_ptr(), wts.data_ptr(), ws.data_ptr(), ws.numel())
    if return_routing:
        return out, idx, wts
    return out
