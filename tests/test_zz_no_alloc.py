"""lisaq_quantized_matmul_noalloc (split-K partials in the library's device
scratch, no workspace argument) against lisaq_quantized_matmul with a caller
workspace: bitwise equal (the same kernels and split), on two calls in a row,
the second one smaller, at shapes whose split uses the scratch (the matmul's
hybrid split at M=2048 x 17408 x 5120 -- the full 64 MiB --, its small-grid
split at M=128 x 5120 x 17408, the streaming matvec's split) and at shapes
that use none."""
import numpy as np
import pytest

from lisa_amd import _lib, ops
from lisa_amd.synth import np_linear, np_x
from tests._util import from_dev_bf16, to_dev_bf16, to_dev_u32

pytestmark = pytest.mark.gpu


def _pair(dev, M, N, K, bits=4, gs=64, seed=0):
    import torch

    rng = np.random.default_rng(seed + M + N + K)
    w, s, b = np_linear(rng, N, K, bits, gs)
    x = np_x(rng, M, K)
    xd, wd, sd, bd = to_dev_bf16(x, dev), to_dev_u32(w, dev), to_dev_bf16(s, dev), to_dev_bf16(b, dev)
    st = torch.cuda.current_stream().cuda_stream
    lib = _lib.load()
    need = lib.lisaq_quantized_matmul_workspace(M, N, K, gs, bits)
    ws = ops.workspace(dev, need)
    y_ws = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
    _lib.call("lisaq_quantized_matmul", st, xd.data_ptr(), wd.data_ptr(), sd.data_ptr(), bd.data_ptr(),
              y_ws.data_ptr(), M, N, K, 1, gs, bits, ws.data_ptr(), ws.numel())
    y_na = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
    _lib.call("lisaq_quantized_matmul_noalloc", st, xd.data_ptr(), wd.data_ptr(), sd.data_ptr(), bd.data_ptr(),
              y_na.data_ptr(), M, N, K, 1, gs, bits)
    torch.cuda.synchronize()
    assert np.array_equal(from_dev_bf16(y_na), from_dev_bf16(y_ws)), (M, N, K, bits, need)
    return need


@pytest.mark.parametrize("first,second", [
    ((2048, 17408, 5120), (128, 5120, 17408)),   # hybrid split (64 MiB), then the small-grid split
    ((128, 5120, 17408), (70, 300, 1024)),       # small-grid split, then a smaller one
    ((8, 2560, 9728), (4, 2560, 9728)),          # streaming matvec split, then the one-stream kernel
    ((1, 17408, 5120), (1, 3072, 1024)),         # no scratch at all
])
def test_noalloc_matches_workspace_entry(dev, first, second):
    n1 = _pair(dev, *first)
    n2 = _pair(dev, *second, seed=1)
    if first[0] >= 128:
        assert n1 > 0  # the first call of each split pair really uses the scratch


def test_noalloc_rejects_like_the_workspace_entry(dev):
    import torch

    with pytest.raises(_lib.LisaqError, match="transpose"):
        _lib.call("lisaq_quantized_matmul_noalloc", 0, 16, 16, 16, 16, 16, 1, 64, 128, 0, 64, 4)
    torch.cuda.synchronize()
