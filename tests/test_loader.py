"""safetensors reader and packed-layout validation (loader.rs:57-150,
quant.rs:273-287, 408-428) on the CPU, and the engine layers built on it
(QuantizedLinear, QuantizedEmbedding, SwitchGlu) on the GPU."""
import json
import struct

import numpy as np
import pytest

from lisa_amd.loader import Shard, ShardError, write_safetensors
from lisa_amd.synth import np_linear, np_x


def _write_raw(path, header_obj, payload=b""):
    hb = json.dumps(header_obj).encode()
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(hb)))
        f.write(hb)
        f.write(payload)


def test_round_trip(tmp_path):
    rng = np.random.default_rng(0)
    w, s, b = np_linear(rng, 32, 256)
    p = str(tmp_path / "m.safetensors")
    write_safetensors(p, {"layer.q.weight": ("U32", w), "layer.q.scales": ("BF16", s), "layer.q.biases": ("BF16", b)},
                      metadata={"format": "mlx"})
    sh = Shard(p)
    assert set(sh.names()) == {"layer.q.weight", "layer.q.scales", "layer.q.biases"}
    assert np.array_equal(sh.numpy("layer.q.weight"), w)
    assert np.array_equal(sh.numpy("layer.q.scales"), s)
    sh.close()


def test_language_model_prefix(tmp_path):
    p = str(tmp_path / "m.safetensors")
    write_safetensors(p, {"language_model.a.weight": ("U32", np.arange(8, dtype=np.uint32).reshape(2, 4))})
    sh = Shard(p)
    assert sh.numpy("a.weight").tolist() == [[0, 1, 2, 3], [4, 5, 6, 7]]
    with pytest.raises(KeyError):
        sh.numpy("b.weight")


@pytest.mark.parametrize("header,payload,msg", [
    ([1, 2], b"", "must be an object"),
    ({"t": {"dtype": "Q4", "shape": [1], "data_offsets": [0, 1]}}, b"\0", "unsupported dtype"),
    ({"t": {"dtype": "U8", "data_offsets": [0, 1]}}, b"\0", "missing shape"),
    ({"t": {"dtype": "U8", "shape": [-1], "data_offsets": [0, 1]}}, b"\0", "invalid dimension"),
    ({"t": {"dtype": "U8", "shape": [2]}}, b"\0\0", "missing data_offsets"),
    ({"t": {"dtype": "U8", "shape": [2], "data_offsets": [0]}}, b"\0\0", "two entries"),
    ({"t": {"dtype": "U8", "shape": [2], "data_offsets": [0, 9]}}, b"\0\0", "payload bounds"),
    ({"t": {"dtype": "U32", "shape": [2], "data_offsets": [0, 4]}}, b"\0" * 8, "byte size differs"),
])
def test_header_rejections(tmp_path, header, payload, msg):
    p = str(tmp_path / "bad.safetensors")
    _write_raw(p, header, payload)
    with pytest.raises(ShardError, match=msg):
        Shard(p)


def test_truncated_and_oversized(tmp_path):
    p = str(tmp_path / "tiny.safetensors")
    open(p, "wb").write(b"\1\2\3")
    with pytest.raises(ShardError, match="too small"):
        Shard(p)
    open(p, "wb").write(struct.pack("<Q", 1 << 40) + b"{}")
    with pytest.raises(ShardError, match="invalid or oversized"):
        Shard(p)


def test_check_layout_and_group_size():
    from lisa_amd import _lib
    from lisa_amd.quant import check_layout

    assert check_layout((17408, 640), (17408, 80), (17408, 80), 4) == (5120, 64)
    assert check_layout((64, 32), (64, 8), (64, 8), 4) == (256, 32)  # smoke.rs gs 32
    assert check_layout((5120, 1088), (5120, 272), (5120, 272), 2) == (17408, 64)
    with pytest.raises(_lib.LisaqError):
        check_layout((10, 640), (10, 80), (9, 80), 4)


@pytest.mark.gpu
def test_quantized_linear_from_shard(dev, oracle, tmp_path):
    import torch

    from lisa_amd.quant import QuantizedEmbedding, QuantizedLinear
    from tests._util import assert_close_bf16, from_dev_bf16, to_dev, to_dev_bf16

    rng = np.random.default_rng(3)
    N, K = 300, 1024
    w, s, b = np_linear(rng, N, K, 4, 32)
    p = str(tmp_path / "m.safetensors")
    write_safetensors(p, {"mlp.up_proj.weight": ("U32", w), "mlp.up_proj.scales": ("BF16", s),
                          "mlp.up_proj.biases": ("BF16", b)})
    lin = QuantizedLinear.load(Shard(p), "mlp", "up_proj", device=dev)
    assert lin.group_size == 32 and lin.dims_out() == N
    x = np_x(rng, 6, K)
    y = lin(to_dev_bf16(x, dev).reshape(2, 3, K))
    assert tuple(y.shape) == (2, 3, N)
    assert_close_bf16(from_dev_bf16(y.reshape(6, N)), oracle.qmv(x, w, s, b, 32, 4), what="QuantizedLinear")
    ys = lin.forward_serial_rows(to_dev_bf16(x[:4], dev).reshape(4, 1, K))
    for r in range(4):
        one = lin(to_dev_bf16(x[r:r + 1], dev))
        assert np.array_equal(from_dev_bf16(ys[r]), from_dev_bf16(one))
    emb = QuantizedEmbedding(lin.weight, lin.scales, lin.biases, 32, 4)
    ids = np.array([[5, 0], [299, 5]], np.int32)
    got = from_dev_bf16(emb.forward(to_dev(ids, dev)))
    ref = oracle.f32_to_bf16(oracle.dequantize(w, s, b, 32, 4))[ids]
    assert np.array_equal(got, ref)
    torch.cuda.synchronize()


@pytest.mark.gpu
def test_switch_glu_from_shard(dev, oracle, tmp_path):
    from lisa_amd import ops
    from lisa_amd.moe import SwitchGlu
    from tests._util import from_dev_bf16, to_dev, to_dev_bf16

    rng = np.random.default_rng(4)
    E, H, I, k, T = 8, 256, 128, 2, 5

    def stack(N, K):
        parts = [np_linear(rng, N, K) for _ in range(E)]
        return [np.stack([p[i] for p in parts]) for i in range(3)]

    g, u, d = stack(I, H), stack(I, H), stack(H, I)
    tensors = {}
    for key, st in (("gate_proj", g), ("up_proj", u), ("down_proj", d)):
        tensors[f"moe.switch_mlp.{key}.weight"] = ("U32", st[0])
        tensors[f"moe.switch_mlp.{key}.scales"] = ("BF16", st[1])
        tensors[f"moe.switch_mlp.{key}.biases"] = ("BF16", st[2])
    p = str(tmp_path / "moe.safetensors")
    write_safetensors(p, tensors)
    sw = SwitchGlu.load(Shard(p), "moe.switch_mlp", device=dev)
    x = np_x(rng, T, H)
    lg = rng.standard_normal((T, E)).astype(np.float32)
    out = sw(to_dev_bf16(x, dev), to_dev(lg, dev), k)
    ref = ops.moe_forward(to_dev_bf16(x, dev), to_dev(lg, dev), sw.gate.triple(), sw.up.triple(), sw.down.triple(), k)
    assert np.array_equal(from_dev_bf16(out), from_dev_bf16(ref))
