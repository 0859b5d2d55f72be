"""Benchmark of the MLX affine quantized linear on one MI355X.

Headline (``value``): 4-bit qmv at M=1, K=5120, N=17408, group 64 -- the
north-star decode matvec -- in GB/s of algorithmic bytes (packed W + scales +
biases + x + y, once each: 50,180,096 B per call) over whole-job time.  A
step is one quantized_matmul call on one of 8 distinct weight sets used in
rotation (8 x 50.2 MB = 401 MB > the 256 MB Infinity Cache), so weights
stream from HBM.  Inputs are resident in HBM before the timed region; the K
timed steps are replayed from a HIP graph so host launch overhead is not
timed, and the device's own clock, stored by a one-lane launch inside the
graph before the first and after the last step, times them (the hipEvent
bracket around the replay, which also holds the replay's start-up on the
device, is reported beside it as ``event_ms_per_step``).  The qmm figure (M=2048, TFLOP/s of 2*M*N*K) is reported beside it.

``cpu_baseline`` times the CPU oracle's fused dequant-dot (the reference's
dequantize-then-matmul arithmetic, oracle/lisaq_oracle.c) on the host cores
over a bounded number of calls of the same shape; its ``materialize`` entry
times the literal chain (W dequantized to f32, then an f32 product).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, GB/s
CLOCK_WARM_S = 0.03  # sustained load before any timed region (steady shader clock)
BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 MFMA, TFLOP/s
METRIC = "4-bit qmv GB/s (% HBM peak) @M=1; qmm TFLOP/s (% bf16 MFMA peak) @M=2048"


# HBM bytes per launch measured with rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE on this workload, each
# scaled by the counter's reading for a 64 MiB device copy (see the profiles/ summaries for the
# commands and raw counts).
QMV_TRAFFIC_BYTES = round((24576.5 * 1.9993 + 136.0) * 1024)
QMM_TRAFFIC_BYTES = round((243697.5 * 1.9993 + 131780.5) * 1024)
QMV_KERNEL = "lisaq::qmvp_kernel<4, 64, 3, 2, 16, 1, false>"
QMM_KERNEL = "lisaq::qmm_kernel<4, 64, 8, 1, 8, true, false, 3, false, 1>"  # M=2048: 256-row tiles, last round split over K (+ qmm_hybrid_reduce_kernel)


def qmv_bytes(M, N, K, bits=4, gs=64):
    return N * K * bits // 8 + 2 * 2 * N * (K // gs) + 2 * M * K + 2 * M * N


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400)
    ap.add_argument("--warmup", type=int, default=40)
    ap.add_argument("--qmm-steps", type=int, default=20)
    ap.add_argument("--sets", type=int, default=8)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-qmm", action="store_true")
    ap.add_argument("--no-table", action="store_true", help="skip the per-configuration table")
    ap.add_argument("--calibrate", action="store_true",
                    help="only run a plain 64 MiB device copy (the reference kernel for the HBM byte counters)")
    ap.add_argument("--blaslt", action="store_true",
                    help="only compare the prefill matmul with dequantize-then-hipBLASLt bf16 GEMM on the same shapes")
    ap.add_argument("--moe", action="store_true",
                    help="only time the MoE block rows (T=1, 64, 4096) of the configuration table")
    ap.add_argument("--moe-tokens", type=int, nargs="*", default=None,
                    help="with --moe: only these of the MoE rows' token counts (1, 64, 4096)")
    ap.add_argument("--read-floor", action="store_true",
                    help="only time read-only streams of the configuration rows' byte counts (lisaq_read_stream): "
                         "the floor a kernel reading those bytes reaches in the same graph replay")
    ap.add_argument("--addnorm", action="store_true",
                    help="only time the residual add + RMSNorm matvec against the plain matvec at the north-star shape")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py: this build runs on one GPU only (no multi-GPU path); use --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch

    from lisa_amd import ops
    from lisa_amd.synth import torch_linear, torch_x

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.calibrate:
        src = torch.empty(64 << 20, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        for _ in range(20):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"calibration": "device copy", "bytes_read": src.numel(), "bytes_written": dst.numel(),
                          "calls": 20}), flush=True)
        return
    gen = torch.Generator(device=dev)
    gen.manual_seed(0x5EED + 1)
    if args.blaslt:
        blaslt_compare(dev, gen)
        return
    if args.addnorm:
        addnorm_compare(dev, gen)
        return
    if args.read_floor:
        for r in read_floor(dev):
            print(json.dumps(r), flush=True)
        return
    if args.moe:
        for r in moe_rows(dev, gen, torch.cuda.Stream(), args.moe_tokens):
            print(json.dumps(r), flush=True)
        return
    M, N, K, bits, gs = 1, 17408, 5120, 4, 64

    # --- qmv: cold-stream rotation over distinct weight sets ------------------
    sets = [torch_linear(N, K, bits, gs, device=dev, generator=gen) for _ in range(args.sets)]
    x = torch_x(M, K, device=dev, generator=gen)
    stream = torch.cuda.Stream()
    torch.cuda.synchronize()

    def step(i):
        w, s, b = sets[i % len(sets)]
        return ops.quantized_matmul(x, w, s, b, True, gs, bits)

    with torch.cuda.stream(stream):
        for i in range(len(sets)):  # eager pass over every weight set (also allocates the workspace)
            step(i)
    stream.synchronize()

    from lisa_amd import _lib

    lib = _lib.load()
    stamps = torch.zeros(2, dtype=torch.int64, device=dev)

    def capture(n, stamped=False):
        # stamped: the GPU's 100 MHz clock stored right before the first and
        # right after the last step, inside the graph (the replay's start on
        # the device, a few us per replay, stays outside; it is in the event
        # bracket, reported beside)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            if stamped:
                _lib.check(lib.lisaq_timestamp(stream.cuda_stream, stamps.data_ptr()))
            for i in range(n):
                step(i)
            if stamped:
                _lib.check(lib.lisaq_timestamp(stream.cuda_stream, stamps.data_ptr() + 8))
        return g

    # W untimed warm-up steps, replayed from a graph like the timed ones, then
    # replays of the same graph until the GPU has run this load for at least
    # CLOCK_WARM_S (it reaches its steady clock after ~20 ms of sustained load;
    # a handful of calls is ~0.1 ms and leaves it ramping)
    g_warm = capture(max(args.warmup, 1))
    g_timed = capture(args.steps, stamped=True)
    t_w = time.perf_counter()
    warm_replays = 0
    while warm_replays < 1 or time.perf_counter() - t_w < CLOCK_WARM_S:
        with torch.cuda.stream(stream):
            g_warm.replay()
        torch.cuda.synchronize()
        warm_replays += 1
    # the timed graph's own first replay (a new graph's first replay runs slow)
    # also stays untimed
    with torch.cuda.stream(stream):
        g_timed.replay()
    torch.cuda.synchronize()

    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    with torch.cuda.stream(stream):
        e0.record(stream)
        g_timed.replay()
        e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    event_ms = e0.elapsed_time(e1)
    t_stamp = stamps.cpu().tolist()
    gpu_ms = (t_stamp[1] - t_stamp[0]) * 1e-5  # 100 MHz ticks
    per_step_s = gpu_ms * 1e-3 / args.steps
    nbytes = qmv_bytes(M, N, K, bits, gs)
    gbs = nbytes / per_step_s / 1e9

    # --- qmm: prefill M=2048, timed like the configuration rows (graph replay
    # after >= CLOCK_WARM_S of replays of the same graph) -------------------------
    Mq = 2048
    wq = sets[0]
    xq = torch_x(Mq, K, device=dev, generator=gen)
    qmm_s = float("nan")
    if not args.no_qmm:
        qmm_s = _time_graph(stream, lambda i: ops.quantized_matmul(xq, *wq, True, gs, bits), 1, args.qmm_steps,
                            warm_s=CLOCK_WARM_S)
    flops = 2.0 * Mq * N * K
    tflops = flops / qmm_s / 1e12

    # --- the other measured configurations (parity cases of the same path) ----
    table = [] if args.no_table else config_table(dev, gen, stream)

    # --- CPU baseline (oracle fused dequant-dot, same shape, bounded sample) ---
    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(M, N, K, bits, gs, args.cpu_seconds)

    out = {
        "metric": METRIC,
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(per_step_s * 1e3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "qmv 4-bit gs64 M=1 K=5120 N=17408 (decode matvec), 8 rotating weight sets",
            "bits": bits, "group_size": gs, "M": M, "K": K, "N": N, "weight_sets": len(sets),
            "bytes_per_step": nbytes,
            "timing": f"HIP graph replay of the timed steps, device clock (lisaq_timestamp) stored inside the "
                      f"graph before the first and after the last step, after the W warm-up steps and "
                      f"{warm_replays} replays of them ({CLOCK_WARM_S * 1e3:.0f} ms of clock warm-up) and one "
                      f"untimed replay of the timed graph",
            "event_ms_per_step": round(event_ms / args.steps, 5),
            "wall_s": round(wall, 4),
        },
        "roofline": {
            "bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": QMV_TRAFFIC_BYTES,
            "kernel": QMV_KERNEL, "bytes_per_launch": nbytes,
            "avg_launch_us": round(per_step_s * 1e6, 3),
        },
        "qmm": {
            "workload": "qmm 4-bit gs64 M=2048 K=5120 N=17408 (prefill)",
            "value": round(tflops, 1), "unit": "TFLOP/s", "ms_per_call": round(qmm_s * 1e3, 4),
            "roofline": {"bound": "mfma", "achieved": round(tflops, 1), "peak": BF16_PEAK_TFLOPS,
                         "unit": "TFLOP/s", "frac": round(tflops / BF16_PEAK_TFLOPS, 4),
                         "traffic": QMM_TRAFFIC_BYTES, "kernel": QMM_KERNEL},
        },
        "cpu_baseline": cpu,
        "configs": table,
    }
    print(json.dumps(out), flush=True)


def _time_graph(stream, fn, n_sets, steps, warm_s=CLOCK_WARM_S):
    """Average seconds per call of fn(i) over `steps` calls replayed from a HIP graph (i cycles
    over n_sets inputs), after untimed replays of the same graph for at least `warm_s` seconds
    (steady clock; the first replays of a new graph over new buffers run slow).  Timed by the
    device clock stored inside the graph before the first and after the last call
    (lisaq_timestamp), as the headline."""
    import torch

    from lisa_amd import _lib

    lib = _lib.load()
    stamps = torch.zeros(2, dtype=torch.int64, device=stream.device)

    # inputs were made on the current stream; the calls below share library
    # workspaces with any eager call still queued there
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for i in range(n_sets):
            fn(i)
    stream.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        _lib.check(lib.lisaq_timestamp(stream.cuda_stream, stamps.data_ptr()))
        for i in range(steps):
            fn(i)
        _lib.check(lib.lisaq_timestamp(stream.cuda_stream, stamps.data_ptr() + 8))
    t0 = time.perf_counter()
    reps = 0
    while reps < 2 or time.perf_counter() - t0 < warm_s:
        with torch.cuda.stream(stream):
            g.replay()
        torch.cuda.synchronize()
        reps += 1
    with torch.cuda.stream(stream):
        g.replay()
    torch.cuda.synchronize()
    del g
    t = stamps.cpu().tolist()
    return (t[1] - t[0]) * 1e-8 / steps  # 100 MHz ticks


def read_floor(dev):
    """Read-only streams (lisaq_read_stream: 16-byte nontemporal loads, 1 KB per wave instruction) of the
    byte counts of the decode rows, over as many rotating buffers as those rows use (> 256 MB, cold), and an
    empty launch (0 bytes read by one workgroup): per-call time in the same graph replay as the matvec."""
    import torch

    from lisa_amd import _lib

    lib = _lib.load()
    stream = torch.cuda.Stream()
    sink = torch.zeros(4, dtype=torch.int32, device=dev)
    rows = []
    for name, nb, sets in (("configs[1] decode, 4-bit M=1 (9728x2560 / 2560x9728)", qmv_bytes(1, 9728, 2560), 24),
                           ("2-bit north-star / down shape, M=1", qmv_bytes(1, 17408, 5120, 2), 15),
                           ("north star 4-bit M=1", qmv_bytes(1, 17408, 5120), 8)):
        nb16 = nb // 16 * 16
        bufs = [torch.ones(nb16, dtype=torch.uint8, device=dev) for _ in range(sets)]
        for L in (1, 2, 4, 8, 16):
            t = _time_graph(stream, lambda i: _lib.check(lib.lisaq_read_stream(
                torch.cuda.current_stream().cuda_stream, bufs[i % sets].data_ptr(), nb16, L, sink.data_ptr())),
                sets, 300)
            rows.append({"workload": f"read-only stream, {name}", "bytes": nb16, "loads_per_lane": L,
                         "us": round(t * 1e6, 2), "GB/s": round(nb16 / t / 1e9, 1),
                         "frac": round(nb16 / t / 1e9 / HBM_PEAK_GBS, 4), "buffers": sets})
        del bufs
    one = torch.ones(4096, dtype=torch.uint8, device=dev)
    t = _time_graph(stream, lambda i: _lib.check(lib.lisaq_read_stream(
        torch.cuda.current_stream().cuda_stream, one.data_ptr(), 16, 1, sink.data_ptr())), 1, 300)
    rows.append({"workload": "one-workgroup launch reading 16 bytes (the per-launch floor)", "us": round(t * 1e6, 2)})
    return rows


def addnorm_compare(dev, gen):
    """lisaq_qmv_addnorm (add + RMSNorm launch, then the matvec) against the plain matvec, 4-bit M=1
    K=5120 N=17408, 8 rotating weight sets, graph-replayed.  One JSON line."""
    import torch

    from lisa_amd import ops
    from lisa_amd.synth import torch_linear, torch_x

    N, K, n_sets = 17408, 5120, 8
    stream = torch.cuda.Stream()
    sets = [torch_linear(N, K, 4, 64, device=dev, generator=gen) for _ in range(n_sets)]
    x = torch_x(1, K, device=dev, generator=gen)
    r = torch_x(1, K, device=dev, generator=gen)
    nw = torch.ones(K, dtype=torch.bfloat16, device=dev)
    t_q = _time_graph(stream, lambda i: ops.quantized_matmul(x, *sets[i % n_sets], True, 64, 4), n_sets, 400)
    t_a = _time_graph(stream, lambda i: ops.qmv_addnorm(x, r, nw, *sets[i % n_sets], 1e-6), n_sets, 400)
    print(json.dumps({"workload": "qmv 4-bit gs64 M=1 K=5120 N=17408", "qmv_us": round(t_q * 1e6, 2),
                      "addnorm_qmv_us": round(t_a * 1e6, 2)}), flush=True)


def blaslt_compare(dev, gen):
    """The prefill matmul against the unfused alternative on the same inputs: W dequantized to
    bf16 by lisaq_dequantize (bf16(s*q+b), the values the fused kernel feeds its matrix cores),
    then torch.matmul (hipBLASLt) on the bf16 operands.  One JSON line per shape."""
    import torch

    from lisa_amd import ops
    from lisa_amd.synth import torch_linear, torch_x

    stream = torch.cuda.Stream()
    for M, N, K in [(2048, 17408, 5120), (2048, 5120, 17408), (512, 17408, 5120), (128, 17408, 5120)]:
        w, s, b = torch_linear(N, K, 4, 64, device=dev, generator=gen)
        x = torch_x(M, K, device=dev, generator=gen)
        wd = ops.dequantize(w, s, b, 64, 4)
        fl = 2.0 * M * N * K
        t_q = _time_graph(stream, lambda i: ops.quantized_matmul(x, w, s, b, True, 64, 4), 1, 10)
        t_b = _time_graph(stream, lambda i: torch.matmul(x, wd.t()), 1, 10)
        t_d = _time_graph(stream, lambda i: ops.dequantize(w, s, b, 64, 4), 1, 10)
        y_q = ops.quantized_matmul(x, w, s, b, True, 64, 4).float()
        y_b = torch.matmul(x, wd.t()).float()
        print(json.dumps({"M": M, "N": N, "K": K, "fused_qmm_us": round(t_q * 1e6, 1),
                          "fused_qmm_tflops": round(fl / t_q / 1e12, 1), "blaslt_bf16_us": round(t_b * 1e6, 1),
                          "blaslt_bf16_tflops": round(fl / t_b / 1e12, 1), "dequantize_us": round(t_d * 1e6, 1),
                          "dequantize_then_blaslt_tflops": round(fl / (t_b + t_d) / 1e12, 1),
                          "max_abs_diff": (y_q - y_b).abs().max().item(),
                          "max_abs_y": y_b.abs().max().item()}), flush=True)
        del w, s, b, x, wd, y_q, y_b


def config_table(dev, gen, stream):
    """Every measured configuration of the path (BASELINE configs [1]-[4]), cold weights:
    distinct weight sets in rotation so more than the 256 MB Infinity Cache is streamed."""
    import torch

    from lisa_amd import ops
    from lisa_amd.synth import torch_linear, torch_x

    rows = []
    gs = 64

    def qmv_row(name, M, N, K, bits, n_sets, steps=200):
        sets = [torch_linear(N, K, bits, gs, device=dev, generator=gen) for _ in range(n_sets)]
        x = torch_x(M, K, device=dev, generator=gen)
        t = _time_graph(stream, lambda i: ops.quantized_matmul(x, *sets[i % n_sets], True, gs, bits), n_sets, steps)
        nb = qmv_bytes(M, N, K, bits, gs)
        rows.append({"workload": name, "M": M, "N": N, "K": K, "bits": bits, "us": round(t * 1e6, 2),
                     "value": round(nb / t / 1e9, 1), "unit": "GB/s", "frac": round(nb / t / 1e9 / HBM_PEAK_GBS, 4),
                     "bytes_per_call": nb, "weight_sets": n_sets})
        del sets

    def qmm_row(name, M, N, K, bits, steps=10):
        w = torch_linear(N, K, bits, gs, device=dev, generator=gen)
        x = torch_x(M, K, device=dev, generator=gen)
        t = _time_graph(stream, lambda i: ops.quantized_matmul(x, *w, True, gs, bits), 1, steps)
        fl = 2.0 * M * N * K
        rows.append({"workload": name, "M": M, "N": N, "K": K, "bits": bits, "us": round(t * 1e6, 1),
                     "value": round(fl / t / 1e12, 1), "unit": "TFLOP/s",
                     "frac": round(fl / t / 1e12 / BF16_PEAK_TFLOPS, 4)})

    # [1] decode: up 9728x2560 and down 2560x9728 (14 MB each; 20 sets), M = 1, 2, 4, 8
    for M in (1, 2, 4, 8):
        qmv_row("decode up 4-bit", M, 9728, 2560, 4, 20)
        qmv_row("decode down 4-bit", M, 2560, 9728, 4, 20)
    # north-star shape at M = 2, 4, 8 (8 sets)
    for M in (2, 4, 8):
        qmv_row("north-star shape 4-bit", M, 17408, 5120, 4, 8)
    # [3] 2-bit decode
    qmv_row("decode 2-bit", 1, 17408, 5120, 2, 10)
    qmv_row("decode 2-bit down", 1, 5120, 17408, 2, 10)
    # [2] prefill: up 17408x5120 and down 5120x17408, M = 128, 512, 2048; [3] 2-bit M = 512
    for M in (128, 512, 2048):
        qmm_row("prefill up 4-bit", M, 17408, 5120, 4)
        qmm_row("prefill down 4-bit", M, 5120, 17408, 4)
    qmm_row("prefill up 2-bit", 512, 17408, 5120, 2)
    qmm_row("prefill down 2-bit", 512, 5120, 17408, 2)
    rows += moe_rows(dev, gen, stream)
    return rows


def moe_rows(dev, gen, stream, only=None):
    """The MoE block rows (BASELINE config [4]): E=128, k=8, H=2048, I=768, 4-bit gs64; T=1 with rotating
    router logits (different experts each call), T=64 (the matvec path between decode and prefill; bytes:
    the weights of the experts the call routes to, each read once) and T=4096."""
    import torch

    from lisa_amd import ops
    from lisa_amd.synth import torch_linear, torch_x

    rows = []
    gs = 64
    # [4] MoE: E=128, k=8, H=2048, I=768 (gate/up/down stacks, 340 MB); T=1 with rotating logits
    # (different experts each call), T=4096
    E, k, H, I = 128, 8, 2048, 768
    gate = torch_linear(I, H, 4, gs, device=dev, generator=gen, experts=E)
    up = torch_linear(I, H, 4, gs, device=dev, generator=gen, experts=E)
    down = torch_linear(H, I, 4, gs, device=dev, generator=gen, experts=E)
    for T, n_logits, steps in ((1, 32, 100), (64, 8, 40), (4096, 1, 5)):
        if only and T not in only:
            continue
        x = torch_x(T, H, device=dev, generator=gen)
        logits = [torch.randn(T, E, device=dev, generator=gen) for _ in range(n_logits)]
        t = _time_graph(stream, lambda i: ops.moe_forward(x, logits[i % n_logits], gate, up, down, k), n_logits, steps)
        per_expert = 3 * (I * H // 2 + 2 * 2 * I * (H // gs))  # packed W + scales + biases of one expert's 3 matrices
        if T <= 64:
            # distinct experts per call, averaged over the logit sets
            used = sum(int(torch.unique(ops.moe_route(lg, k)[0]).numel()) for lg in logits) / n_logits
            nb = int(round(used * per_expert))
            rows.append({"workload": "MoE 4-bit E=128 k=8 (routed block: route, sort, gate|up + SwiGLU, down, combine)", "T": T,
                         "us": round(t * 1e6, 2), "value": round(nb / t / 1e9, 1), "unit": "GB/s",
                         "frac": round(nb / t / 1e9 / HBM_PEAK_GBS, 4), "bytes_per_call": nb})
        else:
            fl = 2.0 * T * k * (2 * I * H + H * I)
            rows.append({"workload": "MoE 4-bit E=128 k=8 (routed block: route, sort, gate|up + SwiGLU, down, combine)", "T": T,
                         "us": round(t * 1e6, 1), "value": round(fl / t / 1e12, 1), "unit": "TFLOP/s",
                         "frac": round(fl / t / 1e12 / BF16_PEAK_TFLOPS, 4)})
    return rows


def cpu_baseline(M, N, K, bits, gs, seconds):
    """Oracle on host threads over a bounded number of calls, two ways: the
    fused dequant-dot (``value``: each weight decoded and used once), and the
    reference's literal chain -- dequantize W to f32 (AO:56-83), then an f32
    matrix-vector product (numpy/BLAS) -- under ``materialize``."""
    import numpy as np

    from lisa_amd.synth import np_linear, np_x
    from oracle import oracle as O

    O.build()
    rng = np.random.default_rng(0x5EED)
    w, s, b = np_linear(rng, N, K, bits, gs)
    x = np_x(rng, M, K)
    # every core this process may run on (the GPU box grants a share of the host's cores)
    host_cpus = os.cpu_count() or 1
    threads = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else host_cpus
    nbytes = qmv_bytes(M, N, K, bits, gs)

    def timed(fn, budget, min_calls=1):
        calls, t0 = 0, time.perf_counter()
        while True:
            fn()
            calls += 1
            el = time.perf_counter() - t0
            if el >= budget and calls >= min_calls:
                return calls, el

    calls, el = timed(lambda: O.qmv_threads(x, w, s, b, gs, bits, threads), seconds * 0.6)
    c1, e1 = timed(lambda: O.qmv_threads(x, w, s, b, gs, bits, 1), seconds * 0.2)
    xf = O.bf16_to_f32(x)
    cm, em = timed(lambda: xf @ O.dequantize(w, s, b, gs, bits).T, seconds * 0.2, min_calls=2)
    # the other M = 1 shapes BASELINE names: configs[0] and the configs[1] decode shapes (same threads)
    shapes = []
    for name, n_, k_ in (("configs[0] 3072x1024", 3072, 1024), ("configs[1] up 9728x2560", 9728, 2560),
                         ("configs[1] down 2560x9728", 2560, 9728)):
        w2, s2, b2 = np_linear(rng, n_, k_, 4, gs, s_floor=1e-3 if n_ == 3072 else 0.0)
        x2 = np_x(rng, 1, k_)
        nb2 = qmv_bytes(1, n_, k_, 4, gs)
        c2, e2 = timed(lambda: O.qmv_threads(x2, w2, s2, b2, gs, 4, threads), max(seconds * 0.1, 0.5), min_calls=3)
        shapes.append({"workload": name, "N": n_, "K": k_, "bits": 4, "M": 1, "cores": threads, "calls": c2,
                       "us_per_call": round(e2 / c2 * 1e6, 1), "value": round(nb2 * c2 / e2 / 1e9, 3), "unit": "GB/s"})
    return {
        "value": round(nbytes * calls / el / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
        "configs": shapes,
        "host_cpus": host_cpus, "single_thread_value": round(nbytes * c1 / e1 / 1e9, 3),
        "sample": f"{calls} calls of the same qmv shape (M={M} K={K} N={N} {bits}-bit) in {el:.1f} s on {threads} "
                  f"threads; 1 thread: {nbytes * c1 / e1 / 1e9:.3f} GB/s ({c1} calls); dequantize-then-matmul: "
                  f"{nbytes * cm / em / 1e9:.3f} GB/s ({cm} calls)",
        "us_per_call": round(el / calls * 1e6, 1),
        "materialize": {"value": round(nbytes * cm / em / 1e9, 3), "unit": "GB/s",
                        "us_per_call": round(em / cm * 1e6, 1), "calls": cm,
                        "what": "single-threaded C dequantize of W to f32, then f32 x @ W^T in numpy"},
    }


if __name__ == "__main__":
    main()
