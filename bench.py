#!/usr/bin/env python3
"""Benchmark of the Volta conv / matmul hot path on one MI355X.

Default workload (the Conv2d fwd+bwd metric's
config): ResNet-style 3x3 conv block, bf16 storage with fp32 accumulation,
N=128, layers 64->64 @56x56, 128->128 @28x28, 256->256 @14x14 (3x3, stride 1,
pad 1) and the 1x1 stride-2 projection 64->128 @56x56.  One step = forward,
input gradient and weight gradient of every layer (dY ~ N(0,1) injected).
Inputs are synthetic and resident in HBM before timing starts.

Prints ONE JSON line (driver contract).  `value` is whole-job TFLOP/s of the
step (algorithmic FLOPs 2*N*K*C*R*S*P*Q per pass) over K steps: forward of
every layer, then input and weight gradients in reverse layer order (the order
of a training step), each weight gradient on a second stream next to the
input-gradient chain (--one-stream: all on one stream).  The same step captured in a HIP
graph gives `graph_ms_per_step`; each pass alone gives `per_op_ms`.  `roofline` is for the
dominant pass, timed with HIP events on the stream it runs on (graph of 10
calls of that pass alone).
`cpu_baseline` times the CPU oracle (a C restatement of Volta's
single-threaded CPU loops) on a bounded sample and extrapolates.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_TFLOPS = {"bf16": 2516.6, "f32": 157.3}  # MI355X dense MFMA
PEAK_HBM_GBS = 8000.0

METRIC = "Conv2d fwd+bwd TFLOP/s & % MFMA peak (1 GPU); GEMM TFLOP/s; vs CPU"

# HBM bytes per call of a pass, from two rocprofv3 counter runs of
# `bench.py --profile-op <pass>` (FETCH_SIZE, then WRITE_SIZE, KiB per dispatch,
# summed over the pass's kernels).  Calibration on the 256 MiB copy of the same
# runs (two dispatches of 128 MiB): WRITE_SIZE reads 131080 KiB per dispatch
# (factor 1), FETCH_SIZE 65550 KiB (factor 2).  Summary:
# profiles/c3_pass_traffic.md.  Keyed by pass name; used for roofline.traffic
# when that pass is the dominant one (which of these is the slowest varies by a
# few percent from run to run).
MEASURED_TRAFFIC_BYTES = {
    # relayout_grouped_kernel: fetch 84.8 KiB x2, write 72; conv_halo_bf16_kernel<3,3,1,4,3,false,false>: fetch 25758.8 x2, write 50176
    "3x3 64->64 @56 fwd": int(((84.8 + 25758.8) * 2 + 72 + 50176) * 1024),
    # relayout_grouped_kernel: fetch 220.0 x2, write 72; conv_halo_bf16_kernel<3,3,1,4,3,false,false>: fetch 25773.0 x2, write 50176
    "3x3 64->64 @56 dgrad": int(((220.0 + 25773.0) * 2 + 72 + 50176) * 1024),
    # conv_halo_bf16_kernel<3,3,1,2,4,true,true,true> (weights read directly): fetch 13903.0 x2, write 25143.1
    "3x3 128->128 @28 fwd": int((13903.0 * 2 + 25143.1) * 1024),
    # wgrad_rows_bf16_kernel<..,true>: fetch 25199.3 x2, write 36864; wgrad_reduce_frag_bf16_kernel: fetch 18465.8 x2, write 288
    "3x3 128->128 @28 wgrad": int(((25199.3 + 18465.8) * 2 + 36864 + 288) * 1024),
    # conv_halo_bf16_kernel<3,3,1,2,4,true,true,true> (weights read directly): fetch 11551.3 x2, write 12674.2
    "3x3 256->256 @14 fwd": int((11551.3 * 2 + 12674.2) * 1024),
    # wgrad_rows_bf16_kernel<..,true>: fetch 12651.5 x2, write 36864; wgrad_reduce_frag_bf16_kernel: fetch 18465.9 x2, write 1152
    "3x3 256->256 @14 wgrad": int(((12651.5 + 18465.9) * 2 + 36864 + 1152) * 1024),
}

# (name, C, O, H, K, stride, pad) at N=128
C3_LAYERS = [
    ("3x3 64->64 @56", 64, 64, 56, 3, 1, 1),
    ("3x3 128->128 @28", 128, 128, 28, 3, 1, 1),
    ("3x3 256->256 @14", 256, 256, 14, 3, 1, 1),
    ("1x1 s2 64->128 @56", 64, 128, 56, 1, 2, 0),
]
C3_BATCH = 128


def conv_out(h, k, s, p):
    return (h + 2 * p - k) // s + 1


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--verbose", action="store_true")
    ap.add_argument("--one-stream", action="store_true",
                    help="issue the whole step on one stream (default: each layer's weight gradient on a "
                         "second stream next to the input-gradient chain)")
    ap.add_argument("--configs", action="store_true",
                    help="instead of the headline line, time a fwd+bwd step of every BASELINE config "
                         "(one JSON line each)")
    ap.add_argument("--config-only", default=None,
                    help="with --configs: only the config whose name starts with this (e.g. 'configs[4]')")
    ap.add_argument("--profile-op", default=None,
                    help="run only this pass (e.g. '3x3 256->256 @14 wgrad') --steps times, then a "
                         "256 MiB device copy, for rocprofv3 counter runs; prints nothing else")
    return ap.parse_args()


def build_layers(torch, vnn, dev):
    g = torch.Generator().manual_seed(0)
    layers = []
    for name, C, O, H, K, S, P in C3_LAYERS:
        conv = vnn.Conv2d(C, O, K, S, P, use_bias=False, device=dev, dtype=torch.bfloat16, generator=g)
        # Kaiming init (fan_in = C*K*K) is what Conv2d::new uses (he_initialization)
        conv.set_algo(vnn.ConvAlgo.IGEMM)
        x = torch.randn((C3_BATCH, C, H, H), generator=g).to(dev, torch.bfloat16)
        HO = conv_out(H, K, S, P)
        dy = torch.randn((C3_BATCH, O, HO, HO), generator=g).to(dev, torch.bfloat16)
        y = torch.empty((C3_BATCH, O, HO, HO), device=dev, dtype=torch.bfloat16)
        dx = torch.empty_like(x)
        dw = torch.empty_like(conv.weight)
        flops = 2.0 * C3_BATCH * O * C * K * K * HO * HO
        byts = 2.0 * (x.numel() + conv.weight.numel() + y.numel())
        layers.append(dict(name=name, conv=conv, x=x, dy=dy, y=y, dx=dx, dw=dw, flops=flops, bytes=byts))
    return layers


def make_train_step(torch, layers, side=None):
    """One training step of the block in dependency order: forward L0..L3, then
    backward L3..L0 (input gradient, then weight gradient, of each layer).  With
    `side` each layer's weight gradient runs on that second stream, started once
    its output gradient exists (after the input gradient of the layer above), next
    to the input-gradient chain -- the usual dW / dX overlap of a training step;
    the split-K reductions and block tails of one pass then share the chip with
    the next pass."""

    def step():
        main = torch.cuda.current_stream()
        for L in layers:
            L["conv"].forward(L["x"], out=L["y"])
        ready = torch.cuda.Event()
        ready.record(main)
        for L in reversed(layers):
            conv = L["conv"]
            if side is not None:
                side.wait_event(ready)
                with torch.cuda.stream(side):
                    conv.backward(L["dy"], L["x"], input_grad=False, weight_grad=True, algo=conv.algo,
                                  outs=(None, L["dw"], None))
            conv.backward(L["dy"], L["x"], input_grad=True, weight_grad=False, algo=conv.algo,
                          outs=(L["dx"], None, None))
            if side is None:
                conv.backward(L["dy"], L["x"], input_grad=False, weight_grad=True, algo=conv.algo,
                              outs=(None, L["dw"], None))
            ready = torch.cuda.Event()
            ready.record(main)
        if side is not None:
            main.wait_stream(side)

    return step


def time_graph_step(torch, step, steps, warmup):
    """Capture `step` in a HIP graph (after eager warm-up on the capture stream,
    so every workspace already exists) and time `steps` replays."""
    cap = torch.cuda.Stream()
    cap.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(cap):
        for _ in range(max(1, warmup)):
            step()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=cap):
        step()
    torch.cuda.synchronize()
    for _ in range(max(1, warmup)):
        g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def time_op_graph(torch, fn, reps, replays):
    """GPU time of one call of `fn`: `reps` calls captured in a HIP graph."""
    def many():
        for _ in range(reps):
            fn()
    return time_graph_step(torch, many, replays, 1) / reps


def time_eager_fn(torch, fn, steps, warmup):
    """`fn` issued eagerly `steps` times between two HIP events (after warm-up)."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def pass_fns(L):
    conv = L["conv"]
    return {
        "fwd": lambda: conv.forward(L["x"], out=L["y"]),
        "dgrad": lambda: conv.backward(L["dy"], L["x"], input_grad=True, weight_grad=False, algo=conv.algo,
                                       outs=(L["dx"], None, None)),
        "wgrad": lambda: conv.backward(L["dy"], L["x"], input_grad=False, weight_grad=True, algo=conv.algo,
                                       outs=(None, L["dw"], None)),
    }


def profile_op(torch, layers, name, reps):
    """Counter runs: the named pass `reps` times, then a plain copy of 256 MiB
    (the calibration kernel: it reads and writes exactly 256 MiB)."""
    layer, op = name.rsplit(" ", 1)
    L = next(L for L in layers if L["name"] == layer)
    fn = pass_fns(L)[op]
    for _ in range(reps):
        fn()
    src = torch.empty(256 << 20, dtype=torch.uint8, device="cuda:0").fill_(1)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()


def config_steps(torch, vnn, dev, steps, warmup, only=None):
    """Fwd+bwd step of each BASELINE config (synthetic inputs of the config's
    shapes, the library's MI355X algorithm choice), one JSON line per config.
    configs[0] and configs[4] run their whole graphs: convolutions with ReLU
    between them, the sum loss, its seeded gradient (dY = 1) and the backward
    chain; configs[3] runs each ConvTranspose2d layer's forward and backward."""
    g = torch.Generator().manual_seed(3)
    dts = {"f32": torch.float32, "bf16": torch.bfloat16}

    def chain(dt, N, H, specs, tail=None):
        """conv -> ReLU -> ... -> conv layers in sequence; specs = (C, O, K, S, P) per
        layer.  Each ReLU is fused into the producing conv's epilogue
        (vh_conv2d_forward_relu) and its backward into the next layer's input
        gradient (vh_conv2d_backward_relu).  Returns run() and the step's
        algorithmic FLOPs (the first layer has no dX)."""
        convs, acts = [], []
        if dt == "bf16" and H == 256:  # configs[4] input ~U[0,1)
            x = torch.rand((N, specs[0][0], H, H), generator=g).to(dev, dts[dt])
        else:
            x = torch.randn((N, specs[0][0], H, H), generator=g).to(dev, dts[dt])
        acts.append(x)
        fl = 0.0
        h = H
        for li, (C, O, K, S, P) in enumerate(specs):
            conv = vnn.Conv2d(C, O, K, S, P, use_bias=True, device=dev, dtype=dts[dt], generator=g)
            ho = conv_out(h, K, S, P)
            convs.append(conv)
            acts.append(torch.empty((N, O, ho, ho), device=dev, dtype=dts[dt]))  # relu(y), or y for the last
            fl += (2 if li == 0 else 3) * 2.0 * N * O * C * K * K * ho * ho
            h = ho
        grads = [torch.empty_like(a) for a in acts]  # grads[i]: gradient w.r.t. acts[i] (pre-ReLU for i > 0)
        wouts = [(torch.empty_like(c.weight), torch.empty_like(c.bias)) for c in convs]
        loss = torch.empty((1,), device=dev, dtype=torch.float32)
        tail_out = tail_dout = None
        if tail is not None:
            tail_out = torch.empty(tail[1], device=dev, dtype=dts[dt])
            tail_dout = torch.empty_like(tail_out)
        L = len(convs)

        def run():
            for li, conv in enumerate(convs):
                conv.forward(acts[li], out=acts[li + 1], relu=li + 1 < L)
            last = acts[L]
            if tail is not None:
                tail[0].forward(last, out=tail_out)
                vnn.sum_loss(tail_out, out=loss)
                vnn.sum_loss_backward(tail_out, 1.0, out=tail_dout)
                tail[0].backward(tail_dout, out=grads[L])
            else:
                vnn.sum_loss(last, out=loss)
                vnn.sum_loss_backward(last, 1.0, out=grads[L])
            for li in range(L - 1, -1, -1):
                dw, db = wouts[li]
                # grads[li] for li > 0 is the gradient before the ReLU that produced acts[li]
                convs[li].backward(grads[li + 1], acts[li], input_grad=li > 0, weight_grad=True,
                                   outs=(grads[li] if li > 0 else None, dw, db), relu_input=li > 0)
        return run, fl

    def convt_layer(dt, N, CI, CO, H, K, S, P):
        ct = vnn.ConvTranspose2d(CI, CO, K, S, P, device=dev, dtype=dts[dt], generator=g)
        x = torch.randn((N, CI, H, H), generator=g).to(dev, dts[dt])
        HO = (H - 1) * S + K - 2 * P
        dy = torch.randn((N, CO, HO, HO), generator=g).to(dev, dts[dt])
        y = torch.empty((N, CO, HO, HO), device=dev, dtype=dts[dt])
        outs = (torch.empty_like(x), torch.empty_like(ct.weight), torch.empty_like(ct.bias))
        fl = 3 * 2.0 * N * H * H * CI * CO * K * K

        def run():
            ct.forward(x, out=y)
            ct.backward(dy, x, outs=outs)
        return run, fl

    ps = vnn.PixelShuffle(3)
    cfgs = {
        "configs[0] MNIST-CNN f32 N=64 (conv-ReLU-conv, sum loss)":
            ("f32", [chain("f32", 64, 28, [(1, 32, 3, 1, 1), (32, 64, 3, 1, 1)])]),
        "configs[3] DCGAN ConvTranspose2d f32 N=128": ("f32", [convt_layer("f32", 128, 100, 512, 1, 4, 1, 0),
                                                               convt_layer("f32", 128, 512, 256, 4, 4, 2, 1),
                                                               convt_layer("f32", 128, 256, 128, 8, 4, 2, 1),
                                                               convt_layer("f32", 128, 128, 64, 16, 4, 2, 1),
                                                               convt_layer("f32", 128, 64, 3, 32, 4, 2, 1)]),
        "configs[4] super-resolution bf16 N=16 256x256 (conv/ReLU chain, PixelShuffle, sum loss)":
            ("bf16", [chain("bf16", 16, 256, [(3, 64, 5, 1, 2), (64, 64, 3, 1, 1), (64, 32, 3, 1, 1),
                                              (32, 27, 3, 1, 1)], tail=(ps, (16, 3, 768, 768)))]),
    }
    for name, (dt, layers) in cfgs.items():
        if only and not name.startswith(only):
            continue

        def step(layers=layers):
            for run, _ in layers:
                run()
        ms = time_eager_fn(torch, step, steps, warmup)
        fl = sum(f for _, f in layers)
        tf = fl / (ms * 1e-3) / 1e12
        print(json.dumps({"config": name, "dtype": dt, "ms_per_step": round(ms, 4), "gflop_per_step": round(fl / 1e9, 3),
                          "tflops": round(tf, 2), "pct_peak": round(100 * tf / PEAK_TFLOPS[dt], 2)}), flush=True)
    if not only or "configs[1]".startswith(only):
        print(json.dumps({"config": "configs[1] Linear / square products", **gemm_secondary(torch, vnn, dev)}),
              flush=True)


def gemm_secondary(torch, vnn, dev, reps=5):
    """Linear 4096x1024 -> 4096 fwd + dX + dW (+ bias) in f32 and bf16, and the
    8192^3 bf16 product; reported beside the headline (same HIP-event timing)."""
    out = {}
    g = torch.Generator().manual_seed(1)
    for dt, name in ((torch.float32, "f32"), (torch.bfloat16, "bf16")):
        lin = vnn.Linear(1024, 4096, device=dev, dtype=dt, generator=g)
        x = torch.randn((4096, 1024), generator=g).to(dev, dt)
        dy = torch.randn((4096, 4096), generator=g).to(dev, dt)
        y = torch.empty((4096, 4096), device=dev, dtype=dt)
        outs = (torch.empty_like(x), torch.empty_like(lin.weight), torch.empty_like(lin.bias))

        def step():
            lin.forward(x, out=y)
            lin.backward(dy, x, outs=outs)
        for _ in range(2):
            step()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            step()
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / reps
        fl = 3 * 2.0 * 4096 * 1024 * 4096
        out[f"linear_4096x1024x4096_fwd_bwd_{name}_tflops"] = round(fl / ms / 1e9, 2)
    import volta_amd
    from volta_amd import ops
    a = torch.randn((8192, 8192), generator=g).to(dev, torch.bfloat16)
    b = torch.randn((8192, 8192), generator=g).to(dev, torch.bfloat16)
    c = torch.empty_like(a)
    st = torch.cuda.current_stream().cuda_stream
    lib = volta_amd.lib()
    for _ in range(2):
        volta_amd.check(lib.vh_matmul(volta_amd.BF16, a.data_ptr(), b.data_ptr(), c.data_ptr(), 8192, 8192, 8192, st))
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        volta_amd.check(lib.vh_matmul(volta_amd.BF16, a.data_ptr(), b.data_ptr(), c.data_ptr(), 8192, 8192, 8192, st))
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / reps
    out["matmul_8192cubed_bf16_tflops"] = round(2.0 * 8192 ** 3 / ms / 1e9, 2)
    return out


def cpu_baseline(images=32, strip_rows=8):
    """Time the oracle's restatement of Volta's CPU Direct loops (what Volta's
    CPU auto-select picks for every C3 layer, conv.rs:55-57) on a sample of
    each loop nest's outer iterations and extrapolate to the full step."""
    import ctypes

    import numpy as np

    import oracle

    lib = oracle.lib()
    rng = np.random.default_rng(0)
    total_s = 0.0
    detail = []
    used = 0.0
    for name, C, O, H, K, S, P in C3_LAYERS:
        HO = conv_out(H, K, S, P)
        # forward (conv.rs:1359-1419): NS images, extrapolated x N/NS
        NS = images
        x = rng.standard_normal((NS, C, H, H)).astype(np.float32)
        w = rng.standard_normal((O, C, K, K)).astype(np.float32)
        t0 = time.perf_counter()
        oracle.direct_conv(x, w, (S, S), (P, P))
        tf = (time.perf_counter() - t0) * C3_BATCH / NS
        # weight grad (conv.rs:544-606): NS images, x N/NS
        dy = rng.standard_normal((NS, O, HO, HO)).astype(np.float32)
        t0 = time.perf_counter()
        oracle.direct_conv_backward_weight(dy, x, w.shape, (S, S), (P, P))
        tw = (time.perf_counter() - t0) * C3_BATCH / NS
        # input grad, literal O(B*C*H*W*O*HO*WO) scan (conv.rs:450-515): run it on
        # a 4-row strip of one input channel of one image, take the cost per
        # (input element x output position) iteration, scale to the full scan
        rows = strip_rows
        HO_s = conv_out(rows, K, S, P)
        ws = np.ascontiguousarray(w[:, :1])
        dys = np.ascontiguousarray(dy[:, :, :HO_s, :])
        dxs = np.empty((1, 1, rows, H), np.float32)
        fp = ctypes.POINTER(ctypes.c_float)
        t0 = time.perf_counter()
        lib.or_direct_conv_backward_input_literal(
            dys.ctypes.data_as(fp), ws.ctypes.data_as(fp), dxs.ctypes.data_as(fp),
            *map(ctypes.c_size_t, (1, 1, O, rows, H, K, K, S, S, P, P)))
        t1 = time.perf_counter() - t0
        per_iter = t1 / (rows * H * O * HO_s * HO)
        td = per_iter * C3_BATCH * C * H * H * O * HO * HO
        used += (tf + tw) * NS / C3_BATCH + t1
        detail.append((name, tf, td, tw))
        total_s += tf + td + tw
    flops = sum(2.0 * C3_BATCH * O * C * K * K * conv_out(H, K, S, P) ** 2 * 3 for _, C, O, H, K, S, P in C3_LAYERS)
    return dict(value=flops / total_s / 1e12, unit="TFLOP/s", cores=1, kind="port",
                sample=("oracle/volta_oracle.c (restated Volta CPU Direct loops, f32, 1 thread): fwd and dW on "
                        f"{images} of 128 images, literal dX scan on a {strip_rows}-row strip of 1 input channel of "
                        f"1 image; extrapolated linearly to the full step ({total_s:.3g} s estimated, {used:.1f} s measured)"),
                seconds_per_step_extrapolated=total_s)


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; multi-GPU sharding is a design note "
                                   "(DESIGN.md), not an implemented path", "n_gpus": args.gpus}))
        sys.exit(2)
    import torch

    import volta_amd
    from volta_amd import nn as vnn

    dev = torch.device("cuda:0")
    volta_amd.lib()
    layers = build_layers(torch, vnn, dev)
    step_flops = 3.0 * sum(L["flops"] for L in layers)

    if args.profile_op:
        profile_op(torch, layers, args.profile_op, args.steps)
        return
    if args.configs:
        config_steps(torch, vnn, dev, args.steps, args.warmup, args.config_only)
        return

    # headline: the training step (forward, then dX and dW in reverse layer
    # order) issued eagerly on one stream, K steps between HIP events; the same
    # step captured in one HIP graph is timed too (graph_ms_per_step)
    train_step = make_train_step(torch, layers, None if args.one_stream else torch.cuda.Stream())
    graph_ms = time_graph_step(torch, train_step, args.steps, args.warmup)
    ms_per_step = time_eager_fn(torch, train_step, args.steps, args.warmup)
    tflops = step_flops / (ms_per_step * 1e-3) / 1e12

    # per-op pass: each pass alone, `reps` calls captured in a HIP graph and
    # replayed (GPU time per call without host launch gaps)
    ops = []
    for L in layers:
        for k, fn in pass_fns(L).items():
            ms = time_op_graph(torch, fn, reps=10, replays=max(2, args.steps // 4))
            ops.append(dict(layer=L["name"], op=k, ms=ms, flops=L["flops"], bytes=L["bytes"]))
    dom = max(ops, key=lambda o: o["ms"])
    ai = dom["flops"] / dom["bytes"]
    ridge = PEAK_TFLOPS["bf16"] * 1e12 / (PEAK_HBM_GBS * 1e9)
    if ai >= ridge:
        ach = dom["flops"] / (dom["ms"] * 1e-3) / 1e12
        roof = dict(bound="mfma", achieved=round(ach, 2), peak=PEAK_TFLOPS["bf16"], unit="TFLOP/s",
                    frac=round(ach / PEAK_TFLOPS["bf16"], 4), traffic=None)
    else:
        ach = dom["bytes"] / (dom["ms"] * 1e-3) / 1e9
        roof = dict(bound="hbm", achieved=round(ach, 1), peak=PEAK_HBM_GBS, unit="GB/s",
                    frac=round(ach / PEAK_HBM_GBS, 4), traffic=None)
    roof["kernel"] = f"{dom['layer']} {dom['op']}"
    roof["traffic"] = MEASURED_TRAFFIC_BYTES.get(roof["kernel"])
    roof["algorithmic_bytes"] = dom["bytes"]
    roof["launch_ms"] = round(dom["ms"], 4)

    secondary = gemm_secondary(torch, vnn, dev)

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline()

    out = {
        "metric": METRIC,
        "value": round(tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "configs[2] ResNet-style 3x3 conv block fwd+dgrad+wgrad, bf16 storage, fp32 accum",
                   "global_batch": C3_BATCH, "layers": [l[0] for l in C3_LAYERS], "bias": False,
                   "algo": "IGEMM", "parallelism": "none (1 GPU)"},
        "pct_bf16_peak": round(100.0 * tflops / PEAK_TFLOPS["bf16"], 2),
        "roofline": roof,
        "cpu_baseline": cpu,
        "schedule": "training step: fwd L0..L3, then dX and dW of L3..L0, eager, "
                    + ("one stream" if args.one_stream else "dW of each layer on a second stream"),
        "graph_ms_per_step": round(graph_ms, 4),
        "per_op_ms": {f"{o['layer']} {o['op']}": round(o["ms"], 4) for o in ops},
        "secondary": secondary,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
