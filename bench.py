#!/usr/bin/env python3
"""Benchmark of the Volta conv / matmul hot path on one MI355X.

Headline workload (the Conv2d fwd+bwd metric's
config): ResNet-style 3x3 conv block, bf16 storage with fp32 accumulation,
N=128, layers 64->64 @56x56, 128->128 @28x28, 256->256 @14x14 (3x3, stride 1,
pad 1) and the 1x1 stride-2 projection 64->128 @56x56.  One step = forward,
input gradient and weight gradient of every layer (dY ~ N(0,1) injected).
Inputs are synthetic and resident in HBM before timing starts.

Prints ONE JSON line (driver contract).  `value` is whole-job TFLOP/s of the
step (algorithmic FLOPs 2*N*K*C*R*S*P*Q per pass) over K steps: forward of
every layer, then input and weight gradients in reverse layer order (the order
of a training step), each weight gradient on a second stream next to the
input-gradient chain (--one-stream: all on one stream).  The same step captured
in a HIP graph gives `graph_ms_per_step`; each pass alone gives `per_op_ms`.
`roofline` is for the dominant pass, timed with HIP events on the stream it
runs on (graph of 10 calls of that pass alone).

`configs` holds every BASELINE config at full size: its fwd+bwd step time,
TFLOP/s, each pass alone (ms, TFLOP/s, GB/s of algorithmic bytes), the
dominant pass's roofline and a CPU baseline.  `cpu_baseline` (and each
config's) times the CPU oracle (a C restatement of Volta's single-threaded CPU
loops) on one pinned core, on a bounded sample of each loop nest,
extrapolated; `host` states the host's cores and CPU model.
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
# `bench.py --profile-op headline` (FETCH_SIZE, then WRITE_SIZE, KiB per
# dispatch, summed over the pass's kernels).  Calibration on the 256 MiB copy
# of the same runs (one dispatch): WRITE_SIZE reads 262144 KiB (factor 1),
# FETCH_SIZE 131088 KiB (factor 2).  Summary: profiles/c3_pass_traffic.md.
# Keyed by pass name; used for roofline.traffic when that pass is the dominant
# one (which pass is the slowest varies by a few percent from run to run).
MEASURED_TRAFFIC_BYTES = {
    # conv_halo_bf16_kernel (fused form, W read directly): fetch 25510 x2, write 50176
    "3x3 64->64 @56 fwd": int((25510 * 2 + 50176) * 1024),
    # relayout_grouped_kernel: fetch 202 x2, write 76; conv_halo_bf16_kernel: fetch 25682 x2, write 50176
    "3x3 64->64 @56 dgrad": int((25884 * 2 + 50252) * 1024),
    # wgrad_rows_bf16_kernel: fetch 52800 x2, write 9216; wgrad_reduce_frag_bf16_kernel: fetch 4646 x2, write 72
    "3x3 64->64 @56 wgrad": int((57446 * 2 + 9288) * 1024),
    # conv_halo_bf16_kernel: fetch 13811 x2, write 25152
    "3x3 128->128 @28 fwd": int((13811 * 2 + 25152) * 1024),
    # relayout_grouped_kernel: fetch 796 x2, write 304; conv_halo_bf16_kernel: fetch 13880 x2, write 25149
    "3x3 128->128 @28 dgrad": int((14676 * 2 + 25453) * 1024),
    # wgrad_rows_bf16_kernel: fetch 25199 x2, write 9216; wgrad_reduce_frag_bf16_kernel: fetch 4646 x2, write 288
    "3x3 128->128 @28 wgrad": int((29845 * 2 + 9504) * 1024),
    # conv_halo_bf16_kernel: fetch 11549 x2, write 12686
    "3x3 256->256 @14 fwd": int((11549 * 2 + 12686) * 1024),
    # relayout_grouped_kernel: fetch 3172 x2, write 1216; conv_halo_bf16_kernel: fetch 11801 x2, write 12650
    "3x3 256->256 @14 dgrad": int((14973 * 2 + 13866) * 1024),
    # wgrad_rows_bf16_kernel: fetch 12651 x2, write 36864; wgrad_reduce_frag_bf16_kernel: fetch 18469 x2, write 1152
    "3x3 256->256 @14 wgrad": int((31120 * 2 + 38016) * 1024),
    # pw_fwd_vec_bf16_kernel: fetch 26593 x2, write 25111
    "1x1 s2 64->128 @56 fwd": int((26593 * 2 + 25111) * 1024),
    # pw_dgrad_vec_bf16_kernel: fetch 15727 x2, write 51674
    "1x1 s2 64->128 @56 dgrad": int((15727 * 2 + 51674) * 1024),
    # pw_wgrad_s2_bf16_kernel: fetch 39878 x2, write 7168; sum_partials_vec4_kernel: fetch 3606 x2, write 16
    "1x1 s2 64->128 @56 wgrad": int((43484 * 2 + 7184) * 1024),
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
    ap.add_argument("--profile-step", action="store_true",
                    help="run only the headline training step, eagerly, --warmup then --steps times (for kernel "
                         "traces of the two-stream schedule); prints the measured ms per step")
    ap.add_argument("--profile-op", default=None,
                    help="run only these passes (e.g. '3x3 256->256 @14 wgrad', several separated by ';', "
                         "or 'headline' for all twelve) --steps times each, then a 256 MiB device copy, for "
                         "rocprofv3 counter runs; prints only the pass names")
    ap.add_argument("--vendor", action="store_true",
                    help="time the same convolution passes and the 8192^3 product through PyTorch-ROCm's own "
                         "libraries (MIOpen, hipBLASLt) instead, for comparison; prints one JSON line")
    return ap.parse_args()


def vendor_reference(torch, dev, steps, warmup):
    """The headline passes, configs[0]'s and configs[4]'s
    convolution passes and the 8192^3 bf16 product through PyTorch-ROCm's
    vendor libraries on the same GPU: torch.nn.functional.conv2d and
    aten.convolution_backward (MIOpen) in NCHW -- the layout of the reference
    and of this library -- and, for configs[2], in NHWC (channels_last, MIOpen's
    preferred layout); torch.mm (hipBLASLt).  Eager calls between HIP events
    (MIOpen calls are not captured in graphs), best of 5 timings of `steps` calls
    after `warmup`.  Not part of the library: a reference point only."""
    g = torch.Generator().manual_seed(0)

    def best_ms(fn):
        return min(time_eager_fn(torch, fn, steps, warmup) for _ in range(5))

    def conv_passes(N, C, O, H, K, S, P, dt, nhwc=False):
        x = torch.randn((N, C, H, H), generator=g).to(dev, dt)
        w = (torch.randn((O, C, K, K), generator=g) * 0.05).to(dev, dt)
        HO = conv_out(H, K, S, P)
        dy = torch.randn((N, O, HO, HO), generator=g).to(dev, dt)
        if nhwc:
            x, w, dy = (t.contiguous(memory_format=torch.channels_last) for t in (x, w, dy))
        bw = torch.ops.aten.convolution_backward
        fns = {"fwd": lambda: torch.nn.functional.conv2d(x, w, None, S, P),
               "dgrad": lambda: bw(dy, x, w, None, [S, S], [P, P], [1, 1], False, [0, 0], 1, [True, False, False]),
               "wgrad": lambda: bw(dy, x, w, None, [S, S], [P, P], [1, 1], False, [0, 0], 1, [False, True, False])}
        return {op: round(best_ms(fn), 4) for op, fn in fns.items()}

    out = {"metric": "vendor-library reference (PyTorch-ROCm: MIOpen convolutions, hipBLASLt GEMM)",
           "unit": "ms per call", "torch": torch.__version__}
    for layout in ("nchw", "nhwc"):
        passes = {}
        for name, C, O, H, K, S, P in C3_LAYERS:
            for op, ms in conv_passes(C3_BATCH, C, O, H, K, S, P, torch.bfloat16, layout == "nhwc").items():
                passes[f"{name} {op}"] = ms
        out[f"configs[2] bf16 {layout}"] = dict(passes=passes, sum_of_passes_ms=round(sum(passes.values()), 4))
    for key, N, H, dt, specs in (("configs[0] f32 nchw", 64, 28, torch.float32,
                                  [("L0 1->32 k3", 1, 32, 3, 1), ("L1 32->64 k3", 32, 64, 3, 1)]),
                                 ("configs[4] bf16 nchw", 16, 256, torch.bfloat16,
                                  [("L0 3->64 k5", 3, 64, 5, 2), ("L1 64->64 k3", 64, 64, 3, 1),
                                   ("L2 64->32 k3", 64, 32, 3, 1), ("L3 32->27 k3", 32, 27, 3, 1)])):
        passes = {}
        for name, C, O, K, P in specs:
            for op, ms in conv_passes(N, C, O, H, K, 1, P, dt).items():
                passes[f"{name} {op}"] = ms
        out[key] = dict(passes=passes, sum_of_passes_ms=round(sum(passes.values()), 4))
    # ConvTranspose2d f32, N=128 (forward, then its input and weight gradients)
    passes = {}
    for CI, CO, H, K, S, P in C4_LAYERS:
        x = torch.randn((C4_BATCH, CI, H, H), generator=g).to(dev)
        w = (torch.randn((CI, CO, K, K), generator=g) * 0.02).to(dev)
        HO = (H - 1) * S + K - 2 * P
        dy = torch.randn((C4_BATCH, CO, HO, HO), generator=g).to(dev)
        bw = torch.ops.aten.convolution_backward
        nm = f"{CI}->{CO} @{HO}"
        for op, fn in (("fwd", lambda: torch.nn.functional.conv_transpose2d(x, w, None, S, P)),
                       ("dX", lambda: bw(dy, x, w, None, [S, S], [P, P], [1, 1], True, [0, 0], 1,
                                         [True, False, False])),
                       ("dW", lambda: bw(dy, x, w, None, [S, S], [P, P], [1, 1], True, [0, 0], 1,
                                         [False, True, False]))):
            passes[f"{nm} {op}"] = round(best_ms(fn), 4)
    out["configs[3] f32 nchw"] = dict(passes=passes, sum_of_passes_ms=round(sum(passes.values()), 4))
    # Linear 4096x1024 -> 4096 (y = x W + b, dX = dY W^T, dW = x^T dY), and the 8192^3 product
    for dt, name in ((torch.float32, "f32"), (torch.bfloat16, "bf16")):
        x = torch.randn((4096, 1024), generator=g).to(dev, dt)
        w = torch.randn((1024, 4096), generator=g).to(dev, dt)
        b = torch.randn((4096,), generator=g).to(dev, dt)
        dy = torch.randn((4096, 4096), generator=g).to(dev, dt)
        wt, xt = w.t().contiguous(), x.t().contiguous()
        passes = {"fwd (+bias)": round(best_ms(lambda: torch.addmm(b, x, w)), 4),
                  "dX": round(best_ms(lambda: torch.mm(dy, wt)), 4),
                  "dW": round(best_ms(lambda: torch.mm(xt, dy)), 4)}
        out[f"configs[1] Linear {name}"] = dict(passes=passes, sum_of_passes_ms=round(sum(passes.values()), 4))
    n = 8192
    a = torch.randn((n, n), generator=g).to(dev, torch.bfloat16)
    b = torch.randn((n, n), generator=g).to(dev, torch.bfloat16)
    ms = best_ms(lambda: torch.mm(a, b))
    out["matmul 8192^3 bf16"] = dict(ms=round(ms, 4), tflops=round(2.0 * n ** 3 / (ms * 1e-3) / 1e12, 1))
    print(json.dumps(out), flush=True)


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


def profile_op(torch, vnn, dev, layers, names, reps):
    """Counter runs: each named pass `reps` times, then a plain copy of 256 MiB
    (the calibration kernel: it reads and writes exactly 256 MiB).  `names` is
    one pass or several separated by ';': a headline pass ('3x3 256->256 @14
    wgrad'), 'configs[i]:<pass>' for a pass of another config ('configs[4]:L1
    64->64 k3 fwd'), or 'headline' for all twelve headline passes.  Before each
    pass one `fill_` of a 4 KiB marker tensor is dispatched, so the dispatches
    of a trace split into the passes in the order given (printed, one per line)."""
    works = None
    todo = []
    for name in names.split(";"):
        name = name.strip()
        if name == "headline":
            todo += [(f"{L['name']} {op}", fn) for L in layers for op, fn in pass_fns(L).items()]
        elif ":" in name:
            cfg, pname = name.split(":", 1)
            works = works or build_workloads(torch, vnn, dev, layers)
            w = next(w for w in works if w.name.startswith(cfg) and (pname in w.passes or pname in w.combined))
            todo.append((name, {**w.passes, **w.combined}[pname][0]))
        else:
            layer, op = name.rsplit(" ", 1)
            L = next(L for L in layers if L["name"] == layer)
            todo.append((name, pass_fns(L)[op]))
    marker = torch.empty(1024, dtype=torch.float32, device=dev)
    for name, fn in todo:
        torch.cuda.synchronize()
        marker.fill_(1.0)
        print("pass:", name, flush=True)
        for _ in range(reps):
            fn()
    torch.cuda.synchronize()
    src = torch.empty(256 << 20, dtype=torch.uint8, device="cuda:0").fill_(1)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()


def conv_pass_work(N, C, O, H, W, K, S, P, es):
    """Algorithmic FLOPs and bytes (|in| + |W| + |out| at storage size es) of
    one conv pass (forward, input or weight gradient: the same three tensors)."""
    HO, WO = conv_out(H, K, S, P), conv_out(W, K, S, P)
    flops = 2.0 * N * O * C * K * K * HO * WO
    byts = es * (N * C * H * W + O * C * K * K + N * O * HO * WO)
    return flops, byts


def roofline_of(flops, byts, ms, dt):
    """Roofline entry of one pass: MFMA-bound when its intensity is at or above
    the dtype's ridge (peak FLOP/s / 8 TB/s), else HBM-bound."""
    peak = PEAK_TFLOPS[dt]
    ridge = peak * 1e12 / (PEAK_HBM_GBS * 1e9)
    if byts and flops / byts < ridge:
        ach = byts / (ms * 1e-3) / 1e9
        return dict(bound="hbm", achieved=round(ach, 1), peak=PEAK_HBM_GBS, unit="GB/s", frac=round(ach / PEAK_HBM_GBS, 4))
    ach = flops / (ms * 1e-3) / 1e12
    return dict(bound="mfma", achieved=round(ach, 2), peak=peak, unit="TFLOP/s", frac=round(ach / peak, 4))


class Workload:
    """One BASELINE config at its full size: `step` (one fwd+bwd step), the
    passes it is made of (name -> (fn, flops, bytes)), its dtype and the CPU
    baseline function (seconds per step of Volta's CPU path, extrapolated).
    `combined`: calls that run several of the passes at once (same form),
    timed and listed but not counted in the step's FLOPs or pass sum."""

    def __init__(self, name, dt, step, passes, cpu, note="", combined=None):
        self.name, self.dt, self.step, self.passes, self.cpu, self.note = name, dt, step, passes, cpu, note
        self.combined = combined or {}


def chain_passes(chain, es):
    """(fn, flops, bytes) of every pass of a ConvChain (convs, tail, loss, seed)."""
    fns = chain.passes()
    out = {}
    for i, conv in enumerate(chain.convs):
        N, C, H, W = chain.acts[i].shape
        O, _, K, _ = conv.weight.shape
        fl, by = conv_pass_work(N, C, O, H, W, K, conv.stride[0], conv.padding[0], es)
        for op in ("fwd", "dgrad", "wgrad"):
            if f"L{i} {op}" in fns:
                out[f"L{i} {C}->{O} k{K} {op}"] = (fns[f"L{i} {op}"], fl, by)
    n_out = chain.output.numel()
    if chain.tail is not None:
        n_in = chain.acts[-1].numel()
        out["PixelShuffle fwd"] = (fns["tail fwd"], 0.0, es * (n_in + n_out))
        out["PixelShuffle bwd"] = (fns["tail bwd"], 0.0, es * (n_in + n_out))
    out["sum loss"] = (fns["loss"], float(n_out), es * n_out)
    out["loss seed"] = (fns["seed"], 0.0, es * n_out)
    return out


def build_workloads(torch, vnn, dev, c3_layers):
    """configs[0..4] (BASELINE.json order) as Workloads."""
    g = torch.Generator().manual_seed(3)
    wl = []
    # MNIST-CNN f32, N=64: conv 1->32 3x3, ReLU, conv 32->64 3x3, sum loss
    x0 = torch.randn((64, 1, 28, 28), generator=g).to(dev, torch.float32)
    c0 = vnn.ConvChain([(1, 32, 3, 1, 1), (32, 64, 3, 1, 1)], x0, generator=g)
    wl.append(Workload("configs[0] MNIST-CNN f32 N=64 (conv-ReLU-conv, sum loss)", "f32", c0.step,
                       chain_passes(c0, 4), cpu_config0))
    # Linear 4096x1024 -> 4096 (f32, bf16) and the 8192^3 bf16 product
    for dt, tdt in (("f32", torch.float32), ("bf16", torch.bfloat16)):
        es = 4 if dt == "f32" else 2
        lin = vnn.Linear(1024, 4096, device=dev, dtype=tdt, generator=g)
        x = torch.randn((4096, 1024), generator=g).to(dev, tdt)
        dy = torch.randn((4096, 4096), generator=g).to(dev, tdt)
        y = torch.empty((4096, 4096), device=dev, dtype=tdt)
        outs = (torch.empty_like(x), torch.empty_like(lin.weight), torch.empty_like(lin.bias))
        fl = 2.0 * 4096 * 1024 * 4096
        by = es * (4096 * 1024 + 1024 * 4096 + 4096 * 4096)
        passes = {
            "fwd (+bias)": (lambda lin=lin, x=x, y=y: lin.forward(x, out=y), fl, by),
            "dX": (lambda lin=lin, x=x, dy=dy, o=outs: lin.backward(dy, x, weight_grad=False,
                                                                   outs=(o[0], None, None)), fl, by),
            "dW (+db)": (lambda lin=lin, x=x, dy=dy, o=outs: lin.backward(dy, x, input_grad=False,
                                                                         outs=(None, o[1], o[2])), fl, by),
        }
        # the step's backward: one call (bf16: dX and dW in one launch)
        combined = {"dX + dW (+db)": (lambda lin=lin, x=x, dy=dy, o=outs: lin.backward(dy, x, outs=o), 2 * fl,
                                      es * (4096 * 4096 + 2 * 4096 * 1024 + 2 * 1024 * 4096))}

        def step(lin=lin, x=x, y=y, dy=dy, o=outs):
            lin.forward(x, out=y)
            lin.backward(dy, x, outs=o)
        wl.append(Workload(f"configs[1] Linear 4096x1024->4096 fwd+bwd {dt}", dt, step, passes, cpu_config1_linear,
                           combined=combined))
    import volta_amd
    lib = volta_amd.lib()
    n = 8192
    a = torch.randn((n, n), generator=g).to(dev, torch.bfloat16)
    b = torch.randn((n, n), generator=g).to(dev, torch.bfloat16)
    gr = torch.randn((n, n), generator=g).to(dev, torch.bfloat16)
    c, da, db_ = torch.empty_like(a), torch.empty_like(a), torch.empty_like(a)
    fl, by = 2.0 * n ** 3, 2.0 * 3 * n ** 2
    cs = lambda: torch.cuda.current_stream().cuda_stream  # noqa: E731
    sq = {"C = A.B": (lambda: volta_amd.check(lib.vh_matmul(volta_amd.BF16, a.data_ptr(), b.data_ptr(),
                                                             c.data_ptr(), n, n, n, cs())), fl, by),
          "dA = G.B^T": (lambda: volta_amd.check(lib.vh_matmul_backward_a(volta_amd.BF16, gr.data_ptr(), b.data_ptr(),
                                                                           da.data_ptr(), n, n, n, cs())), fl, by),
          "dB = A^T.G": (lambda: volta_amd.check(lib.vh_matmul_backward_b(volta_amd.BF16, a.data_ptr(), gr.data_ptr(),
                                                                           db_.data_ptr(), n, n, n, cs())), fl, by)}

    def sq_step():
        for fn, _, _ in sq.values():
            fn()
    wl.append(Workload("configs[1] square 8192^3 bf16 fwd+bwd (C, dA, dB)", "bf16", sq_step, sq, cpu_config1_square))
    # the headline block (timed above; its passes are the headline's per_op_ms)
    passes2 = {}
    for L in c3_layers:
        for op, fn in pass_fns(L).items():
            passes2[f"{L['name']} {op}"] = (fn, L["flops"], L["bytes"])
    wl.append(Workload("configs[2] ResNet-style 3x3 block bf16 N=128 (the headline)", "bf16", None, passes2,
                       cpu_config2))
    # DCGAN generator ConvTranspose2d f32, N=128
    passes3 = {}
    steps3 = []
    for CI, CO, H, K, S, P in C4_LAYERS:
        ct = vnn.ConvTranspose2d(CI, CO, K, S, P, device=dev, dtype=torch.float32, generator=g)
        ct.weight = (torch.randn(ct.weight.shape, generator=g) * 0.02).to(dev)
        x = torch.randn((C4_BATCH, CI, H, H), generator=g).to(dev)
        HO = (H - 1) * S + K - 2 * P
        dy = torch.randn((C4_BATCH, CO, HO, HO), generator=g).to(dev)
        y = torch.empty((C4_BATCH, CO, HO, HO), device=dev)
        outs = (torch.empty_like(x), torch.empty_like(ct.weight), torch.empty_like(ct.bias))
        fl = 2.0 * C4_BATCH * H * H * CI * CO * K * K
        by = 4.0 * (x.numel() + ct.weight.numel() + y.numel())
        nm = f"{CI}->{CO} @{HO}"
        passes3[f"{nm} fwd"] = (lambda ct=ct, x=x, y=y: ct.forward(x, out=y), fl, by)
        passes3[f"{nm} dX"] = (lambda ct=ct, x=x, dy=dy, o=outs: ct.backward(dy, x, weight_grad=False,
                                                                           outs=(o[0], None, None)), fl, by)
        passes3[f"{nm} dW (+db)"] = (lambda ct=ct, x=x, dy=dy, o=outs: ct.backward(dy, x, input_grad=False,
                                                                                 outs=(None, o[1], o[2])), fl, by)
        steps3.append((ct, x, y, dy, outs))

    def step3():
        for ct, x, y, dy, o in steps3:
            ct.forward(x, out=y)
            ct.backward(dy, x, outs=o)
    wl.append(Workload("configs[3] DCGAN ConvTranspose2d f32 N=128 (each layer fwd+bwd)", "f32", step3, passes3,
                       cpu_config3))
    # super-resolution bf16, N=16, 3x256x256 ~U[0,1): conv/ReLU chain, PixelShuffle r=3, sum loss
    x4 = torch.rand((16, 3, 256, 256), generator=g).to(dev, torch.bfloat16)
    c4 = vnn.ConvChain([(3, 64, 5, 1, 2), (64, 64, 3, 1, 1), (64, 32, 3, 1, 1), (32, 27, 3, 1, 1)], x4,
                       tail=vnn.PixelShuffle(3), generator=g)
    wl.append(Workload("configs[4] super-resolution bf16 N=16 256x256 (conv/ReLU chain, PixelShuffle, sum loss)",
                       "bf16", c4.step, chain_passes(c4, 2), cpu_config4))
    return wl


def measure_workload(torch, w, steps, warmup, step_ms=None, pass_ms=None):
    """Step time, per-pass times (each pass alone, 10 calls in a HIP graph) and
    the dominant pass's roofline.  The step is timed both ways it can be issued
    -- eagerly (HIP events around `steps` steps) and as one captured HIP graph
    replayed `steps` times -- and `ms_per_step` is the faster, named in `issue`
    (a one-stream chain of many short launches runs faster from a graph).  A
    given `step_ms` (the headline, timed by the caller) is used as it is."""
    eager_ms = graph_ms = None
    issue = "eager"
    if step_ms is None:
        eager_ms = time_eager_fn(torch, w.step, steps, warmup)
        graph_ms = time_graph_step(torch, w.step, steps, warmup)
        step_ms = min(eager_ms, graph_ms)
        issue = "graph" if graph_ms < eager_ms else "eager"
    passes = {}
    for name, (fn, fl, by) in w.passes.items():
        ms = pass_ms[name] if pass_ms and name in pass_ms else time_op_graph(torch, fn, reps=10, replays=3)
        passes[name] = dict(ms=round(ms, 4), tflops=round(fl / (ms * 1e-3) / 1e12, 2) if fl else 0.0,
                            gbs=round(by / (ms * 1e-3) / 1e9, 1))
    combined = {}
    for name, (fn, fl, by) in w.combined.items():
        ms = time_op_graph(torch, fn, reps=10, replays=3)
        combined[name] = dict(ms=round(ms, 4), tflops=round(fl / (ms * 1e-3) / 1e12, 2),
                              gbs=round(by / (ms * 1e-3) / 1e9, 1))
    fl = sum(f for _, f, _ in w.passes.values() if f > 1e6)  # conv / GEMM FLOPs (not the loss adds)
    dom = max(w.passes, key=lambda n: passes[n]["ms"])
    _, dfl, dby = w.passes[dom]
    roof = roofline_of(dfl, dby, passes[dom]["ms"], w.dt)
    roof.update(kernel=dom, launch_ms=passes[dom]["ms"], algorithmic_bytes=dby)
    tf = fl / (step_ms * 1e-3) / 1e12
    times = {} if eager_ms is None else dict(issue=issue, eager_ms_per_step=round(eager_ms, 4),
                                             graph_ms_per_step=round(graph_ms, 4))
    return dict(dtype=w.dt, ms_per_step=round(step_ms, 4), **times, gflop_per_step=round(fl / 1e9, 3),
                tflops=round(tf, 2),
                pct_peak=round(100 * tf / PEAK_TFLOPS[w.dt], 2), roofline=roof,
                sum_of_passes_ms=round(sum(p["ms"] for p in passes.values()), 4), passes=passes,
                **(dict(combined_calls=combined) if combined else {}))


C4_BATCH = 128
# configs[3] layers: (CI, CO, H, K, stride, pad)
C4_LAYERS = [(100, 512, 1, 4, 1, 0), (512, 256, 4, 4, 2, 1), (256, 128, 8, 4, 2, 1), (128, 64, 16, 4, 2, 1),
             (64, 3, 32, 4, 2, 1)]
CPU_NOTE = ("oracle/volta_oracle.c: a C restatement of Volta's single-threaded CPU loops (f32, -O2, FMA "
            "contraction off; its GEMM is a plain-loop stand-in for matrixmultiply 0.3.10), 1 thread pinned to "
            "one core")


def _t(fn, *a, **k):
    t0 = time.perf_counter()
    fn(*a, **k)
    return time.perf_counter() - t0


def _dx_literal_per_iter(O, K, S, P, W, rows=8):
    """Seconds per (input element x output position) iteration of Volta's literal
    Direct input-gradient scan (conv.rs:450-515), timed on a `rows`-row strip of
    one input channel of one image."""
    import ctypes

    import numpy as np

    import oracle
    rng = np.random.default_rng(1)
    HO_s, WO = conv_out(rows, K, S, P), conv_out(W, K, S, P)
    w = rng.standard_normal((O, 1, K, K)).astype(np.float32)
    dy = rng.standard_normal((1, O, HO_s, WO)).astype(np.float32)
    dx = np.empty((1, 1, rows, W), np.float32)
    fp = ctypes.POINTER(ctypes.c_float)
    t = _t(oracle.lib().or_direct_conv_backward_input_literal, dy.ctypes.data_as(fp), w.ctypes.data_as(fp),
           dx.ctypes.data_as(fp), *map(ctypes.c_size_t, (1, 1, O, rows, W, K, K, S, S, P, P)))
    return t / (rows * W * O * HO_s * WO), t


def cpu_config0():
    """configs[0] on Volta's CPU path in full (auto-select: conv1 Im2col, conv2
    Direct, conv.rs:55-68): forward, sum loss, seed, conv2's Direct weight
    gradient and its literal O(B*C*H*W*O*P*Q) input-gradient scan
    (conv.rs:450-515, 8.0e10 iterations), the ReLU backward and conv1's Im2col
    backward, all at N=64."""
    import numpy as np

    import oracle
    rng = np.random.default_rng(0)
    N = 64
    x = rng.standard_normal((N, 1, 28, 28)).astype(np.float32)
    w1 = rng.uniform(-0.8165, 0.8165, (32, 1, 3, 3)).astype(np.float32)
    w2 = rng.uniform(-0.1443, 0.1443, (64, 32, 3, 3)).astype(np.float32)
    kw = dict(stride=(1, 1), pad=(1, 1))
    t0 = time.perf_counter()
    h = oracle.relu(oracle.im2col_conv_forward(x, w1, **kw))
    y = oracle.direct_conv(h, w2, **kw)
    oracle.sum_all(y)
    dy = oracle.sum_backward(1.0, y.shape)
    oracle.direct_conv_backward_weight(dy, h, w2.shape, **kw)
    dh = oracle.direct_conv_backward_input(dy, w2, h.shape, literal=True, **kw)
    dh = oracle.relu_backward(dh, h)
    oracle.im2col_conv_backward(dh, x, w1, **kw)
    t = time.perf_counter() - t0
    return t, t, "the full graph at N=64, conv2's input gradient as Volta's literal Direct scan"


_LINEAR_CPU = {}


def cpu_config1_linear():
    """configs[1] Linear 4096x1024 -> 4096 fwd + dX + dW + db in full
    (MatMulGradFn, matmul.rs:450-460, 563-574; bias grad binary.rs:533-598).
    bf16 has no CPU arithmetic in the reference (f32 math on bf16-rounded
    values): the same loops, timed once."""
    if "v" not in _LINEAR_CPU:
        import numpy as np

        import oracle
        rng = np.random.default_rng(0)
        m = 4096
        x = rng.standard_normal((m, 1024)).astype(np.float32)
        w = rng.uniform(-0.0765, 0.0765, (1024, 4096)).astype(np.float32)
        b = np.zeros(4096, np.float32)
        dy = rng.standard_normal((m, 4096)).astype(np.float32)
        t = _t(oracle.linear_forward, x, w, b) + _t(oracle.linear_backward, dy, x, w)
        _LINEAR_CPU["v"] = (t, t)
    tot, meas = _LINEAR_CPU["v"]
    return tot, meas, "all 4096 rows of fwd, dX, dW and db (timed once for both dtypes)"


def cpu_config1_square():
    """configs[1] 8192^3: C = A.B, dA = G.B^T, dB = A^T.G (matmul.rs:450-460,
    563-574, transposes materialised as the reference does) on 16 of the 8192
    rows of A and G (each product is linear in them), x512."""
    import numpy as np

    import oracle
    rng = np.random.default_rng(0)
    ms, n = 16, 8192
    a = rng.standard_normal((ms, n)).astype(np.float32)
    b = rng.standard_normal((n, n)).astype(np.float32)
    g = rng.standard_normal((ms, n)).astype(np.float32)
    t = _t(oracle.matmul, a, b) + _t(oracle.matmul_backward_a, g, b) + _t(oracle.matmul_backward_b, a, g)
    return t * n / ms, t, "16 of 8192 rows of A and G for C, dA and dB, x512"


def cpu_config3():
    """configs[3] ConvTranspose2d layers (conv_transpose.rs:356-435 forward,
    161-341 backward) in full: every layer's forward and backward at N=128."""
    import numpy as np

    import oracle
    rng = np.random.default_rng(0)
    t = 0.0
    for CI, CO, H, K, S, P in C4_LAYERS:
        x = rng.standard_normal((C4_BATCH, CI, H, H)).astype(np.float32)
        w = rng.normal(0, 0.02, (CI, CO, K, K)).astype(np.float32)
        b = np.zeros(CO, np.float32)
        kw = dict(stride=(S, S), pad=(P, P))
        t0 = time.perf_counter()
        y = oracle.conv_transpose_forward(x, w, b, **kw)
        oracle.conv_transpose_backward(np.ones_like(y), x, w, **kw)
        t += time.perf_counter() - t0
    return t, t, f"every layer's forward and backward at N={C4_BATCH}, in full"


def cpu_config4(rows=8):
    """configs[4] on Volta's CPU path (auto-select: Direct for every layer,
    conv.rs:55-57): each Direct forward and weight gradient on a `rows`-row strip
    of one image, scaled per output position; the literal input-gradient scans on
    a strip of one input channel (per-iteration cost x iteration count);
    PixelShuffle, ReLU and the sum on one image, x16."""
    import numpy as np

    import oracle
    rng = np.random.default_rng(0)
    N, H = 16, 256
    specs = [(3, 64, 5, 2), (64, 64, 3, 1), (64, 32, 3, 1), (32, 27, 3, 1)]
    tot = meas = 0.0
    for li, (C, O, K, P) in enumerate(specs):
        kw = dict(stride=(1, 1), pad=(P, P))
        x = rng.standard_normal((1, C, rows, H)).astype(np.float32)
        w = rng.standard_normal((O, C, K, K)).astype(np.float32)
        tf = _t(oracle.direct_conv, x, w, **kw)
        dy = np.ones((1, O, conv_out(rows, K, 1, P), H), np.float32)
        tw = _t(oracle.direct_conv_backward_weight, dy, x, w.shape, **kw)
        per_pos = conv_out(rows, K, 1, P) * H
        tot += (tf + tw) * N * H * H / per_pos
        meas += tf + tw
        if li > 0:
            per, ts = _dx_literal_per_iter(O, K, 1, P, H)
            tot += per * N * C * H * H * O * H * H
            meas += ts
    y = rng.standard_normal((1, 27, H, H)).astype(np.float32)
    te = (_t(oracle.pixel_shuffle, y, 3) + _t(oracle.pixel_shuffle_backward, np.ones((1, 3, 3 * H, 3 * H),
                                                                                          np.float32), 3)
          + _t(oracle.sum_all, y) + 3 * (_t(oracle.relu, y) + _t(oracle.relu_backward, y, y)) * 64 / 27)
    tot += te * N
    meas += te
    return tot, meas, (f"Direct fwd and dW of each layer on a {rows}-row strip of 1 image (per output position), "
                       "literal dX scans on an 8-row strip of 1 input channel (per iteration), PixelShuffle / ReLU / "
                       "sum on 1 image; extrapolated linearly")


def cpu_config2():
    r = cpu_baseline()
    return r["seconds_per_step_extrapolated"], r["measured_s"], r["sample"]


class pinned_one_core:
    """Runs the CPU leg on one core of this process's affinity set (restored after)."""

    def __enter__(self):
        self.prev = os.sched_getaffinity(0)
        self.core = min(self.prev)
        os.sched_setaffinity(0, {self.core})
        return self

    def __exit__(self, *exc):
        os.sched_setaffinity(0, self.prev)


def host_info():
    model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return dict(nproc=os.cpu_count(), affinity_cpus=len(os.sched_getaffinity(0)), cpu_model=model)


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
                seconds_per_step_extrapolated=total_s, measured_s=used)


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
        profile_op(torch, vnn, dev, layers, args.profile_op, args.steps)
        return
    if args.vendor:
        vendor_reference(torch, dev, args.steps, args.warmup)
        return
    if args.profile_step:
        step = make_train_step(torch, layers, None if args.one_stream else torch.cuda.Stream())
        print("headline step ms:", round(time_eager_fn(torch, step, args.steps, args.warmup), 4), flush=True)
        return

    # headline: the training step (forward, then dX and dW in reverse layer
    # order) issued eagerly, K steps between HIP events; the same step captured
    # in one HIP graph is timed too (graph_ms_per_step)
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
    roof = roofline_of(dom["flops"], dom["bytes"], dom["ms"], "bf16")
    roof["kernel"] = f"{dom['layer']} {dom['op']}"
    roof["traffic"] = MEASURED_TRAFFIC_BYTES.get(roof["kernel"])
    roof["algorithmic_bytes"] = dom["bytes"]
    roof["launch_ms"] = round(dom["ms"], 4)

    # every BASELINE config: step, per-pass times and rooflines (configs[2] = the headline's numbers)
    configs = {}
    works = build_workloads(torch, vnn, dev, layers)
    for w in works:
        if w.step is None:
            r = measure_workload(torch, w, args.steps, args.warmup, step_ms=ms_per_step,
                                 pass_ms={f"{o['layer']} {o['op']}": o["ms"] for o in ops})
        else:
            r = measure_workload(torch, w, args.steps, args.warmup)
        configs[w.name] = r
    torch.cuda.synchronize()

    host = host_info()
    cpu = None
    if not args.no_cpu:
        # Volta's CPU path per config, one thread pinned to one core of this process
        with pinned_one_core() as pin:
            host["cpu_leg_core"] = pin.core
            for w in works:
                r = configs[w.name]
                tot, meas, sample = w.cpu()
                r["cpu_baseline"] = dict(value=round(r["gflop_per_step"] / tot / 1e3, 6), unit="TFLOP/s", cores=1,
                                         kind="port", seconds_per_step=round(tot, 4),
                                         measured_s=round(meas, 2), sample=sample)
                r["speedup_vs_cpu"] = round(tot * 1e3 / r["ms_per_step"], 1)
        c2 = next(configs[w.name]["cpu_baseline"] for w in works if w.name.startswith("configs[2]"))
        cpu = dict(c2, sample=c2["sample"] + "; " + CPU_NOTE)

    lin = {w.name: configs[w.name] for w in works if w.name.startswith("configs[1]")}
    secondary = {
        "linear_4096x1024x4096_fwd_bwd_f32_tflops": next(v["tflops"] for k, v in lin.items() if k.endswith("f32")),
        "linear_4096x1024x4096_fwd_bwd_bf16_tflops": next(v["tflops"] for k, v in lin.items() if k.endswith("bf16")),
        "matmul_8192cubed_bf16_tflops": next(v["passes"]["C = A.B"]["tflops"] for k, v in lin.items()
                                             if "square" in k),
    }

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
        "host": host,
        "configs": configs,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
