"""GPU: the configs[0] and configs[4] graphs at full size, as bench.py runs them
(volta_amd.nn.ConvChain): conv -> ReLU (fused into the conv epilogue) -> ...
-> conv, PixelShuffle tail, sum loss, seeded backward with the
ReLU masks fused into the input gradients.

Every layer is checked on a few images against the oracle fed with the
device's own inputs to that layer (so one bf16 rounding of an earlier layer
does not propagate into the comparison): forward + bias + ReLU, the masked
input gradient, the tail and the loss seed bit for bit, the loss against a
float64 sum of the device output.  Weight gradients of every layer against the
oracle over the whole batch (configs[4]'s over image chunks in a thread pool,
`tests/oracle_pool.py`), and bit-identical to a separate call of the same
pass; bias gradients against a float64 sum of the device's output gradient.

The same step captured in a HIP graph (as bench.py times it) is replayed at
full size and must reproduce every buffer of the eager step bit for bit."""
import numpy as np
import pytest
import torch

import oracle
from tests.oracle_pool import batch_sum
from tests.parity import assert_parity, k_conv_dgrad, k_conv_fwd, k_conv_wgrad
from volta_amd import nn as vnn

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def host(t):
    torch.cuda.synchronize()
    return t.float().cpu().numpy()


def _build(name):
    g = torch.Generator().manual_seed(3)
    if name == "configs[0]":
        x = torch.randn((64, 1, 28, 28), generator=g).to(DEV, torch.float32)
        return vnn.ConvChain([(1, 32, 3, 1, 1), (32, 64, 3, 1, 1)], x, generator=g), "f32"
    x = torch.rand((16, 3, 256, 256), generator=g).to(DEV, torch.bfloat16)
    specs = [(3, 64, 5, 1, 2), (64, 64, 3, 1, 1), (64, 32, 3, 1, 1), (32, 27, 3, 1, 1)]
    return vnn.ConvChain(specs, x, tail=vnn.PixelShuffle(3), generator=g), "bf16"


def _set_biases(chain, dt):
    # non-zero biases so the fused bias path is exercised (Conv2d::new starts at 0)
    g = torch.Generator().manual_seed(9)
    for c in chain.convs:
        c.bias = (torch.rand(c.bias.shape, generator=g) * 0.2 - 0.1).to(DEV, c.bias.dtype)


@pytest.mark.parametrize("name,images", [("configs[0]", (0, 31, 63)), ("configs[4]", (0, 15))])
def test_config_graph_full_size(name, images):
    chain, dt = _build(name)
    _set_biases(chain, dt)
    print(f"{name}: forward + backward at full size", flush=True)
    loss = chain.forward()
    chain.backward()
    L = len(chain.convs)
    acts = [host(a) for a in chain.acts]
    grads = [None] + [host(gr) for gr in chain.grads[1:]]
    for li, conv in enumerate(chain.convs):
        w, b = host(conv.weight), host(conv.bias)
        C, O, K = w.shape[1], w.shape[0], w.shape[2]
        S, P = conv.stride[0], conv.padding[0]
        kw = dict(stride=(S, S), pad=(P, P))
        bb = b[None, :, None, None]
        for i in images:
            xi = acts[li][i:i + 1]
            ref = oracle.direct_conv(xi, w, **kw) + bb
            sc = oracle.direct_conv(np.abs(xi), np.abs(w), **kw) + np.abs(bb)
            if li + 1 < L:  # ReLU fused into the epilogue
                ref = np.maximum(ref, 0)
            assert_parity(acts[li + 1][i:i + 1], ref, sc, dt, f"{name} L{li} fwd image {i}",
                          k=k_conv_fwd(C, K, K))
            if li > 0:  # masked input gradient (the ReLU backward of layer li-1)
                gi = grads[li + 1][i:i + 1]
                ref = oracle.direct_conv_backward_input(gi, w, xi.shape, **kw)
                sc = oracle.direct_conv_backward_input(np.abs(gi), np.abs(w), xi.shape, **kw)
                got = grads[li][i:i + 1]
                assert (got[xi <= 0] == 0).all(), f"{name} L{li} dgrad: not masked where the input is <= 0"
                assert_parity(got, np.where(xi > 0, ref, 0), sc, dt, f"{name} L{li} dgrad image {i}",
                              k=k_conv_dgrad(O, K, K))
        # weight and bias gradients over the whole batch
        dw, db = host(chain.wgrads[li][0]), host(chain.wgrads[li][1])
        gl = grads[li + 1]
        HO, WO = gl.shape[2:]
        kwg = k_conv_wgrad(gl.shape[0], HO, WO)
        db_ref = gl.astype(np.float64).sum(axis=(0, 2, 3))
        db_sc = np.abs(gl).astype(np.float64).sum(axis=(0, 2, 3))
        assert_parity(db, db_ref, db_sc, dt, f"{name} L{li} db", k=kwg)
        print(f"{name} L{li}: oracle weight gradient over the whole batch", flush=True)
        ref, sc = batch_sum(oracle.direct_conv_backward_weight, (gl, acts[li]), (w.shape,), kw)
        assert_parity(dw, ref, sc, dt, f"{name} L{li} dw", k=kwg)
        _, dw2, _ = conv.backward(chain.grads[li + 1], chain.acts[li], input_grad=False, weight_grad=True)
        assert np.array_equal(dw, host(dw2)), f"{name} L{li} dw differs from the same pass called alone"
    out = host(chain.output)
    if chain.tail is not None:
        assert np.array_equal(out, oracle.pixel_shuffle(acts[L], 3)), "PixelShuffle tail differs"
        assert np.array_equal(host(chain.tail_grad), np.ones_like(out)), "loss seed is not 1 everywhere"
        assert np.array_equal(grads[L], np.ones_like(acts[L])), "PixelShuffle backward of ones is not ones"
    else:
        assert np.array_equal(grads[L], np.ones_like(acts[L])), "loss seed is not 1 everywhere"
    exact = float(out.astype(np.float64).sum())
    assert abs(float(host(loss)[0]) - exact) <= 1e-6 * float(np.abs(out).astype(np.float64).sum())


@pytest.mark.parametrize("name", ["configs[0]", "configs[4]"])
def test_config_graph_capture_replay_full_size(name):
    """ConvChain.step() captured in a HIP graph after an eager warm-up on the
    capture stream (bench.py's graph_ms_per_step): each replay, with the
    buffers poisoned before it and eager library work between replays, equals
    the eager step bit for bit."""
    chain, dt = _build(name)
    _set_biases(chain, dt)
    bufs = lambda: ([chain.loss, chain.output] + list(chain.acts[1:]) + list(chain.grads[1:])
                    + [t for pair in chain.wgrads for t in pair])
    cap = torch.cuda.Stream()
    cap.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(cap):
        chain.step()
    torch.cuda.synchronize()
    ref = [b.clone() for b in bufs()]
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=cap):
        chain.step()
    torch.cuda.synchronize()
    for rep in range(2):
        for b in bufs():
            b.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for i, (b, r) in enumerate(zip(bufs(), ref)):
            assert torch.equal(b, r), f"{name} replay {rep}: buffer {i} differs from the eager step"
        chain.convs[-1].forward(chain.acts[-2])  # eager library work on the default stream between replays
        torch.cuda.synchronize()
