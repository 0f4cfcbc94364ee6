"""GPU: the library's calls captured in a HIP graph (as bench.py runs the
training step) replay to exactly the eager results.

Every kernel here is deterministic (fixed split-K summation order), so each
replay must reproduce the eager outputs bit for bit.  Between replays the
program does other eager work through the same library (a different layer on
the default stream) and synchronizes, so replays that depend on stale
workspace contents or on state left by the eager calls would show up."""
import pytest
import torch

from volta_amd import nn as vnn

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _layer(C, O, K, S, P, N, H, seed):
    g = torch.Generator().manual_seed(seed)
    conv = vnn.Conv2d(C, O, K, S, P, use_bias=True, device=DEV, dtype=torch.bfloat16, generator=g)
    conv.bias = torch.randn(O, generator=g).to(DEV, torch.bfloat16)
    conv.set_algo(vnn.ConvAlgo.IGEMM)
    x = torch.randn(N, C, H, H, generator=g).to(DEV, torch.bfloat16)
    HO = (H + 2 * P - K) // S + 1
    dy = torch.randn(N, O, HO, HO, generator=g).to(DEV, torch.bfloat16)
    outs = dict(y=torch.empty(N, O, HO, HO, device=DEV, dtype=torch.bfloat16), dx=torch.empty_like(x),
                dw=torch.empty_like(conv.weight), db=torch.empty_like(conv.bias))
    return conv, x, dy, outs


def _run(conv, x, dy, o, side):
    conv.forward(x, out=o["y"])
    ready = torch.cuda.Event()
    ready.record(torch.cuda.current_stream())
    side.wait_event(ready)
    with torch.cuda.stream(side):
        conv.backward(dy, x, input_grad=False, weight_grad=True, algo=conv.algo, outs=(None, o["dw"], o["db"]))
    conv.backward(dy, x, input_grad=True, weight_grad=False, algo=conv.algo, outs=(o["dx"], None, None))
    torch.cuda.current_stream().wait_stream(side)


@pytest.mark.parametrize("shape", [(64, 64, 3, 1, 1, 4, 14), (64, 128, 1, 2, 0, 4, 16), (32, 48, 3, 1, 1, 2, 9)],
                         ids=["3x3", "1x1s2", "3x3odd"])
def test_graph_replay_matches_eager(shape):
    C, O, K, S, P, N, H = shape
    conv, x, dy, o = _layer(C, O, K, S, P, N, H, seed=sum(shape))
    other, ox, ody, oo = _layer(C, O, K, S, P, N + 1, H, seed=7)
    side = torch.cuda.Stream()
    cap = torch.cuda.Stream()
    cap.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(cap):
        _run(conv, x, dy, o, side)  # eager reference on the capture stream (also creates its workspace)
    torch.cuda.synchronize()
    ref = {k: v.clone() for k, v in o.items()}
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=cap):
        _run(conv, x, dy, o, side)
    torch.cuda.synchronize()
    for rep in range(3):
        for v in o.values():
            v.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for k in o:
            assert torch.equal(o[k], ref[k]), f"replay {rep}: {k} differs from the eager result"
        _run(other, ox, ody, oo, side)  # eager work through the library between replays
        torch.cuda.synchronize()


def test_workspace_growth_keeps_captured_graph_valid():
    """A small layer is captured on `cap` / `side`; between replays a much larger
    layer runs eagerly on the same two streams, so both streams' workspaces grow
    (more split-K partials).  The outgrown buffers the graph holds are retired,
    not freed: every replay still matches the eager result bit for bit."""
    conv, x, dy, o = _layer(64, 64, 3, 1, 1, 2, 14, seed=3)
    big, bx, bdy, bo = _layer(64, 64, 3, 1, 1, 16, 56, seed=9)
    side = torch.cuda.Stream()
    cap = torch.cuda.Stream()
    cap.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(cap):
        _run(conv, x, dy, o, side)
    torch.cuda.synchronize()
    ref = {k: v.clone() for k, v in o.items()}
    with torch.cuda.stream(cap):
        _run(big, bx, bdy, bo, side)
    torch.cuda.synchronize()
    big_ref = {k: v.clone() for k, v in bo.items()}
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=cap):
        _run(conv, x, dy, o, side)
    torch.cuda.synchronize()
    for rep in range(3):
        for v in o.values():
            v.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for k in o:
            assert torch.equal(o[k], ref[k]), f"replay {rep}: {k} differs from the eager result"
        # a layer twice as deep in images and 4x the area on the capture streams: workspace growth
        big2, b2x, b2dy, b2o = _layer(64, 64, 3, 1, 1, 16 * (rep + 2), 56, seed=9 + rep)
        with torch.cuda.stream(cap):
            _run(big2, b2x, b2dy, b2o, side)
            _run(big, bx, bdy, bo, side)
        torch.cuda.synchronize()
        for k in bo:
            assert torch.equal(bo[k], big_ref[k]), f"eager {k} after replay {rep} differs"


def test_workspace_growth_during_capture_is_an_error():
    """A call whose workspace would have to grow inside a capture returns
    VH_ERR_CAPTURE (nothing is allocated, freed or synchronised); the same call
    run once eagerly first then captures fine."""
    import volta_amd
    conv, x, dy, o = _layer(64, 64, 3, 1, 1, 4, 28, seed=5)
    cap = torch.cuda.Stream()
    cap.wait_stream(torch.cuda.current_stream())
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with pytest.raises(volta_amd.VoltaHipError) as e:
        with torch.cuda.graph(g, stream=cap):
            conv.backward(dy, x, input_grad=False, weight_grad=True, algo=conv.algo,
                          outs=(None, o["dw"], o["db"]))
    assert e.value.status == volta_amd._lib.VH_ERR_CAPTURE
    torch.cuda.synchronize()
    with torch.cuda.stream(cap):
        conv.backward(dy, x, input_grad=False, weight_grad=True, algo=conv.algo, outs=(None, o["dw"], o["db"]))
    torch.cuda.synchronize()
    ref = o["dw"].clone()
    g2 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g2, stream=cap):
        conv.backward(dy, x, input_grad=False, weight_grad=True, algo=conv.algo, outs=(None, o["dw"], o["db"]))
    o["dw"].fill_(float("nan"))
    torch.cuda.synchronize()
    g2.replay()
    torch.cuda.synchronize()
    assert torch.equal(o["dw"], ref)
