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


def _hip_runtime():
    """The HIP runtime already mapped into this process (torch's, which the
    library shares through its soname)."""
    import ctypes
    paths = sorted({l.split()[-1] for l in open("/proc/self/maps") if "libamdhip64" in l})
    assert len(paths) == 1, f"expected one HIP runtime in the process, found {paths}"
    rt = ctypes.CDLL(paths[0])
    rt.hipMemGetAddressRange.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.POINTER(ctypes.c_size_t),
                                         ctypes.c_void_p]
    rt.hipMemGetAddressRange.restype = ctypes.c_int
    return rt


def _ws_info(stream):
    import ctypes
    from volta_amd import lib
    p, b, r = ctypes.c_void_p(), ctypes.c_size_t(), ctypes.c_size_t()
    assert lib().vh_workspace_info(ctypes.c_void_p(stream.cuda_stream), ctypes.byref(p), ctypes.byref(b),
                                   ctypes.byref(r)) == 0
    return p.value, b.value, r.value


def test_workspace_retire_rule():
    """The rule that keeps captured graphs valid, pinned on the allocations
    themselves: a workspace that a captured call used is retired when the
    stream's workspace grows (it stays a live allocation of its full size, and
    a replay still reproduces the eager result), while one that no capture
    used is freed on growth (the retired count does not change).  A library
    that freed every outgrown workspace fails the first part; one that
    retired every outgrown workspace (unbounded memory) fails the second."""
    import ctypes
    rt = _hip_runtime()
    conv, x, dy, o = _layer(64, 64, 3, 1, 1, 2, 14, seed=21)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())

    def wgrad(layer, xx, gg, oo):
        layer.backward(gg, xx, input_grad=False, weight_grad=True, algo=layer.algo, outs=(None, oo["dw"], oo["db"]))

    with torch.cuda.stream(s):
        wgrad(conv, x, dy, o)
    torch.cuda.synchronize()
    ref = o["dw"].clone()
    p1, b1, r0 = _ws_info(s)
    assert p1 and b1 > 0, "the weight gradient should take split-K workspace"
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        wgrad(conv, x, dy, o)
    torch.cuda.synchronize()
    assert _ws_info(s)[0] == p1, "a capture must not move the workspace"

    # larger layers, run eagerly on `s` one after the other until the workspace grows
    cands = iter([(64, 64, 16, 56), (128, 128, 32, 28), (256, 256, 32, 14), (256, 256, 128, 14),
                  (128, 128, 128, 28), (64, 64, 128, 56)])

    def grow():
        before = _ws_info(s)
        for i, (C, O, n, h) in enumerate(cands):
            layer, xx, gg, oo = _layer(C, O, 3, 1, 1, n, h, seed=22 + i)
            with torch.cuda.stream(s):
                wgrad(layer, xx, gg, oo)
            torch.cuda.synchronize()
            if _ws_info(s)[1] > before[1]:
                return _ws_info(s)
        raise AssertionError("no candidate layer grew the workspace")

    # growth after a capture: p1 retired, still allocated in full
    p2, b2, r1 = grow()
    assert p2 != p1 and b2 > b1
    assert r1 == r0 + 1, "the workspace a captured call used must be retired"
    base, size = ctypes.c_void_p(), ctypes.c_size_t()
    assert rt.hipMemGetAddressRange(ctypes.byref(base), ctypes.byref(size), ctypes.c_void_p(p1)) == 0, \
        "the captured graph's workspace was freed"
    assert base.value == p1 and size.value >= b1
    o["dw"].fill_(float("nan"))
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    assert torch.equal(o["dw"], ref), "replay after the workspace grew differs from the eager result"

    # growth with no capture in between: p2 is freed, nothing more is retired
    p3, b3, r2 = grow()
    assert b3 > b2
    assert r2 == r1, "an outgrown workspace that no capture used must be freed, not retired"
