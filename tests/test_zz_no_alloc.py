"""The allocation-free norm backward (sfp8_norm_bwd_noalloc) against the
workspace form (sfp8_norm_bwd) through the C ABI: dh, d_norm_w, the e5m2
dy8 (K-slab of [T, D]) or dy8t (token-contiguous copy) and amax slot 4
bit-identical, on two calls in a row (the second smaller, so the fixed
scratch holds the first call's partials when it starts), and a too-large
shape refused before anything is launched."""
import pytest
import torch

import spark_gpt_amd as sg
from spark_gpt_amd import _lib, ops

pytestmark = pytest.mark.gpu


def _noalloc():
    return _lib.load().sfp8_norm_bwd_noalloc  # argument types from _lib.SIGNATURES


def _inputs(dev, T, D, seed):
    g = torch.Generator(device=dev).manual_seed(seed)
    h = torch.randn(T, D, generator=g, device=dev).to(torch.bfloat16)
    dxn = torch.randn(T, D, generator=g, device=dev).to(torch.bfloat16)
    dy = (torch.randn(T, D, generator=g, device=dev) * 1e-3).to(torch.bfloat16)
    rstd = torch.rand(T, generator=g, device=dev) + 0.5
    nw = torch.rand(D, generator=g, device=dev) + 0.5
    scale = torch.tensor([1, 1, 1, 1, 2.0 ** 15], device=dev)
    return h, dxn, dy, rstd, nw, scale


def _run_noalloc(fn, h, dxn, dy, rstd, nw, scale, rows):
    T, D = h.shape
    ldt = ops.ldt_of(T)
    amax = torch.zeros(5, device=h.device)
    dh = torch.empty(T, D, dtype=torch.bfloat16, device=h.device)
    dnw = torch.empty(D, device=h.device)
    dy8 = ops.kslab_empty(ldt, D, ops.E5M2, h.device) if rows else ops.slab_empty(D, T, ops.E5M2, h.device)
    torch.cuda.synchronize()  # every buffer above exists before the call (no allocation after it)
    rc = fn(h.data_ptr(), rstd.data_ptr(), dxn.data_ptr(), dy.data_ptr(), nw.data_ptr(), T, D, scale.data_ptr(),
            amax.data_ptr(), dh.data_ptr(), dnw.data_ptr(), dy8.data_ptr() if rows else None,
            None if rows else dy8.data_ptr(), ldt, _lib.stream_of(h))
    assert rc == 0, rc
    return dh, dnw, dy8, amax


@pytest.mark.parametrize("rows", [True, False])
@pytest.mark.parametrize("shapes", [((1000, 1024), (300, 1024)), ((4096, 256), (257, 256)),
                                    ((65536, 1024), (1000, 1024))])
def test_noalloc_matches_workspace_form(dev, shapes, rows):
    fn = _noalloc()
    for k, (T, D) in enumerate(shapes):
        args = _inputs(dev, T, D, 100 + k)
        got = _run_noalloc(fn, *args, rows)
        h, dxn, dy, rstd, nw, scale = args
        amax = torch.zeros(5, device=dev)
        ref = ops.norm_bwd(h, rstd, dxn, dy, nw, scale, amax, rows=rows) + (amax,)
        torch.cuda.synchronize()
        for name, a, b in zip(("dh", "dnw", "dy8", "amax"), got, ref):
            assert torch.equal(a.view(torch.uint8) if a.dtype == ops.E5M2 else a,
                               b.view(torch.uint8) if b.dtype == ops.E5M2 else b), (T, D, name)


def test_noalloc_refuses_beyond_scratch(dev):
    fn = _noalloc()
    D, ldt = 4096, 65536
    need = _lib.query("sfp8_norm_bwd_partials", D, ldt) * D
    assert need > 8 << 20  # SFP8_NOALLOC_SCRATCH_FLOATS
    # refused on the host (non-null stand-in pointers are never dereferenced)
    assert fn(16, 16, 16, 16, 16, ldt, D, 16, 16, 16, 16, 16, None, ldt, None) == -5


def test_noalloc_under_graph_capture(dev):
    """The entry point as a captured HIP graph: after one eager call on the
    device (which looks up the scratch address), a capture of one call
    replays with the bytes of sfp8_norm_bwd on whatever the static inputs
    hold at each replay.  Each replay is checked against its own eager
    result, with eager work and synchronisations between the replays; the
    graph holds only kernel launches (no memset nodes)."""
    fn = _noalloc()
    T, D = 4096, 1024
    h, dxn, dy, rstd, nw, scale = _inputs(dev, T, D, 7)
    ldt = ops.ldt_of(T)
    amax = torch.zeros(5, device=dev)
    dh = torch.empty(T, D, dtype=torch.bfloat16, device=dev)
    dnw = torch.empty(D, device=dev)
    dy8t = ops.slab_empty(D, T, ops.E5M2, dev)
    args = lambda: (h.data_ptr(), rstd.data_ptr(), dxn.data_ptr(), dy.data_ptr(), nw.data_ptr(), T, D,  # noqa: E731
                    scale.data_ptr(), amax.data_ptr(), dh.data_ptr(), dnw.data_ptr(), None, dy8t.data_ptr(), ldt,
                    _lib.stream_of(h))
    assert fn(*args()) == 0  # eager: resolves this device's scratch address
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            rc = fn(*args())
    torch.cuda.current_stream().wait_stream(side)
    assert rc == 0, rc
    for rep in range(4):
        nh, ndxn, ndy, nrstd, nnw, _ = _inputs(dev, T, D, 200 + rep)
        for dst, src in ((h, nh), (dxn, ndxn), (dy, ndy), (rstd, nrstd), (nw, nnw)):
            dst.copy_(src)
        amax.zero_()
        ref_amax = torch.zeros(5, device=dev)
        ref = ops.norm_bwd(h, rstd, dxn, dy, nw, scale, ref_amax, rows=False)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for name, a, b in zip(("dh", "dnw", "dy8t", "amax"), (dh, dnw, dy8t, amax), ref + (ref_amax,)):
            assert torch.equal(a.view(torch.uint8) if a.dtype == ops.E5M2 else a,
                               b.view(torch.uint8) if b.dtype == ops.E5M2 else b), (rep, name)
