"""The decode step captured in a HIP graph (torch.cuda.CUDAGraph over the C-ABI launches).

A serving loop replays the per-token launches (conv + diagonal step, GLA step) as one graph to
drop the per-launch gaps. The step kernels use no workspace and no memset, so a captured step
must equal the eager one bit for bit: the graph is replayed three times, with eager state resets
and synchronisations between the replays, and every replay is checked against one eager run
from the same initial states.
"""
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_mod():
    import torch

    assert torch.cuda.is_available()
    return torch


@pytest.fixture(scope="module")
def plugin():
    from mira_amd import _lib, mira

    assert _lib.library() is not None, _lib.why()
    return mira


@pytest.mark.parametrize("overlap", [False, True], ids=["one_stream", "side_stream"])
def test_decode_steps_replayed_from_a_graph(torch_mod, plugin, overlap):
    """With overlap, each step's conv + diagonal launch goes to a side stream forked from the
    main stream and joined before the next step (the decode bench's launch scheme)."""
    torch = torch_mod
    B, D, H, d, N = 8, 256, 2, 128, 6
    g = torch.Generator(device="cuda").manual_seed(5)
    bf = torch.bfloat16
    xs = torch.randn(N, B, D, device="cuda", generator=g).to(bf)
    as_ = torch.sigmoid(torch.rand(N, B, D, device="cuda", generator=g) * 4 + 2).to(bf)
    w = torch.randn(D, 4, device="cuda", generator=g) * 0.5
    bias = torch.randn(D, device="cuda", generator=g) * 0.1
    normal = torch.nn.functional.normalize
    qs = normal(torch.randn(N, B, H, d, device="cuda", generator=g), dim=-1).to(bf)
    ks = normal(torch.randn(N, B, H, d, device="cuda", generator=g), dim=-1).to(bf)
    vs = torch.randn(N, B, H, d, device="cuda", generator=g).to(bf)
    gs = torch.rand(N, B, H, device="cuda", generator=g) * -0.099 - 0.001
    h0 = torch.randn(B, D, device="cuda", generator=g) * 0.1
    ring0 = (torch.randn(B, D, 3, device="cuda", generator=g) * 0.1).to(bf)
    S0 = torch.randn(B, H, d, d, device="cuda", generator=g) * 0.1

    def run(h, ring, S, ys, os_):
        for t in range(N):
            plugin.diag_conv_step(xs[t], as_[t], w, bias, h, ring, pos=t, out=ys[t])
            plugin.gla_step(qs[t], ks[t], vs[t], gs[t], S, out=os_[t])

    def run_overlapped(h, ring, S, ys, os_):
        main, side = torch.cuda.current_stream(), torch.cuda.Stream()
        for t in range(N):
            side.wait_stream(main)
            with torch.cuda.stream(side):
                plugin.diag_conv_step(xs[t], as_[t], w, bias, h, ring, pos=t, out=ys[t])
            plugin.gla_step(qs[t], ks[t], vs[t], gs[t], S, out=os_[t])
            main.wait_stream(side)

    he, re, Se = h0.clone(), ring0.clone(), S0.clone()
    ye, oe = torch.empty(N, B, D, device="cuda", dtype=bf), torch.empty(N, B, H, d, device="cuda", dtype=bf)
    run(he, re, Se, ye, oe)
    torch.cuda.synchronize()

    hg, rg, Sg = h0.clone(), ring0.clone(), S0.clone()
    yg, og = torch.empty_like(ye), torch.empty_like(oe)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        (run_overlapped if overlap else run)(hg, rg, Sg, yg, og)
    for replay in range(3):
        hg.copy_(h0)
        rg.copy_(ring0)
        Sg.copy_(S0)
        yg.zero_()
        og.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(yg, ye) and torch.equal(og, oe), f"replay {replay}: outputs"
        assert torch.equal(hg, he) and torch.equal(rg, re) and torch.equal(Sg, Se), \
            f"replay {replay}: states"
