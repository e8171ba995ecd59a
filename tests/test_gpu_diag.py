"""GPU parity of the BASELINE conv + diagonal scan (mira_diag_conv_scan / mira_diag_conv_step).

Anchors: the fp64 closed forms of oracle/baseline.py; the reference CPU mixer's own output on
the exact K=1 lattice realisation of the scan (tests/golden/diag_cfg1_reduced.npz, compared as
h = y / 32, exact in float32); and, at BASELINE cfg2's full size, channel subsets checked against
the oracle (channels are independent) plus streaming == one shot. The conv has no reference
counterpart, so its parity with the reference is unpinned; the closed form pins it.
Tolerances: float32 max abs <= 1e-5; bf16/f16 scaled <= 2e-2.
"""
import numpy as np
import pytest

from _util import FP32_ABS, HALF_SCALED, GOLDEN, max_abs, rounded, scaled, to_device, to_numpy
from oracle import baseline as Bl
from oracle import lattice as L

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


def _oracle(x, a, w, h0=None, ring=None, pos=0, dtype="float32", torch=None):
    td = getattr(torch, dtype)
    xs, as_ = rounded(x, td), rounded(a, td)
    rs = None if ring is None else rounded(ring, td)
    return Bl.diag_conv_scan(xs, as_, w, None, h0, rs, pos)


def _check(got, want, dtype, what):
    if dtype == "float32":
        assert max_abs(got, want) <= FP32_ABS, f"{what}: max abs {max_abs(got, want):.3e}"
    else:
        assert scaled(got, want) <= HALF_SCALED, f"{what}: scaled {scaled(got, want):.3e}"


def test_cfg1_fp32_against_closed_form(torch_mod, plugin):
    """BASELINE cfg1: B=1, T=512, D=256, float32, h0 = 0."""
    rng = np.random.default_rng(0)
    x, a, w, bias, _ = Bl.diag_inputs(rng, 1, 512, 256)
    y, hT, _ = plugin.diag_conv_scan(to_device(x), to_device(a), to_device(w), to_device(bias),
                                     return_state=True)
    h, h_last, _ = Bl.diag_conv_scan(x, a, w, bias)
    _check(to_numpy(y), h, "float32", "cfg1 y")
    _check(to_numpy(hT), h_last, "float32", "cfg1 h_T")
    closed = Bl.diag_scan_closed_form(Bl.causal_conv(x, w, bias)[:, :64], a[:, :64])
    _check(to_numpy(y)[:, :64], closed, "float32", "cfg1 closed form")


def test_golden_reference_path(torch_mod, plugin):
    """The reference CPU mixer's output on the K=1, M=1 realisation (y = 32 h)."""
    d = np.load(f"{GOLDEN}/diag_cfg1_reduced.npz")
    y = plugin.diag_conv_scan(to_device(d["x"]), to_device(d["a"]), to_device(d["w"]),
                              to_device(d["bias"]), h0=to_device(d["h0"]))
    _check(to_numpy(y), d["y"] / 32.0, "float32", "vs reference mixer (h = y/32)")


@pytest.mark.parametrize("dtype", ["float32", "bfloat16", "float16"])
@pytest.mark.parametrize("B,T,D", [(1, 1, 4), (2, 3, 8), (3, 63, 60), (2, 64, 64), (2, 65, 128),
                                   (1, 200, 68), (2, 777, 256)])
def test_shapes_and_dtypes(torch_mod, plugin, dtype, B, T, D):
    torch = torch_mod
    rng = np.random.default_rng(B * 1000 + T + D)
    x, a, w, bias, h0 = Bl.diag_inputs(rng, B, T, D, h0_scale=0.1)
    bias = (rng.standard_normal(D) * 0.1).astype(np.float32)
    td = getattr(torch, dtype)
    y, hT, _ = plugin.diag_conv_scan(to_device(x, td), to_device(a, td), to_device(w),
                                     to_device(bias), h0=to_device(h0), return_state=True)
    h, h_last, _ = Bl.diag_conv_scan(rounded(x, td), rounded(a, td), w, bias, h0)
    _check(to_numpy(y), h, dtype, "y")
    assert max_abs(to_numpy(hT), h_last) <= (FP32_ABS if dtype == "float32" else 1e-3)


@pytest.mark.parametrize("dtype", ["float32", "bfloat16", "float16"])
@pytest.mark.parametrize("B,T,D", [(2, 333, 4096), (128, 130, 64), (3, 257, 2900), (64, 1, 128)])
def test_column_form_shapes(torch_mod, plugin, dtype, B, T, D):
    """Batches with at least 128 columns of 64 channels (the column form on a 256-CU part):
    ragged token tails, a partial last column (2900 = 45 x 64 + 20), T = 1, bias and h0."""
    torch = torch_mod
    rng = np.random.default_rng(B * 7 + T * 3 + D)
    x, a, w, bias, h0 = Bl.diag_inputs(rng, B, T, D, h0_scale=0.1)
    bias = (rng.standard_normal(D) * 0.1).astype(np.float32)
    td = getattr(torch, dtype)
    y, hT, _ = plugin.diag_conv_scan(to_device(x, td), to_device(a, td), to_device(w),
                                     to_device(bias), h0=to_device(h0), return_state=True)
    h, h_last, _ = Bl.diag_conv_scan(rounded(x, td), rounded(a, td), w, bias, h0)
    _check(to_numpy(y), h, dtype, "y")
    assert max_abs(to_numpy(hT), h_last) <= (FP32_ABS if dtype == "float32" else 1e-3)
    assert plugin.diag_workspace_error() == 0


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
@pytest.mark.parametrize("T1,T2", [(1, 2), (5, 300), (128, 129)])
def test_column_form_streaming_with_ring(torch_mod, plugin, dtype, T1, T2):
    """The column form carrying h and the ring across calls (the second call updates the ring in
    place) equals one call, and the ring holds the last three tokens."""
    torch = torch_mod
    td = getattr(torch, dtype)
    rng = np.random.default_rng(T1 * 11 + T2)
    B, D = 2, 4096
    x, a, w, bias, h0 = Bl.diag_inputs(rng, B, T1 + T2, D, h0_scale=0.1)
    X, A, W = to_device(x, td), to_device(a, td), to_device(w)
    y_all, h_all, _ = plugin.diag_conv_scan(X, A, W, h0=to_device(h0), return_state=True)
    ring = torch.zeros(B, D, 3, device="cuda", dtype=td)
    y1, h1, ring = plugin.diag_conv_scan(X[:, :T1], A[:, :T1], W, h0=to_device(h0), ring=ring,
                                         pos=0, return_state=True)
    y2, h2, ring = plugin.diag_conv_scan(X[:, T1:], A[:, T1:], W, h0=h1, ring=ring, pos=T1,
                                         return_state=True)
    y_two = to_numpy(torch.cat([y1, y2], 1))
    if dtype == "float32":
        _check(y_two, to_numpy(y_all), dtype, "streamed y")
    else:
        assert scaled(y_two, to_numpy(y_all)) <= 1e-2
    assert max_abs(to_numpy(h2), to_numpy(h_all)) <= 1e-5
    want_ring = Bl.ring_after(rounded(x, td), np.zeros((B, D, 3), np.float32), 0)
    assert np.array_equal(to_numpy(ring), want_ring), "ring after the stream"


@pytest.mark.parametrize("T1,T2", [(1, 1), (2, 5), (64, 64), (100, 37), (3, 300)])
def test_streaming_with_ring(torch_mod, plugin, T1, T2):
    """[0,T1) then [T1,T1+T2) carrying h and the ring equals one call."""
    torch = torch_mod
    rng = np.random.default_rng(T1 * 7 + T2)
    B, D = 2, 64
    x, a, w, bias, h0 = Bl.diag_inputs(rng, B, T1 + T2, D, h0_scale=0.1)
    X, A, W = to_device(x), to_device(a), to_device(w)
    y_all, h_all, _ = plugin.diag_conv_scan(X, A, W, h0=to_device(h0), return_state=True)
    ring = torch.zeros(B, D, 3, device="cuda")
    y1, h1, ring = plugin.diag_conv_scan(X[:, :T1], A[:, :T1], W, h0=to_device(h0), ring=ring,
                                         pos=0, return_state=True)
    y2, h2, ring = plugin.diag_conv_scan(X[:, T1:], A[:, T1:], W, h0=h1, ring=ring, pos=T1,
                                         return_state=True)
    _check(to_numpy(torch.cat([y1, y2], 1)), to_numpy(y_all), "float32", "streamed y")
    _check(to_numpy(h2), to_numpy(h_all), "float32", "streamed h")
    want_ring = Bl.ring_after(x, np.zeros((B, D, 3), np.float32), 0)
    assert np.array_equal(to_numpy(ring), want_ring), "ring after the stream"


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
def test_decode_steps_equal_prefill(torch_mod, plugin, dtype):
    torch = torch_mod
    td = getattr(torch, dtype)
    rng = np.random.default_rng(42)
    B, N, D = 3, 20, 96
    x, a, w, bias, h0 = Bl.diag_inputs(rng, B, N, D, h0_scale=0.1)
    X, A, W, Bs = to_device(x, td), to_device(a, td), to_device(w), to_device(bias)
    y_pre, h_pre, _ = plugin.diag_conv_scan(X, A, W, Bs, h0=to_device(h0), return_state=True)
    h = to_device(h0).clone()
    ring = torch.zeros(B, D, 3, device="cuda", dtype=td)
    outs = []
    for t in range(N):
        outs.append(plugin.diag_conv_step(X[:, t].contiguous(), A[:, t].contiguous(), W, Bs, h,
                                          ring, pos=t))
    got = torch.stack(outs, 1)
    if dtype == "float32":
        _check(to_numpy(got), to_numpy(y_pre), dtype, "decode y")
        _check(to_numpy(h), to_numpy(h_pre), dtype, "decode state")
    else:
        assert scaled(to_numpy(got), to_numpy(y_pre)) <= 1e-2
        assert max_abs(to_numpy(h), to_numpy(h_pre)) <= 1e-5
    want_ring = Bl.ring_after(rounded(x, td), np.zeros((B, D, 3), np.float32), 0)
    assert np.array_equal(to_numpy(ring), want_ring)


def test_cfg2_full_size_bf16(torch_mod, plugin):
    """BASELINE cfg2 at full size: B=8, T=4096, D=2048 bf16 with h0 ~ N(0, 0.1^2). Channels are
    independent, so a subset of channels is checked against the fp64 oracle over the full token
    axis; the whole output against a two-call stream; the watchdog stays 0."""
    torch = torch_mod
    g = torch.Generator(device="cuda").manual_seed(0)
    B, T, D = 8, 4096, 2048
    x = torch.randn(B, T, D, device="cuda", generator=g).to(torch.bfloat16)
    a = torch.sigmoid(torch.rand(B, T, D, device="cuda", generator=g) * 4 + 2).to(torch.bfloat16)
    w = torch.randn(D, 4, device="cuda", generator=g) * 0.5
    h0 = torch.randn(B, D, device="cuda", generator=g) * 0.1
    y, hT, _ = plugin.diag_conv_scan(x, a, w, h0=h0, return_state=True)
    torch.cuda.synchronize()
    cols = np.r_[0:4, 1020:1028, 2044:2048]
    for b in (0, 7):
        xs = to_numpy(x[b:b + 1, :, cols])
        as_ = to_numpy(a[b:b + 1, :, cols])
        h, h_last, _ = Bl.diag_conv_scan(xs, as_, to_numpy(w)[cols], None, to_numpy(h0)[b:b + 1, cols])
        assert scaled(to_numpy(y[b:b + 1, :, cols]), h) <= HALF_SCALED
        assert max_abs(to_numpy(hT[b:b + 1, cols]), h_last) <= 1e-5
    y1, h1, _ = plugin.diag_conv_scan(x[:, :1000], a[:, :1000], w, h0=h0, return_state=True)
    ring = torch.zeros(B, D, 3, device="cuda", dtype=torch.bfloat16)
    ring[:, :, 997 % 3] = x[:, 997]
    ring[:, :, 998 % 3] = x[:, 998]
    ring[:, :, 999 % 3] = x[:, 999]
    y2, h2, _ = plugin.diag_conv_scan(x[:, 1000:], a[:, 1000:], w, h0=h1, ring=ring, pos=1000,
                                      return_state=True)
    assert torch.equal(torch.cat([y1, y2], 1), y) or scaled(
        to_numpy(torch.cat([y1, y2], 1)), to_numpy(y)) <= 1e-2
    assert max_abs(to_numpy(h2), to_numpy(hT)) <= 1e-5
    assert plugin.diag_workspace_error() == 0


def test_reference_path_realisation_matches(torch_mod, plugin):
    """The BASELINE kernel equals the reference operator on the Appendix-B inputs: the lattice
    kernel (K=1, M=1) fed the realisation of the same conv output and decays."""
    rng = np.random.default_rng(9)
    x, a, w, bias, h0 = Bl.diag_inputs(rng, 2, 300, 64, h0_scale=0.1)
    y = plugin.diag_conv_scan(to_device(x), to_device(a), to_device(w), h0=to_device(h0))
    u = Bl.causal_conv(x, w, dtype=np.float32).astype(np.float32)
    lat = Bl.diag_as_lattice(u, a, h0)
    out, _ = plugin.matrix_lattice_iir(*[to_device(v) for v in lat[:6]], raw_beta=to_device(lat[6]),
                                       state=to_device(lat[7]), return_state=True)
    _check(to_numpy(y), to_numpy(out) / 32.0, "float32", "kernel vs lattice realisation")
    ref, _ = L.lattice_scan_batched(*lat[:7], state=lat[7])
    _check(to_numpy(y), ref / 32.0, "float32", "kernel vs oracle of the reference path")


def test_look_back_prefill_refuses_graph_capture(torch_mod, plugin):
    """The look-back form (a batch too narrow for one column per half of the CUs) tags its
    records with a per-launch epoch passed as a kernel argument, which a graph would freeze:
    the library refuses capture (ValueError) instead of replaying stale records. The column
    form takes no epoch and captures normally."""
    torch = torch_mod
    rng = np.random.default_rng(21)
    x, a, w, _, _ = Bl.diag_inputs(rng, 1, 96, 256)
    xd, ad, wd = to_device(x), to_device(a), to_device(w)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        eager = plugin.diag_conv_scan(xd, ad, wd)          # allocates this stream's workspace
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with pytest.raises(ValueError, match="captured"):
        with torch.cuda.graph(graph, stream=side):
            plugin.diag_conv_scan(xd, ad, wd)
    torch.cuda.synchronize()
    want, _, _ = _oracle(x, a, w, torch=torch)
    _check(to_numpy(eager), want, "float32", "eager look-back prefill")
    # a batch wide enough for the column form is captured and replayed like any kernel
    x2, a2, w2, _, _ = Bl.diag_inputs(rng, 8, 40, 2048)
    xd2, ad2, wd2 = to_device(x2), to_device(a2), to_device(w2)
    with torch.cuda.stream(side):
        plugin.diag_conv_scan(xd2, ad2, wd2)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        captured = plugin.diag_conv_scan(xd2, ad2, wd2)
    want2, _, _ = _oracle(x2, a2, w2, torch=torch)
    for _ in range(2):
        graph.replay()
        torch.cuda.synchronize()
        _check(to_numpy(captured), want2, "float32", "captured column prefill")
