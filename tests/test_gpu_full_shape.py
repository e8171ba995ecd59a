"""Value checks at the full BASELINE shapes that the other GPU tests only time.

  * cfg4 decode: batch 256, 128 steps of the conv + diagonal step (state [256, 2048], ring
    [256, 2048, 3]) and the GLA step (state [256, 16, 128, 128]); sampled sequences and heads
    against the fp64 oracle recurrences (oracle/baseline.py), and the whole decode against the
    prefill kernels over the same 128 tokens (decode-N == prefill).
  * cfg5's scan call: matrix_lattice_iir at B=4 T=2048 C=2048 K=2 d_m=64 bf16 with a carried-in
    state (256-token chunks, the matrix-core summary); sampled channels against the fp64 oracle
    (channels are independent given the shared write and read vectors).
  * the cfg5 stack itself: 24 MiraBlocks at d_model 2048, prompt then single-token steps through a
    PrefixCache against the one-shot forward (float32).
Tolerances: bf16 outputs scaled <= 2e-2 against the oracle on the rounded inputs; fp32 states
scaled <= 1e-4 (1e-3 for the lattice state after 2,048 tokens).
"""
import numpy as np
import pytest

from _util import HALF_SCALED, rounded, scaled, to_numpy
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


def test_cfg4_decode_full_shape(torch_mod, plugin):
    torch = torch_mod
    B, D, H, d, N = 256, 2048, 16, 128, 128
    bf = torch.bfloat16
    g = torch.Generator(device="cuda").manual_seed(40)
    h0 = torch.randn(B, D, device="cuda", generator=g) * 0.1
    ring0 = (torch.randn(B, D, 3, device="cuda", generator=g) * 0.1).to(bf)
    w = torch.randn(D, 4, device="cuda", generator=g) * 0.5
    bias = torch.randn(D, device="cuda", generator=g) * 0.1
    x = torch.randn(N, B, D, device="cuda", generator=g).to(bf)
    a = torch.sigmoid(torch.rand(N, B, D, device="cuda", generator=g) * 4 + 2).to(bf)
    S0 = torch.randn(B, H, d, d, device="cuda", generator=g) * 0.1
    q = torch.nn.functional.normalize(torch.randn(N, B, H, d, device="cuda", generator=g), dim=-1).to(bf)
    k = torch.nn.functional.normalize(torch.randn(N, B, H, d, device="cuda", generator=g), dim=-1).to(bf)
    v = torch.randn(N, B, H, d, device="cuda", generator=g).to(bf)
    gd = torch.rand(N, B, H, device="cuda", generator=g) * -0.099 - 0.001
    pos0 = 3                                    # the ring holds three earlier tokens

    h, ring, S = h0.clone(), ring0.clone(), S0.clone()
    ys, os_ = [], []
    for t in range(N):
        ys.append(plugin.diag_conv_step(x[t], a[t], w, bias, h, ring, pos=pos0 + t))
        os_.append(plugin.gla_step(q[t], k[t], v[t], gd[t], S))
    y, o = torch.stack(ys, 1), torch.stack(os_, 1)            # [B, N, D], [B, N, H, d]
    torch.cuda.synchronize()

    # sampled sequences and heads against the fp64 recurrences
    seqs, heads = [0, 97, 255], [0, 9, 15]
    xs = to_numpy(x[:, seqs].transpose(0, 1))
    as_ = to_numpy(a[:, seqs].transpose(0, 1))
    want_y, want_h, want_ring = Bl.diag_conv_scan(xs, as_, to_numpy(w), to_numpy(bias),
                                                  to_numpy(h0[seqs]), to_numpy(ring0[seqs]),
                                                  pos0)
    assert scaled(to_numpy(y[seqs]), want_y) <= HALF_SCALED
    assert scaled(to_numpy(h[seqs]), want_h) <= 1e-4
    assert np.array_equal(to_numpy(ring[seqs]), want_ring)
    pick = lambda t: to_numpy(t[:, seqs][:, :, heads].transpose(0, 1))  # noqa: E731
    want_o, want_S = Bl.gla_recurrent(pick(q), pick(k), pick(v),
                                      to_numpy(gd[:, seqs][:, :, heads].transpose(0, 1)),
                                      to_numpy(S0[seqs][:, heads]))
    assert scaled(to_numpy(o[seqs][:, :, heads]), want_o) <= HALF_SCALED
    assert scaled(to_numpy(S[seqs][:, heads]), want_S) <= 1e-4

    # decode-128 == prefill of the same tokens from the same states, at the full shape
    y_pre, h_pre, ring_pre = plugin.diag_conv_scan(
        x.transpose(0, 1).contiguous(), a.transpose(0, 1).contiguous(), w, bias, h0=h0,
        ring=ring0.clone(), pos=pos0, return_state=True)
    assert scaled(to_numpy(y_pre), to_numpy(y)) <= 1e-2
    assert scaled(to_numpy(h_pre), to_numpy(h)) <= 1e-4
    assert torch.equal(ring_pre, ring)
    o_pre, S_pre = plugin.gla_chunked(q.transpose(0, 1).contiguous(), k.transpose(0, 1).contiguous(),
                                      v.transpose(0, 1).contiguous(), gd.transpose(0, 1).contiguous(),
                                      state=S0, return_state=True)
    assert scaled(to_numpy(o_pre), to_numpy(o)) <= HALF_SCALED
    assert scaled(to_numpy(S_pre), to_numpy(S)) <= 1e-4


def test_cfg5_scan_full_shape(torch_mod, plugin):
    torch = torch_mod
    from mira_amd import _lib

    B, T, C, K, M = 4, 2048, 2048, 2, 64
    assert _lib.require().mira_lattice_plan_chunk(B, T, C, K, M) == 256
    rng = np.random.default_rng(41)
    values = L.random_inputs(rng, B, T, C, K, M)
    state = (rng.standard_normal((B, K, C, M)) * 0.1).astype(np.float32)
    valid = rng.random((B, T)) > 0.05
    bf = torch.bfloat16
    dev = [torch.from_numpy(v).to("cuda", bf) for v in values]
    y, final = plugin.matrix_lattice_iir(*dev[:6], raw_beta=dev[6],
                                         valid=torch.from_numpy(valid).cuda(),
                                         state=torch.from_numpy(state).cuda(), return_state=True)
    torch.cuda.synchronize()
    channels = [0, 1023, 2047]
    seen = [rounded(v, bf) for v in values]
    x, alpha, rho, gamma, write, read, beta = seen
    want_y, want_state = L.lattice_scan_sequential(
        x[:, :, channels], alpha[:, :, channels], rho[:, :, channels], gamma[:, :, channels],
        write, read, beta[:, :, channels], valid=valid, state=state[:, :, channels],
        arch="cauchy_x_hyperbolic", dtype=np.float64)
    assert scaled(to_numpy(y[:, :, channels]), want_y) <= HALF_SCALED
    assert scaled(to_numpy(final[:, :, channels]), want_state) <= 1e-3


def test_cfg5_model_stepped_equals_one_shot(torch_mod, plugin):
    """The 24-layer d_model 2048 stack (BASELINE configs[4] geometry: d_e 2048, K 2, d_m 64,
    d_r 128, FFN 8192, vocab 32000), float32: a 40-token prompt then 8 single-token steps through
    a PrefixCache give the one-shot forward's logits."""
    torch = torch_mod
    from mira_amd.llm import MiraLLM
    from mira_amd.prefix_cache import PrefixCache

    with torch.device("cuda"):
        torch.manual_seed(42)
        model = MiraLLM(vocab_size=32000, n_layer=24, n_embd=2048, lattice_d_e=2048,
                        lattice_order=2, memory_dimension=64, coefficient_bottleneck=128,
                        ffn_hidden=8192).eval()
    ids = torch.randint(0, 32000, (2, 48), device="cuda",
                        generator=torch.Generator(device="cuda").manual_seed(43))
    with torch.no_grad():
        full = model(ids).logits
        cache = PrefixCache(24, budget=0)
        parts = [model(ids[:, :40], cache=cache).logits]
        for t in range(40, 48):
            parts.append(model(ids[:, t:t + 1], cache=cache).logits)
    stepped = torch.cat(parts, dim=1)
    error = scaled(to_numpy(stepped), to_numpy(full))
    del model
    torch.cuda.empty_cache()
    assert error <= 1e-4, f"stepped vs one-shot: scaled error {error:.3e}"
