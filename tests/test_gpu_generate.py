"""Decoding through the prefix cache on the GPU (mira_amd.generate, the reference's streaming
consumer mirachat.py:753-849, batched): greedy tokens agree with one-shot forwards over the
growing sequence, the HIP-graph replay of the single-token step gives the same tokens and logits
as eager steps, seeded sampling is reproducible, and a row that emits eos keeps emitting it."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

CFG = dict(vocab_size=61, n_layer=2, n_embd=64, lattice_d_e=96, lattice_order=2,
           coefficient_bottleneck=16, memory_dimension=32, ffn_hidden=128)


@pytest.fixture(scope="module")
def torch_mod():
    import torch

    assert torch.cuda.is_available()
    return torch


@pytest.fixture(scope="module")
def parts():
    from mira_amd import _lib
    from mira_amd.generate import generate
    from mira_amd.llm import MiraLLM

    assert _lib.library() is not None, _lib.why()
    return MiraLLM, generate


def _model(torch, MiraLLM, seed):
    torch.manual_seed(seed)
    model = MiraLLM(**CFG)
    with torch.no_grad():
        for name, value in model.named_parameters():
            if name.endswith("weight") and value.dim() == 2:
                value.normal_(0.0, 1.5 / np.sqrt(value.shape[1]))
    return model.cuda().eval()


def test_greedy_tokens_match_one_shot_forwards(torch_mod, parts):
    torch = torch_mod
    MiraLLM, generate = parts
    model = _model(torch, MiraLLM, 0)
    prompt = torch.tensor(np.random.default_rng(1).integers(0, CFG["vocab_size"], (3, 9)),
                          device="cuda")
    tokens = generate(model, prompt, 12)
    assert tokens.shape == (3, 12)
    with torch.no_grad():
        logits = model(torch.cat([prompt, tokens], dim=1)).logits.float()
    for i in range(12):
        row = logits[:, prompt.shape[1] - 1 + i]
        chosen = row.gather(1, tokens[:, i:i + 1])[:, 0]
        # the token stepped through the cache is the one-shot argmax, up to fp32 rounding ties
        assert torch.all(chosen >= row.max(dim=1).values - 1e-4 * row.abs().max()), f"step {i}"


def test_graph_replay_equals_eager_steps(torch_mod, parts):
    torch = torch_mod
    MiraLLM, generate = parts
    model = _model(torch, MiraLLM, 2)
    prompt = torch.tensor(np.random.default_rng(3).integers(0, CFG["vocab_size"], (4, 7)),
                          device="cuda")
    seen = {}

    def keep(name):
        def hook(tokens):
            seen.setdefault(name, []).append(tokens[:, -1].clone())
        return hook

    eager = generate(model, prompt, 10, on_token=keep("eager"))
    kept = [block.mixer.__dict__["_packed_projection"]["tensors"] for block in model.blocks]
    replayed = generate(model, prompt, 10, graph=True, on_token=keep("graph"))
    assert torch.equal(eager, replayed)
    # the packed input weights serve the warm-up's stream and the capture as they are: nothing
    # is rebuilt, so the captured step holds no weight copies
    for block, before in zip(model.blocks, kept):
        after = block.mixer.__dict__["_packed_projection"]["tensors"]
        assert all(a is b for a, b in zip(after, before))
    assert len(seen["eager"]) == len(seen["graph"]) == 10
    assert all(torch.equal(a, b) for a, b in zip(seen["eager"], seen["graph"]))
    again = generate(model, prompt, 10, graph=True)
    assert torch.equal(again, eager)


def test_seeded_sampling_is_reproducible_and_eos_sticks(torch_mod, parts):
    torch = torch_mod
    MiraLLM, generate = parts
    model = _model(torch, MiraLLM, 4)
    prompt = torch.tensor(np.random.default_rng(5).integers(0, CFG["vocab_size"], (5, 4)),
                          device="cuda")
    draws = [generate(model, prompt, 16, temperature=1.3, top_k=20, top_p=0.9,
                      generator=torch.Generator(device="cuda").manual_seed(9)) for _ in range(2)]
    assert torch.equal(draws[0], draws[1])
    eos = int(draws[0][0, 3])                 # a token the first row emits at step 3
    cut = generate(model, prompt, 16, temperature=1.3, top_k=20, top_p=0.9, eos_id=eos,
                   generator=torch.Generator(device="cuda").manual_seed(9))
    for row in cut:
        hits = (row == eos).nonzero()
        if len(hits):
            assert torch.all(row[int(hits[0]):] == eos)
    assert torch.all(cut[0, 3:] == eos)
