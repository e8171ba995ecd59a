"""transformers generate() through the HIP lattice state (mira_amd.hf_model, the interface of
model/hf_model.py:199-499): greedy tokens equal the argmax of the one-shot forward recomputed
over the whole sequence at every step, and equal mira_amd.generate's (the mirachat loop); beam
search runs through MiraCache.reorder_cache."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_mod():
    import torch

    assert torch.cuda.is_available()
    return torch


def _model(torch, dtype):
    from mira_amd import _lib
    from mira_amd.llm import MiraLLM

    assert _lib.library() is not None, _lib.why()
    torch.manual_seed(21)
    model = MiraLLM(vocab_size=211, n_layer=3, n_embd=64, lattice_d_e=96, lattice_order=2,
                    coefficient_bottleneck=16, memory_dimension=32, ffn_hidden=128)
    with torch.no_grad():
        for value in model.parameters():
            if value.dim() == 2:
                value.normal_(0.0, 1.0 / np.sqrt(value.shape[1]))
    return model.to("cuda", dtype).eval()


def test_greedy_generate_equals_one_shot_recompute(torch_mod):
    torch = torch_mod
    from mira_amd.hf_model import MiraForCausalLM

    model = _model(torch, torch.float32)
    hf = MiraForCausalLM.from_mira(model).eval()
    ids = torch.tensor(np.random.default_rng(3).integers(0, 211, (3, 11)), device="cuda")
    with torch.no_grad():
        got = hf.generate(ids, attention_mask=torch.ones_like(ids), max_new_tokens=12,
                          do_sample=False, pad_token_id=0)
        want = ids
        for _ in range(12):
            logits = model(want).logits[:, -1]
            want = torch.cat([want, logits.argmax(-1, keepdim=True)], dim=1)
    assert torch.equal(got, want)


def test_hf_generate_matches_the_decode_loop_in_bf16(torch_mod):
    torch = torch_mod
    from mira_amd.generate import generate
    from mira_amd.hf_model import MiraForCausalLM

    model = _model(torch, torch.bfloat16)
    hf = MiraForCausalLM.from_mira(model).eval()
    ids = torch.tensor(np.random.default_rng(4).integers(0, 211, (2, 9)), device="cuda")
    with torch.no_grad():
        got = hf.generate(ids, max_new_tokens=10, do_sample=False, pad_token_id=0)
    assert torch.equal(got[:, ids.shape[1]:], generate(model, ids, 10))


def test_beam_search_reorders_the_state(torch_mod):
    torch = torch_mod
    from mira_amd.hf_model import MiraCache, MiraForCausalLM

    model = _model(torch, torch.float32)
    hf = MiraForCausalLM.from_mira(model).eval()
    calls = []
    original = MiraCache.reorder_cache

    def counting(self, beam_idx):
        calls.append(beam_idx.numel())
        return original(self, beam_idx)

    MiraCache.reorder_cache = counting
    try:
        ids = torch.tensor([[5, 17, 42, 7]], device="cuda")
        with torch.no_grad():
            out = hf.generate(ids, max_new_tokens=6, num_beams=3, do_sample=False,
                              pad_token_id=0, early_stopping=True)
    finally:
        MiraCache.reorder_cache = original
    assert out.shape[0] == 1 and out.shape[1] == 10
    assert torch.equal(out[:, :4], ids)
