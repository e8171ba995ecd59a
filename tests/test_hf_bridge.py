"""The HuggingFace bridge (mira_amd.hf_model, the interface of model/hf_model.py): transformers'
generate() through MiraCache. On the CPU the scan is the fp64 oracle (so the bridge's plumbing --
prompt once, then only unabsorbed tokens, the cache's two interfaces, beam reordering -- is
checked without a GPU); tests/test_gpu_hf_bridge.py runs the HIP path."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytest.importorskip("transformers")

from mira_amd import config, hf_model  # noqa: E402
from mira_amd import mixer as mixer_module  # noqa: E402
from mira_amd.llm import MiraLLM  # noqa: E402
from oracle import lattice as L  # noqa: E402

CFG = dict(vocab_size=31, n_layer=2, n_embd=16, lattice_d_e=12, lattice_order=2,
           coefficient_bottleneck=4, memory_dimension=8, ffn_hidden=24)


def _oracle_scan(x, raw_alpha, raw_rho, gamma, memory_write, memory_read, raw_beta=None,
                 valid=None, state=None, return_state=False, arch="cauchy_x_hyperbolic",
                 **unused):
    arrays = [t.detach().double().numpy() for t in
              (x, raw_alpha, raw_rho, gamma, memory_write, memory_read, raw_beta)]
    y, final = L.lattice_scan_sequential(
        *arrays, valid=None if valid is None else valid.numpy(),
        state=None if state is None else state.double().numpy(), arch=arch, dtype=np.float64)
    y = torch.from_numpy(y).to(x.dtype)
    return (y, torch.from_numpy(final).float()) if return_state else y


def _oracle_step(x, raw_alpha, raw_rho, gamma, memory_write, memory_read, raw_beta, state,
                 valid=None, arch="cauchy_x_hyperbolic", inplace=False, **unused):
    return _oracle_scan(x, raw_alpha, raw_rho, gamma, memory_write, memory_read, raw_beta,
                        valid=valid, state=state, return_state=True, arch=arch)


@pytest.fixture
def cpu_model(monkeypatch):
    monkeypatch.setattr(mixer_module.plugin, "matrix_lattice_iir", _oracle_scan)
    monkeypatch.setattr(mixer_module.plugin, "matrix_lattice_step", _oracle_step)
    torch.manual_seed(0)
    model = MiraLLM(**CFG).double().eval()
    with torch.no_grad():
        for name, value in model.named_parameters():
            if value.dim() == 2:
                value.normal_(0.0, 1.0 / np.sqrt(value.shape[1]))
    return model


def _greedy_by_recompute(model, ids, new):
    out = ids
    with torch.no_grad():
        for _ in range(new):
            logits = model(out).logits[:, -1]
            out = torch.cat([out, logits.argmax(-1, keepdim=True)], dim=1)
    return out


def test_greedy_generate_equals_recompute(cpu_model):
    hf = hf_model.MiraForCausalLM.from_mira(cpu_model).eval()
    assert hf.config.hidden_size == 16 and hf.config.num_hidden_layers == 2
    ids = torch.tensor(np.random.default_rng(1).integers(0, 31, (2, 7)))
    got = hf.generate(ids, attention_mask=torch.ones_like(ids), max_new_tokens=6,
                      do_sample=False, pad_token_id=0)
    assert torch.equal(got, _greedy_by_recompute(cpu_model, ids, 6))


def test_cache_interfaces(cpu_model):
    hf = hf_model.MiraForCausalLM.from_mira(cpu_model).eval()
    cache = hf._new_cache()
    assert isinstance(cache, hf_model.MiraCache) and cache.get_seq_length() == 0
    ids = torch.tensor([[3, 4, 5, 6]])
    with torch.no_grad():
        out = hf(ids, past_key_values=cache, use_cache=True)
    assert out.past_key_values is cache and len(cache) == 4 and cache.get_seq_length() == 4
    assert cache.get(0).shape == (1, 2, 12, 8) and cache.get_max_cache_shape() is None
    inputs = hf.prepare_inputs_for_generation(torch.tensor([[3, 4, 5, 6, 9]]), cache)
    assert inputs["input_ids"].tolist() == [[9]]
    with pytest.raises(NotImplementedError):
        cache.crop(2)
    two = hf._new_cache()
    with torch.no_grad():
        hf(torch.tensor([[1, 2], [3, 4]]), past_key_values=two, use_cache=True)
    first = two.get(1)[0].clone()
    two.reorder_cache(torch.tensor([1, 0]))
    assert torch.equal(two.get(1)[1], first)
    with pytest.raises(ValueError, match="attention"):
        hf(ids, output_attentions=True)


def test_loss_is_per_sequence_mean(cpu_model):
    hf = hf_model.MiraForCausalLM.from_mira(cpu_model).eval()
    ids = torch.tensor([[1, 2, 3, 4], [5, 6, 7, 8]])
    labels = ids.clone()
    labels[1, :3] = -100                        # the second sequence predicts one token
    with torch.no_grad():
        out = hf(ids, labels=labels)
        log_probs = torch.log_softmax(out.logits.double(), -1)
    first = -log_probs[0, :-1].gather(-1, ids[0, 1:, None]).mean()
    second = -log_probs[1, 2, ids[1, 3]]
    torch.testing.assert_close(out.loss.double(), (first + second) / 2)


def test_switched_off_prefix_cache_is_explained(cpu_model, monkeypatch):
    hf = hf_model.MiraForCausalLM.from_mira(cpu_model).eval()
    monkeypatch.setitem(config.INFERENCE, "prefix_cache", 0)
    with pytest.raises(ValueError, match="prefix_cache"):
        hf(torch.tensor([[1, 2]]), use_cache=True)


def test_save_and_load_round_trip(cpu_model, tmp_path):
    hf = hf_model.MiraForCausalLM.from_mira(cpu_model).eval()
    hf.save_pretrained(tmp_path)
    back = hf_model.MiraForCausalLM.from_pretrained(tmp_path).double().eval()
    ids = torch.tensor([[1, 5, 9, 2]])
    with torch.no_grad():
        torch.testing.assert_close(back(ids).logits, hf(ids).logits)
    assert back.mira.tok.weight is back.mira.head.weight
