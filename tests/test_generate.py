"""CPU checks of the decoding rule (mira_amd.generate.sample, mirachat.py:824-838): greedy at
temperature 0, top-k keeps the k largest, top-p keeps the smallest head of the sorted
distribution whose mass before each kept token is <= p (always the top token), and the draw
follows the renormalised distribution."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")


def _sample():
    from mira_amd.generate import sample
    return sample


def test_temperature_zero_is_argmax():
    logits = torch.randn(6, 50, generator=torch.Generator().manual_seed(0))
    assert torch.equal(_sample()(logits, temperature=0.0), logits.argmax(dim=-1))


def test_top_k_one_is_argmax_at_any_temperature():
    g = torch.Generator().manual_seed(1)
    logits = torch.randn(8, 40, generator=g)
    for _ in range(5):
        assert torch.equal(_sample()(logits, temperature=3.0, top_k=1, generator=g),
                           logits.argmax(dim=-1))


def test_top_p_keeps_the_head_and_always_the_top_token():
    g = torch.Generator().manual_seed(2)
    # probabilities 0.5, 0.3, 0.15, 0.05: top_p = 0.6 keeps {0, 1} (mass before 1 is 0.5 <= 0.6,
    # before 2 is 0.8 > 0.6); top_p = 0.01 keeps {0} only
    probs = torch.tensor([[0.05, 0.5, 0.15, 0.3]])
    logits = probs.log().repeat(4000, 1)
    draws = _sample()(logits, temperature=1.0, top_p=0.6, generator=g)
    counts = np.bincount(draws.numpy(), minlength=4)
    assert counts[0] == 0 and counts[2] == 0
    share = counts[1] / counts.sum()                      # 0.5 / 0.8 = 0.625
    assert abs(share - 0.625) < 4 * np.sqrt(0.625 * 0.375 / 4000)
    only = _sample()(logits[:100], temperature=1.0, top_p=0.01, generator=g)
    assert torch.all(only == 1)


def test_draws_follow_the_tempered_distribution():
    g = torch.Generator().manual_seed(3)
    base = torch.tensor([[0.0, 1.0, 2.0]])
    logits = base.repeat(6000, 1)
    draws = _sample()(logits, temperature=2.0, generator=g)
    want = torch.softmax(base[0] / 2.0, dim=0).numpy()
    got = np.bincount(draws.numpy(), minlength=3) / 6000
    assert np.all(np.abs(got - want) < 4 * np.sqrt(want * (1 - want) / 6000))
