"""HuggingFace bridge over the MI355X MiraLLM: the interface of model/hf_model.py (MiraConfig
:139-196, MiraCache :199-321, MiraForCausalLM :381-499), so `transformers` generate() -- greedy,
sampling, beam search, streamers -- decodes through the HIP lattice state.

* MiraConfig carries the model's own geometry (`mira_cfg`, mira_amd.llm.MiraLLM's keywords)
  and nothing transformer-shaped: no head count; width and depth are derived properties.
* MiraCache is the prefix cache dressed as a transformers Cache: the trunk reads and writes it
  through get / put / advance / within_budget / key_valid (what mira_amd.mixer and
  mira_amd.llm call), generate() through get_seq_length / reorder_cache / update. The state is
  one fp32 [B, K, d_e, d_m] tensor per layer and does not grow, so it has no maximum length and
  cannot be cropped.
* MiraForCausalLM holds a MiraLLM under `mira.` and feeds generate() the prompt once, then only
  the tokens the cache has not absorbed (a recurrence must not see a token twice). An all-ones
  attention mask is passed on as no mask.

Checkpoint conversion from the reference's training checkpoints and the BPE tokenizer wrapper
are outside this path; `MiraForCausalLM.from_mira` wraps a model already in memory, and
save_pretrained / from_pretrained work as for any PreTrainedModel.
"""
from __future__ import annotations

import inspect

import torch
import torch.nn as nn
from transformers import GenerationMixin, PretrainedConfig, PreTrainedModel
from transformers.cache_utils import Cache
from transformers.modeling_outputs import CausalLMOutputWithPast

from . import config as run_config
from . import prefix_cache
from .llm import MiraLLM


def model_kwargs(mira_cfg):
    """`mira_cfg` reduced to the keywords MiraLLM takes (vocab_size is the config's own)."""
    accepted = set(inspect.signature(MiraLLM.__init__).parameters) - {"self", "vocab_size",
                                                                     "unused"}
    return {k: v for k, v in dict(mira_cfg or {}).items() if k in accepted}


class MiraConfig(PretrainedConfig):
    """The lattice model's geometry, verbatim: `mira_cfg` holds MiraLLM's constructor keywords
    (n_layer, n_embd, lattice_d_e, lattice_order, memory_dimension, coefficient_bottleneck,
    ffn_hidden, arch, ...). max_position_embeddings is a ceiling (nothing in the model refers
    to an absolute position), by default INFERENCE["max_context"]."""

    model_type = "mira"
    keys_to_ignore_at_inference = ["past_key_values"]

    @property
    def hidden_size(self):
        return int(self.mira_cfg.get("n_embd", 0) or 0)

    @property
    def num_hidden_layers(self):
        return int(self.mira_cfg.get("n_layer", 0) or 0)

    def __init__(self, mira_cfg=None, vocab_size=50259, tie_word_embeddings=True,
                 max_position_embeddings=None, **kw):
        for derived in ("hidden_size", "num_hidden_layers", "num_attention_heads"):
            kw.pop(derived, None)                 # derived here; an old config.json may carry them
        self.mira_cfg = dict(mira_cfg or {})
        self.vocab_size = int(self.mira_cfg.get("vocab_size", vocab_size) or vocab_size)
        ceiling = run_config.INFERENCE.get("max_context", 262144)
        self.max_position_embeddings = int(ceiling if max_position_embeddings is None
                                           else max_position_embeddings)
        super().__init__(tie_word_embeddings=bool(tie_word_embeddings), **kw)


class MiraCache(Cache):
    """The lattice state behind both interfaces (see the module docstring)."""

    def __init__(self, layers, model, budget=None):
        try:
            super().__init__(layers=[])
        except Exception:                          # the base class's signature varies by release
            pass
        self.model = model
        self._inner = prefix_cache.PrefixCache(int(layers), budget=budget)
        self.key_valid = None
        self.in_place = False

    # -- the trunk's interface (mira_amd.mixer, mira_amd.llm) --------------------------------
    def __len__(self):
        return self._inner.tokens                 # tokens absorbed, as the trunk reads len()

    def get(self, layer):
        return self._inner.get(layer)

    def put(self, layer, state):
        return self._inner.put(layer, state)

    def advance(self, tokens):
        self._inner.advance(tokens)

    def within_budget(self):
        return self._inner.within_budget()

    def nbytes(self):
        return self._inner.nbytes()

    def clear_states(self):
        self._inner.clear_states()
        self.key_valid = None

    def reset(self):
        self._inner.reset(self.model)
        self.key_valid = None

    # -- the transformers interface --------------------------------------------------------
    def get_seq_length(self, layer_idx=0):
        return self._inner.tokens

    def get_max_cache_shape(self, layer_idx=0):
        return None                               # no length at which the state stops fitting

    def get_max_length(self):
        return None

    @property
    def is_compileable(self):
        return False

    def update(self, key_states, value_states, layer_idx, cache_kwargs=None):
        """Nothing passes keys and values through here: the mixer writes the state itself."""
        return key_states, value_states

    def reorder_cache(self, beam_idx):
        """Beams reorder the batch; every layer's state moves with its beam."""
        for layer in range(self._inner.layers):
            state = self._inner.get(layer)
            if state is not None:
                self._inner.put(layer, state.index_select(0, beam_idx.to(state.device)))
        if self.key_valid is not None:
            self.key_valid = self.key_valid.index_select(0, beam_idx.to(self.key_valid.device))
        return self

    def batch_select_indices(self, indices):
        self.reorder_cache(indices)

    def to_legacy_cache(self):
        return self

    def crop(self, max_length):
        raise NotImplementedError(
            "MiraCache cannot be cropped: every token so far is folded into the same K state "
            f"matrices per layer, so there is no newest part to drop (asked for {max_length})")


class MiraForCausalLM(PreTrainedModel, GenerationMixin):
    """MiraLLM behind PreTrainedModel; the trunk is held as `self.mira`."""

    config_class = MiraConfig
    base_model_prefix = "mira"
    _no_split_modules = ["MiraBlock"]
    # the head is the embedding matrix (MiraLLM ties them); saved once, re-tied on load
    _tied_weights_keys = {"mira.head.weight": "mira.tok.weight"}

    def __init__(self, config):
        super().__init__(config)
        self.mira = MiraLLM(vocab_size=config.vocab_size, **model_kwargs(config.mira_cfg))
        self.post_init()

    def _init_weights(self, module):
        """MiraLLM initialises itself in its constructor; loading overwrites everything."""

    @classmethod
    def from_mira(cls, model):
        """Wrap a MiraLLM already in memory (its parameters are shared, not copied)."""
        cfg = dict(model.cfg)
        wrapper = cls(MiraConfig(mira_cfg=cfg, vocab_size=cfg["vocab_size"]))
        wrapper.mira = model
        return wrapper.to(next(model.parameters()).device)

    def get_input_embeddings(self):
        return self.mira.tok

    def set_input_embeddings(self, value):
        self.mira.tok = value

    def get_output_embeddings(self):
        return self.mira.head

    def set_output_embeddings(self, value):
        self.mira.head = value

    def _new_cache(self):
        """A MiraCache for this trunk, or the reason there is none (model/hf_model.py:429-448)."""
        if not prefix_cache.enabled():
            raise ValueError("use_cache was asked for but INFERENCE['prefix_cache'] is 0, so the "
                             "lattice state cannot be carried between calls; set it to 1, or pass "
                             "use_cache=False and re-run the prefix at every step")
        return MiraCache(len(self.mira.blocks), model=self.mira)

    @classmethod
    def _supports_default_dynamic_cache(cls):
        return False                              # a DynamicCache holds keys and values; no use

    def _prepare_cache_for_generation(self, generation_config, model_kwargs, *args, **kwargs):
        """generate() starts from a MiraCache unless the caller passed a cache or asked for none."""
        if model_kwargs.get("past_key_values") is None and generation_config.use_cache is not False:
            model_kwargs["past_key_values"] = self._new_cache()

    def prepare_inputs_for_generation(self, input_ids, past_key_values=None, attention_mask=None,
                                      use_cache=True, **kw):
        """The whole prompt once, then only the tokens the cache has not absorbed."""
        seen = past_key_values.get_seq_length() if past_key_values is not None else 0
        if seen and input_ids.shape[1] > seen:
            input_ids = input_ids[:, seen:]
        return {"input_ids": input_ids, "past_key_values": past_key_values,
                "attention_mask": attention_mask, "use_cache": bool(use_cache)}

    def _reorder_cache(self, past_key_values, beam_idx):
        return past_key_values.reorder_cache(beam_idx)

    @staticmethod
    def _real_mask(attention_mask):
        """An all-ones mask is no mask: the scan then runs without the per-token flag."""
        if attention_mask is None:
            return None
        return None if bool(attention_mask.all()) else attention_mask.bool()

    def forward(self, input_ids=None, attention_mask=None, labels=None, past_key_values=None,
                use_cache=None, inputs_embeds=None, output_attentions=None,
                output_hidden_states=None, return_dict=None, **unused):
        if inputs_embeds is not None:
            raise NotImplementedError("MiraForCausalLM takes input_ids; the trunk embeds them")
        if output_attentions:
            raise ValueError("this architecture has no attention to report: each layer carries a "
                             "lattice state, not queries, keys and values")
        if use_cache and past_key_values is None:
            past_key_values = self._new_cache()
        if past_key_values is not None and not isinstance(past_key_values, MiraCache):
            raise TypeError(f"MiraForCausalLM decodes through a MiraCache, not "
                            f"{type(past_key_values).__name__}")
        hidden = self.mira.hidden_states(input_ids, attention_mask=self._real_mask(attention_mask),
                                         cache=past_key_values)
        logits = self.mira.head(hidden)
        loss = None
        if labels is not None:
            # per sequence: the mean negative log-likelihood of its own predicted tokens, then
            # the mean over the batch (model/lm.py:151-170)
            target = labels[:, 1:]
            weight = (target != -100).to(torch.float32)
            log_probs = nn.functional.log_softmax(logits.float(), -1)[:, :-1]
            picked = log_probs.gather(-1, target.masked_fill(target == -100, 0).unsqueeze(-1))
            per_sequence = -(picked.squeeze(-1) * weight).sum(1) / weight.sum(1).clamp_min(1.0)
            loss = per_sequence.mean()
        if return_dict is False:
            return (logits,) if loss is None else (loss, logits)
        return CausalLMOutputWithPast(loss=loss, logits=logits, past_key_values=past_key_values,
                                      hidden_states=(hidden,) if output_hidden_states else None,
                                      attentions=None)
