"""Drop-ins for the reference's HF-factory model routes: ``llama_*``
(models/llama.py:5-56, transformers LlamaForCausalLM) and ``mistral_*``
(models/mistral.py:5-35, MistralForCausalLM), on this build's decoder layers.

The model hub reads these models through a fixed set of attributes
(models/hub.py: ``get_layers`` -> ``model.model.layers`` at :163 / :183,
``get_embedding_layer`` -> ``model.model.embed_tokens`` at :247 / :267,
``get_layer_attention`` / ``get_layer_feed_forward`` -> ``layer.self_attn`` /
``layer.mlp`` at :276-318, the parameter count over ``model.model.embed_tokens``,
``model.model.norm`` and ``model.lm_head`` at :414-418 / :488-491, and
``hidden_size`` / ``_hidden_size``); the classes here keep exactly those, with
``model.model.layers`` a ModuleList of ``llama_simple.LlamaDecoderLayer`` --
the fused gfx950 layer, one flat parameter each, whose submodule names and
parameter shapes are HF's.  The layer profiler (utils/runtime_estimator.py:
198-243) calls ``layer(embedding)`` and takes ``output[0]``; the layer's
forward takes HF's keyword arguments (``attention_mask`` must be None: the
layer applies the causal / sliding-window mask itself; the rotary tables are
computed from ``position_ids``, and ``position_embeddings`` is ignored).
Initialisation as HF's ``_init_weights`` with initializer_range 0.02: linear
and embedding weights N(0, 0.02), norm weights 1.

Shapes, as the factories set them:
  * llama_*: LlamaConfig defaults (MHA, rms eps 1e-6, rope theta 1e4) with the
    hidden size / depth / heads of models/llama.py:12-47 and FFN = 4 x hidden
    (:50);
  * mistral_*: MistralConfig defaults (8 KV heads, rms eps 1e-6, rope theta
    1e4, sliding window 4096; causal attention over the last 4096 keys, the
    mask HF's Mistral model builds) with models/mistral.py:16-26.
llama_6.7b, 13b, 33b, 65b and the Mistral models have head dim 128, which the
attention kernels take directly; llama_1b..5b have head dims 48, 68, 84, 98,
110, for which the layer zero-pads q, k, v to 64 / 128 around the attention
kernels (layer._attn_padded_dim).
"""
from __future__ import annotations

from types import SimpleNamespace

import torch
import torch.nn as nn

from . import kernels as K
from .lm_head import lm_head_cross_entropy
from .llama_simple import LlamaDecoderLayer, LlamaRMSNorm, llama_config
from .mistral_simple import mistral_config

# models/llama.py:12-47: hidden size, layers, attention heads
LLAMA_SHAPES = {
    "llama_1b": (1536, 24, 32),
    "llama_2b": (2176, 24, 32),
    "llama_3b": (2688, 24, 32),
    "llama_4b": (3136, 24, 32),
    "llama_5b": (3520, 24, 32),
    "llama_6.7b": (4096, 32, 32),
    "llama_13b": (5120, 40, 40),
    "llama_33b": (6656, 60, 52),
    "llama_65b": (8192, 80, 64),
}

# models/mistral.py:16-26: hidden size, layers, attention heads, FFN
MISTRAL_SHAPES = {
    "mistral_7b": (4096, 32, 32, 14336),
    "mistral_toy": (4096, 5, 32, 14336),
}

INIT_STD = 0.02  # LlamaConfig / MistralConfig initializer_range


class DecoderModel(nn.Module):
    """LlamaModel / MistralModel: token embedding, the decoder layers and the
    final RMSNorm (HF applies the norm inside the base model)."""

    def __init__(self, config, sliding_window=None, **layer_kw):
        super().__init__()
        self.config = config
        self.padding_idx = config.pad_token_id
        self.vocab_size = config.vocab_size
        self.embed_tokens = nn.Embedding(config.vocab_size, config.hidden_size, self.padding_idx)
        nn.init.normal_(self.embed_tokens.weight, 0.0, INIT_STD)
        self.layers = nn.ModuleList(
            LlamaDecoderLayer(config, i, sliding_window=sliding_window, **layer_kw)
            for i in range(config.num_hidden_layers))
        self.norm = LlamaRMSNorm(config.hidden_size, eps=config.rms_norm_eps)

    def forward(self, input_ids=None, inputs_embeds=None, position_ids=None, **kwargs):
        h = self.embed_tokens(input_ids) if inputs_embeds is None else inputs_embeds
        for layer in self.layers:
            h = layer(h, position_ids=position_ids)[0]
        return self.norm(h)


class CausalLM(nn.Module):
    """LlamaForCausalLM / MistralForCausalLM: ``model`` (DecoderModel) and
    ``lm_head``.  forward(input_ids, labels) returns an object with ``loss``
    and ``logits`` as HF's CausalLMOutputWithPast does: with labels, the
    causal-LM loss (position t predicts label t + 1, mean over labels other
    than -100) from the LM-head kernels (lm_head.lm_head_cross_entropy: the
    logits never returned, held whole only up to 1 GiB; ``logits`` is None);
    without labels, the logits."""

    def __init__(self, config, sliding_window=None, **layer_kw):
        super().__init__()
        self.config = config
        self.model = DecoderModel(config, sliding_window, **layer_kw)
        self.vocab_size = config.vocab_size
        self.lm_head = nn.Linear(config.hidden_size, config.vocab_size, bias=False)
        nn.init.normal_(self.lm_head.weight, 0.0, INIT_STD)

    def forward(self, input_ids=None, labels=None, inputs_embeds=None, position_ids=None,
                **kwargs):
        h = self.model(input_ids=input_ids, inputs_embeds=inputs_embeds,
                       position_ids=position_ids)
        w = self.lm_head.weight
        if labels is not None:
            loss = lm_head_cross_entropy(h[:, :-1], w, labels[:, 1:].contiguous())
            return SimpleNamespace(loss=loss, logits=None)
        x = h.reshape(-1, h.shape[-1])
        logits = K.gemm(x, w if w.dtype == x.dtype else w.to(x.dtype))
        return SimpleNamespace(loss=None, logits=logits.view(*h.shape[:-1], -1))


def _check_head_dim(model_name, hidden, heads):
    if hidden % heads or (hidden // heads) % 2 or hidden // heads > 128:
        raise NotImplementedError(
            f"{model_name}: head dim {hidden} / {heads}; the attention kernels take even head "
            f"dims up to 128")


def get_llama_model(model_name, vocab_size=49152, seq_length=2048, layers=None, **layer_kw):
    """models/llama.py:5-56 (``layers`` as the hub's shared model argument)."""
    if model_name not in LLAMA_SHAPES:
        raise ValueError(f"Unsupported model: {model_name}")
    hidden, n_layers, heads = LLAMA_SHAPES[model_name]
    _check_head_dim(model_name, hidden, heads)
    config = llama_config(vocab_size=vocab_size, max_position_embeddings=seq_length,
                          hidden_size=hidden, num_hidden_layers=layers or n_layers,
                          num_attention_heads=heads, intermediate_size=4 * hidden)
    layer_kw.setdefault("init_std", INIT_STD)
    model = CausalLM(config, **layer_kw)
    model.hidden_size = hidden
    model._hidden_size = hidden
    return model


def get_mistral_model(model_name, vocab_size=49152, seq_length=2048, layers=None, **layer_kw):
    """models/mistral.py:5-35."""
    if model_name not in MISTRAL_SHAPES:
        raise ValueError(f"Unsupported model: {model_name}")
    hidden, n_layers, heads, ffn = MISTRAL_SHAPES[model_name]
    _check_head_dim(model_name, hidden, heads)
    config = mistral_config(vocab_size=vocab_size, max_position_embeddings=seq_length,
                            hidden_size=hidden, num_hidden_layers=layers or n_layers,
                            num_attention_heads=heads, intermediate_size=ffn)
    layer_kw.setdefault("init_std", INIT_STD)
    model = CausalLM(config, sliding_window=config.sliding_window, **layer_kw)
    model._hidden_size = hidden
    return model


def get_model(model_name, vocab_size=49152, seq_length=2048, layers=None, **layer_kw):
    """The hub's routes for ``llama*`` and ``mistral*`` names (models/hub.py:
    55-56, 76-77)."""
    name = model_name.lower()
    if name.startswith("llama"):
        model = get_llama_model(name, vocab_size, seq_length, layers, **layer_kw)
    elif name.startswith("mistral"):
        model = get_mistral_model(name, vocab_size, seq_length, layers, **layer_kw)
    else:
        raise ValueError(f"Unsupported model: {model_name}")
    model._model_name = name
    model._num_layers = len(model.model.layers)
    return model


def get_layers(model):
    """models/hub.py:159-188 for these routes."""
    return model.model.layers
