"""Drop-in for the reference's DeepspeedMistral (models/mistral_simple.py).

Same decoder-layer machinery as ``llama_simple`` with MistralConfig's
defaults (transformers configuration_mistral: 8 KV heads, rms eps 1e-6,
sliding_window 4096, rope theta 1e4).  The layer applies causal attention
with the sliding window (key j visible from query i iff i - W < j <= i);
see the module docstring of ``llama_simple`` for what is kept and changed.
"""
from __future__ import annotations

import torch
import torch.nn as nn

from .llama_simple import Block as _LlamaBlock
from .llama_simple import LlamaRMSNorm, NoOp, llama_config


def mistral_config(**kw):
    cfg = dict(vocab_size=32000, hidden_size=4096, intermediate_size=14336,
               num_hidden_layers=32, num_attention_heads=32, num_key_value_heads=8,
               max_position_embeddings=4096 * 32, rms_norm_eps=1e-6, rope_theta=10000.0,
               sliding_window=4096)
    cfg.update(kw)
    return llama_config(**cfg)


class Block(_LlamaBlock):
    """models/mistral_simple.py:13-41."""

    def __init__(self, config, layer_idx, **layer_kw):
        layer_kw.setdefault("sliding_window", getattr(config, "sliding_window", None))
        super().__init__(config, layer_idx, torch.float32, **layer_kw)


class DeepspeedMistral(nn.Module):
    """models/mistral_simple.py:44-100."""

    def __init__(self, vocab_size=49152, seq_length=2048, hidden_size=2048,
                 intermediate_size=5632, num_hidden_layers=22, num_attention_heads=32,
                 insert_noop=False, num_key_value_heads=8, rope_theta=10000.0,
                 sliding_window=4096, **layer_kw):
        super().__init__()
        config = mistral_config(vocab_size=vocab_size, max_position_embeddings=seq_length,
                                hidden_size=hidden_size, num_hidden_layers=num_hidden_layers,
                                num_attention_heads=num_attention_heads,
                                intermediate_size=intermediate_size,
                                num_key_value_heads=num_key_value_heads,
                                rope_theta=rope_theta, sliding_window=sliding_window)
        self.config = config
        self.padding_idx = config.pad_token_id
        self.vocab_size = config.vocab_size
        self.embed_tokens = nn.Embedding(config.vocab_size, config.hidden_size, self.padding_idx)
        layers = []
        for i in range(config.num_hidden_layers):
            layers.append(Block(config, i, **layer_kw))
            if insert_noop:
                layers.append(NoOp())
        self.layers = nn.ModuleList(layers)
        self.norm = LlamaRMSNorm(config.hidden_size, eps=config.rms_norm_eps)
        self.lm_head = nn.Linear(config.hidden_size, config.vocab_size, bias=False)
        self.output_layer = nn.Sequential(self.norm, self.lm_head)

    def forward(self, x, labels=None):
        x = self.embed_tokens(x)
        for block in self.layers:
            x = block(x)
        return self.output_layer(x)

    def join_layers(self):
        return [self.embed_tokens] + list(self.layers) + [self.output_layer]


def get_model(model_name, vocab_size=49152, seq_length=2048, layers=None,
              insert_noop=False, **kw):
    """models/mistral_simple.py:103-138.  Sets ``model._hidden_size`` (the
    reference assigns a misspelled local at :136, so its model lacks the
    attribute the pipeline schedule reads)."""
    if model_name not in ("deepspeedmistral_7b", "deepspeedmistral_toy"):
        raise ValueError(f"Unsupported model: {model_name}")
    n_layers = 32 if model_name == "deepspeedmistral_7b" else 5
    if layers:
        n_layers = layers
    model = DeepspeedMistral(vocab_size=vocab_size, seq_length=seq_length, hidden_size=4096,
                             intermediate_size=14336, num_hidden_layers=n_layers,
                             num_attention_heads=32, insert_noop=insert_noop, **kw)
    model._hidden_size = 4096
    return model
