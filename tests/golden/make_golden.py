"""Write the golden fixtures in this directory from the transformers modules
the reference composes its decoder layer from (LlamaDecoderLayer /
MistralDecoderLayer, LlamaRMSNorm, LlamaMLP, LlamaRotaryEmbedding,
apply_rotary_pos_emb, eager attention with repeat_kv -- imported by the
reference at models/llama_simple.py:7-13 and models/mistral_simple.py:5-9).

This is the installed transformers (5.x), not the reference's pinned 4.46.2
and not the reference itself: it is an implementation of the same
arithmetic, independent of this repository's oracle, run in fp64 on the CPU.
The causal / sliding-window masks come from transformers.masking_utils'
mask functions evaluated on index grids.

Each fixture (.npz, float32 for compactness, computed in fp64) holds the
layer's weights by short name, the input x, the upstream gradient dout, the
output, dx and every weight gradient.  Regenerate with
    python tests/golden/make_golden.py
"""
from __future__ import annotations

import os

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))

CASES = {
    # name: (family, hidden, heads, kv_heads, head_dim, ffn, batch, seq, theta, window, seed)
    "llama_gqa_d16": ("llama", 32, 2, 1, 16, 48, 2, 16, 1e4, 0, 10),
    "llama_mha_d64": ("llama", 64, 1, 1, 64, 64, 1, 48, 1e4, 0, 11),
    "mistral_swa_d64": ("mistral", 64, 2, 1, 64, 64, 1, 40, 1e6, 16, 12),
}


def _mask(seq: int, window: int) -> torch.Tensor:
    from transformers.masking_utils import (causal_mask_function,
                                            sliding_window_causal_mask_function)
    fn = sliding_window_causal_mask_function(window) if window else causal_mask_function
    q = torch.arange(seq)[:, None]
    k = torch.arange(seq)[None, :]
    vis = fn(0, 0, q, k)
    add = torch.zeros(seq, seq, dtype=torch.float64)
    add.masked_fill_(~vis, float("-inf"))
    return add[None, None]


def make(name, family, hidden, heads, kv, head_dim, ffn, batch, seq, theta, window, seed):
    from transformers import LlamaConfig, MistralConfig
    from transformers.models.llama.modeling_llama import LlamaDecoderLayer, LlamaRotaryEmbedding
    from transformers.models.mistral.modeling_mistral import MistralDecoderLayer

    common = dict(hidden_size=hidden, num_attention_heads=heads, num_key_value_heads=kv,
                  head_dim=head_dim,
                  intermediate_size=ffn, rms_norm_eps=1e-6, max_position_embeddings=seq,
                  rope_theta=theta, attention_dropout=0.0)
    if family == "llama":
        cfg = LlamaConfig(**common)
        cfg._attn_implementation = "eager"
        layer = LlamaDecoderLayer(cfg, 0)
    else:
        cfg = MistralConfig(sliding_window=window, **common)
        cfg._attn_implementation = "eager"
        layer = MistralDecoderLayer(cfg, 0)
    rope = LlamaRotaryEmbedding(cfg)
    g = torch.Generator().manual_seed(seed)
    names = {"q": layer.self_attn.q_proj.weight, "k": layer.self_attn.k_proj.weight,
             "v": layer.self_attn.v_proj.weight, "o": layer.self_attn.o_proj.weight,
             "gate": layer.mlp.gate_proj.weight, "up": layer.mlp.up_proj.weight,
             "down": layer.mlp.down_proj.weight, "ln1": layer.input_layernorm.weight,
             "ln2": layer.post_attention_layernorm.weight}
    with torch.no_grad():
        for k, p in names.items():
            if k.startswith("ln"):
                p.copy_(1.0 + 0.1 * torch.randn(p.shape, generator=g))
            else:
                p.copy_(0.05 * torch.randn(p.shape, generator=g))
    layer = layer.double()
    rope = rope.double()
    x = torch.randn(batch, seq, hidden, generator=g, dtype=torch.float64)
    dout = torch.randn(batch, seq, hidden, generator=g, dtype=torch.float64)
    xr = x.clone().requires_grad_(True)
    pos = torch.arange(seq)[None].expand(batch, seq)
    cos, sin = rope(xr, pos)
    out = layer(xr, attention_mask=_mask(seq, window if family == "mistral" else 0),
                position_ids=pos, position_embeddings=(cos.double(), sin.double()))
    if isinstance(out, tuple):
        out = out[0]
    out.backward(dout)
    arrays = {"x": x, "dout": dout, "out": out.detach(), "dx": xr.grad}
    for k, p in names.items():
        arrays["w_" + k] = p.detach()
        arrays["g_" + k] = p.grad
    meta = np.array([hidden, heads, kv, head_dim, ffn, batch, seq, theta, window, seed],
                    dtype=np.float64)
    np.savez_compressed(os.path.join(HERE, name + ".npz"), meta=meta,
                        **{k: v.to(torch.float32).numpy() for k, v in arrays.items()})


if __name__ == "__main__":
    torch.set_num_threads(4)
    for name, args in CASES.items():
        make(name, *args)
        print("wrote", name)
