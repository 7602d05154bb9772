"""Drop-in for the reference's torchtitan-style Llama (models/llama_v2.py).

Kept from the reference: ``ModelArgs`` (models/llama_v2.py:82-99) with its
defaults (RMSNorm eps 1e-5), the FFN width rule of ``FeedForward``
(:281-325), ``TransformerBlock(layer_id, model_args, freqs_cis)`` with
``forward(x)`` (:328-399), its submodule names (``attention.{wq,wk,wv,wo}``,
``feed_forward.{w1,w2,w3}``, ``attention_norm``, ``ffn_norm``), the
depth-scaled truncated-normal ``init_weights``, ``Transformer`` with
``join_layers`` and ``get_model`` for the named sizes (:545-631).

The arithmetic is the same fused decoder layer as ``llama_simple`` with the
interleaved-pair (complex) RoPE of ``apply_rotary_emb`` (:151-177) and causal
attention (SDPA ``is_causal=True`` at :273).  The flat parameter keeps gate
(w1) and up (w3) adjacent for the fused gate|up GEMM, so its order is wq, wk,
wv, wo, w1, w3, w2, attention_norm, ffn_norm; ``orig_named_parameters``
yields the reference's names.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch
import torch.nn as nn

from .layer import LayerSpec
from .llama_simple import FlatDecoderLayer, FlatLinear, FlatRMSNorm, LlamaRMSNorm


@dataclass
class ModelArgs:
    dim: int = 4096
    intermediate_size: Optional[int] = None
    n_layers: int = 32
    n_heads: int = 32
    n_kv_heads: Optional[int] = None
    vocab_size: int = -1
    multiple_of: int = 256
    ffn_dim_multiplier: Optional[float] = None
    norm_eps: float = 1e-5
    rope_theta: float = 10000
    max_seq_len: int = 2048
    depth_init: bool = True
    norm_type: str = "rmsnorm"


def ffn_hidden_dim(args: ModelArgs) -> int:
    """FeedForward's hidden width (models/llama_v2.py:300-309): 2/3 of 4 dim,
    times the optional multiplier, rounded up to multiple_of; an explicit
    intermediate_size wins."""
    hidden = int(2 * (4 * args.dim) / 3)
    if args.ffn_dim_multiplier is not None:
        hidden = int(args.ffn_dim_multiplier * hidden)
    hidden = args.multiple_of * ((hidden + args.multiple_of - 1) // args.multiple_of)
    if args.intermediate_size is not None:
        hidden = args.intermediate_size
    return hidden


def spec_from_args(args: ModelArgs) -> LayerSpec:
    kv = args.n_heads if args.n_kv_heads is None else args.n_kv_heads
    if args.norm_type not in ("rmsnorm", "fused_rmsnorm"):
        raise NotImplementedError(f"norm_type {args.norm_type!r}: only RMSNorm is provided")
    return LayerSpec(hidden=args.dim, heads=args.n_heads, kv_heads=kv,
                     head_dim=args.dim // args.n_heads, ffn=ffn_hidden_dim(args),
                     eps=args.norm_eps, rope_theta=float(args.rope_theta), causal=True,
                     window=0, interleaved_rope=True)


class Attention(nn.Module):
    def __init__(self, owner, spec: LayerSpec):
        super().__init__()
        self.n_heads, self.n_kv_heads = spec.heads, spec.kv_heads
        self.n_rep = spec.heads // spec.kv_heads
        self.head_dim = spec.head_dim
        self.wq = FlatLinear(owner, "q", spec.hidden, spec.q_dim)
        self.wk = FlatLinear(owner, "k", spec.hidden, spec.kv_dim)
        self.wv = FlatLinear(owner, "v", spec.hidden, spec.kv_dim)
        self.wo = FlatLinear(owner, "o", spec.q_dim, spec.hidden)


class FeedForward(nn.Module):
    def __init__(self, owner, spec: LayerSpec):
        super().__init__()
        self.w1 = FlatLinear(owner, "gate", spec.hidden, spec.ffn)
        self.w2 = FlatLinear(owner, "down", spec.ffn, spec.hidden)
        self.w3 = FlatLinear(owner, "up", spec.hidden, spec.ffn)


class TransformerBlock(FlatDecoderLayer):
    """models/llama_v2.py:328-399: h = x + attention(attention_norm(x));
    out = h + feed_forward(ffn_norm(h)).  ``freqs_cis`` is accepted for
    signature compatibility; the rotation tables are built from
    ``model_args.rope_theta`` on the device."""

    ORIG_NAMES = {"q": "attention.wq.weight", "k": "attention.wk.weight",
                  "v": "attention.wv.weight", "o": "attention.wo.weight",
                  "gate": "feed_forward.w1.weight", "up": "feed_forward.w3.weight",
                  "down": "feed_forward.w2.weight", "ln1": "attention_norm.weight",
                  "ln2": "ffn_norm.weight"}

    def __init__(self, layer_id: int, model_args: ModelArgs, freqs_cis=None, *, device=None,
                 param_dtype=torch.float32, generator: torch.Generator | None = None):
        spec = spec_from_args(model_args)
        super().__init__(spec, device=device, param_dtype=param_dtype)
        self.n_heads, self.dim = model_args.n_heads, model_args.dim
        self.layer_id, self.num_layers = layer_id, model_args.n_layers
        self.attention = Attention(self, spec)
        self.feed_forward = FeedForward(self, spec)
        self.attention_norm = FlatRMSNorm(self, "ln1", spec.hidden, spec.eps)
        self.ffn_norm = FlatRMSNorm(self, "ln2", spec.hidden, spec.eps)
        if model_args.depth_init:
            self.weight_init_std = 0.02 / (2 * (self.layer_id + 1)) ** 0.5
        else:
            self.weight_init_std = 0.02 / (2 * self.num_layers) ** 0.5
        self.init_weights(generator)

    @torch.no_grad()
    def init_weights(self, generator: torch.Generator | None = None):
        """Truncated normal (torch's default cut at +-2): wq, wk, wv and w1 with
        std 0.02, wo, w2 and w3 with the depth-scaled std; norms ones
        (models/llama_v2.py:231-234, 322-325, 395-399)."""
        for name, shp in self.spec.shapes().items():
            view = self.param_view(name)
            if name.startswith("ln"):
                view.fill_(1.0)
                continue
            std = 0.02 if name in ("q", "k", "v", "gate") else self.weight_init_std
            w = torch.empty(shp)
            if w.device.type != "meta":
                torch.nn.init.trunc_normal_(w, mean=0.0, std=std, generator=generator)
            view.copy_(w)
        self._lowp_cache = None

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self._run(x)


class Transformer(nn.Module):
    """models/llama_v2.py:402-543 (embedding, blocks, norm, output)."""

    def __init__(self, model_args: ModelArgs, **block_kw):
        super().__init__()
        self.model_args = model_args
        self.vocab_size = model_args.vocab_size
        self.n_layers = model_args.n_layers
        self.tok_embeddings = nn.Embedding(model_args.vocab_size, model_args.dim)
        self.layers = nn.ModuleList([TransformerBlock(i, model_args, None, **block_kw)
                                     for i in range(model_args.n_layers)])
        self.norm = LlamaRMSNorm(model_args.dim, eps=model_args.norm_eps)
        self.output = nn.Linear(model_args.dim, model_args.vocab_size, bias=False)
        self.output_layer = nn.Sequential(self.norm, self.output)
        with torch.no_grad():
            nn.init.normal_(self.tok_embeddings.weight)
            std = model_args.dim ** -0.5
            nn.init.trunc_normal_(self.output.weight, mean=0.0, std=std, a=-3 * std, b=3 * std)

    @classmethod
    def from_model_args(cls, model_args: ModelArgs) -> "Transformer":
        return cls(model_args)

    def forward(self, tokens: torch.Tensor, labels=None):
        h = self.tok_embeddings(tokens) if self.tok_embeddings else tokens
        for layer in self.layers:
            h = layer(h)
        if self.output_layer is not None:
            h = self.output_layer(h)
        return h

    def join_layers(self):
        out = []
        if self.tok_embeddings:
            out.append(self.tok_embeddings)
        out.extend(self.layers)
        if self.output_layer:
            out.append(self.output_layer)
        return out


MODEL_SHAPES = {
    # models/llama_v2.py:566-625: dim, intermediate_size, n_heads, n_layers
    "deepspeedllamav2_tiny": (2048, 5632, 32, 22),
    "deepspeedllamav2_3b": (3200, 8640, 32, 26),
    "deepspeedllamav2_7b": (4096, 11008, 32, 32),
    "deepspeedllamav2_13b": (5120, 13824, 40, 40),
    "deepspeedllamav2_33b": (6656, 17920, 56, 60),
    "deepspeedllamav2_65b": (8192, 22016, 64, 80),
}


def get_model(model_name: str, vocab_size: int = 49152, seq_length: int = 2048,
              layers: Optional[int] = None, insert_noop: bool = False, **block_kw) -> Transformer:
    if model_name not in MODEL_SHAPES:
        raise ValueError(f"Unsupported model: {model_name}")
    dim, inter, heads, n_layers = MODEL_SHAPES[model_name]
    args = ModelArgs(dim=dim, intermediate_size=inter, n_heads=heads,
                     n_layers=n_layers if layers is None else layers, vocab_size=vocab_size,
                     max_seq_len=seq_length)
    model = Transformer(args, **block_kw)
    model._hidden_size = dim
    return model
