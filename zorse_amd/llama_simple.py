"""Drop-in for the reference's DeepspeedLlama decoder stack
(models/llama_simple.py), running on the gfx950 kernels.

Kept from the reference (models/llama_simple.py:391-652): the class names,
constructor signatures, forward signatures and return conventions, the
submodule and attribute names read by the model hub accessors
(``block.self_attn.{q,k,v,o}_proj.weight``, ``block.mlp.{gate,up,down}_proj
.weight``, ``block.{input,post_attention}_layernorm.weight``), parameter counts
(data/model_stats.json:92,104) and the config defaults of LlamaConfig.

Changed for the GPU: each decoder layer owns ONE flat parameter (1-D, in the
reference's registration order q, k, v, o, gate, up, down, ln1, ln2 -- the
layout FSDP gives the same module with use_orig_params=False), and the named
weights are views of it.  The whole layer is one autograd node
(``layer.DecoderLayerFunction``).  Attention is always the causal flash kernel
(the reference picks FA2 / SDPA, both causal, at :396-416), with an optional
sliding window for Mistral.
"""
from __future__ import annotations

import math
import weakref
from types import SimpleNamespace

import torch
import torch.nn as nn

from . import functional as Fn
from .layer import DecoderLayerFunction, LayerSpec


def llama_config(**kw) -> SimpleNamespace:
    """Config object with LlamaConfig's defaults for the fields the layer
    reads (the reference builds LlamaConfig at models/llama_simple.py:540-547).
    Any object with these attributes (e.g. a transformers LlamaConfig) works."""
    cfg = dict(vocab_size=32000, hidden_size=4096, intermediate_size=11008,
               num_hidden_layers=32, num_attention_heads=32, num_key_value_heads=None,
               head_dim=None, max_position_embeddings=2048, rms_norm_eps=1e-6,
               rope_theta=10000.0, sliding_window=None, pad_token_id=None)
    cfg.update(kw)
    if cfg["num_key_value_heads"] is None:
        cfg["num_key_value_heads"] = cfg["num_attention_heads"]
    if cfg["head_dim"] is None:
        cfg["head_dim"] = cfg["hidden_size"] // cfg["num_attention_heads"]
    return SimpleNamespace(**cfg)


def spec_from_config(config, sliding_window=None) -> LayerSpec:
    heads = config.num_attention_heads
    kv = getattr(config, "num_key_value_heads", None) or heads
    hd = getattr(config, "head_dim", None) or config.hidden_size // heads
    theta = getattr(config, "rope_theta", None)
    if theta is None:  # transformers >= 5 keeps it in rope_parameters
        theta = (getattr(config, "rope_parameters", None) or {}).get("rope_theta", 10000.0)
    window = sliding_window if sliding_window is not None else 0
    return LayerSpec(hidden=config.hidden_size, heads=heads, kv_heads=kv, head_dim=hd,
                     ffn=config.intermediate_size,
                     eps=getattr(config, "rms_norm_eps", 1e-6), rope_theta=float(theta),
                     causal=True, window=int(window or 0))


# ------------------------------------------------------- weight-view modules --

class _FlatSlot(nn.Module):
    """Submodule whose ``weight`` is a live view of its layer's flat
    parameter (no Parameter of its own)."""

    def __init__(self, owner: "LlamaDecoderLayer", name: str):
        super().__init__()
        object.__setattr__(self, "_owner", weakref.ref(owner))
        object.__setattr__(self, "_slot", name)

    @property
    def weight(self) -> torch.Tensor:
        return self._owner().param_view(self._slot)


class FlatLinear(_FlatSlot):
    """nn.Linear(in_features, out_features, bias=False) stand-in."""

    def __init__(self, owner, name, in_features, out_features):
        super().__init__(owner, name)
        self.in_features, self.out_features = in_features, out_features

    def forward(self, x):
        return torch.nn.functional.linear(x, self.weight.to(x.dtype))

    def extra_repr(self):
        return f"in_features={self.in_features}, out_features={self.out_features}, bias=False"


class FlatRMSNorm(_FlatSlot):
    """LlamaRMSNorm stand-in whose weight lives in the layer's flat param."""

    def __init__(self, owner, name, hidden_size, eps):
        super().__init__(owner, name)
        self.variance_epsilon = eps
        self.hidden_size = hidden_size

    def forward(self, x):
        return Fn.rms_norm(x, self.weight, self.variance_epsilon)


class LlamaRMSNorm(nn.Module):
    """Standalone RMSNorm with its own weight (HF LlamaRMSNorm, used for the
    final norm at models/llama_simple.py:557)."""

    def __init__(self, hidden_size, eps=1e-6):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(hidden_size))
        self.variance_epsilon = eps

    def forward(self, x):
        return Fn.rms_norm(x, self.weight, self.variance_epsilon)


class LlamaAttention(nn.Module):
    """Holds the projection views and head geometry (models/llama_simple.py:
    176-221); the arithmetic runs inside the fused layer node."""

    def __init__(self, owner, spec: LayerSpec, layer_idx=None):
        super().__init__()
        self.layer_idx = layer_idx
        self.hidden_size = spec.hidden
        self.num_heads = spec.heads
        self.num_key_value_heads = spec.kv_heads
        self.num_key_value_groups = spec.heads // spec.kv_heads
        self.head_dim = spec.head_dim
        self.rope_theta = spec.rope_theta
        self.is_causal = True
        self.sliding_window = spec.window or None
        self.q_proj = FlatLinear(owner, "q", spec.hidden, spec.q_dim)
        self.k_proj = FlatLinear(owner, "k", spec.hidden, spec.kv_dim)
        self.v_proj = FlatLinear(owner, "v", spec.hidden, spec.kv_dim)
        self.o_proj = FlatLinear(owner, "o", spec.q_dim, spec.hidden)


class LlamaMLP(nn.Module):
    def __init__(self, owner, spec: LayerSpec):
        super().__init__()
        self.hidden_size, self.intermediate_size = spec.hidden, spec.ffn
        self.gate_proj = FlatLinear(owner, "gate", spec.hidden, spec.ffn)
        self.up_proj = FlatLinear(owner, "up", spec.hidden, spec.ffn)
        self.down_proj = FlatLinear(owner, "down", spec.ffn, spec.hidden)


# -------------------------------------------------------------- the layer --

class FlatDecoderLayer(nn.Module):
    """A decoder layer whose parameters live in ONE flat buffer laid out as
    LayerSpec.offsets() (q, k, v, o, gate, up, down, ln1, ln2); the named
    weights of the reference modules are views of it.  Subclasses create the
    reference's submodule names."""

    def __init__(self, spec: LayerSpec, *, device=None, param_dtype=torch.float32,
                 init_std: float | None = None, generator: torch.Generator | None = None):
        super().__init__()
        self.spec = spec
        self._offsets = spec.offsets()
        self.flat_param = nn.Parameter(torch.empty(spec.numel, dtype=param_dtype, device=device))
        self._lowp_cache = None
        self._init_std, self._init_gen = init_std, generator
        # AttentionCache shared by the two forwards of a recomputed micro-batch
        # (set by the stage runner; None = always compute attention)
        self.attn_cache = None

    # -- parameters -----------------------------------------------------------
    def param_view(self, name: str) -> torch.Tensor:
        a, b = self._offsets[name]
        return self.flat_param[a:b].view(self.spec.shapes()[name])

    ORIG_NAMES: dict = {}

    def orig_named_parameters(self):
        """(reference parameter name, view) pairs in registration order."""
        for k in self._offsets:
            yield self.ORIG_NAMES.get(k, k), self.param_view(k)

    @torch.no_grad()
    def reset_parameters(self, std: float | None = None,
                         generator: torch.Generator | None = None):
        """Linear weights: nn.Linear's default U(-1/sqrt(in), 1/sqrt(in)) or,
        with ``std``, N(0, std); norm weights: ones.  Drawn on the CPU so a
        seeded generator gives the same values on every device."""
        for name, shp in self.spec.shapes().items():
            view = self.param_view(name)
            if name.startswith("ln"):
                view.fill_(1.0)
                continue
            if std is None:
                bound = 1.0 / math.sqrt(shp[1])
                w = torch.empty(shp).uniform_(-bound, bound, generator=generator)
            else:
                w = torch.randn(shp, generator=generator) * std
            view.copy_(w)
        self._lowp_cache = None

    def load_named(self, tensors: dict[str, torch.Tensor]) -> None:
        """Copy weights given by short name (q, k, v, o, gate, up, down, ln1, ln2)."""
        with torch.no_grad():
            for k, t in tensors.items():
                self.param_view(k).copy_(t)
        self._lowp_cache = None

    def _compute_weights(self, dtype: torch.dtype):
        p = self.flat_param
        if p.dtype == dtype:
            return None
        key = (p.data_ptr(), p._version, dtype)
        if self._lowp_cache is not None and self._lowp_cache[0] == key:
            return self._lowp_cache[1]
        w = p.detach().to(dtype)
        self._lowp_cache = (key, w)
        return w

    def _run(self, x: torch.Tensor, positions: torch.Tensor | None = None) -> torch.Tensor:
        """The fused layer on x [B, S, h]; under autocast an fp32 input runs in
        the autocast dtype (the profiler protocol).  ``positions``: int64 [S]
        RoPE positions on x's device, or None for 0 .. S-1."""
        cdt = x.dtype
        if cdt == torch.float32 and torch.is_autocast_enabled("cuda"):
            cdt = torch.get_autocast_dtype("cuda")
            x = x.to(cdt)
        return DecoderLayerFunction.apply(x, self.flat_param, self.spec,
                                          self._compute_weights(cdt), self.attn_cache, positions)

    # position_ids tensors known to hold arange(S) (the Block's cached ids):
    # recognised by identity, so the common call costs no check
    _arange_ids = None

    def _positions(self, position_ids, S, device):
        """None when position_ids is None or 0 .. S-1, else the int64 [S]
        positions on ``device`` (every batch row must hold the same ids)."""
        if position_ids is None or position_ids is self._arange_ids:
            return None
        ids = position_ids.reshape(-1, position_ids.shape[-1])
        if ids.shape[-1] != S:
            raise ValueError(f"position_ids has {ids.shape[-1]} positions for {S} tokens")
        if ids.dtype not in (torch.int32, torch.int64):
            raise ValueError("position_ids must be an integer tensor")
        if ids.shape[0] > 1 and not bool((ids == ids[:1]).all()):
            raise NotImplementedError("position_ids that differ between batch rows are not "
                                      "supported")
        pos = ids[0].to(device=device, dtype=torch.int64).contiguous()
        if bool((pos < 0).any()):
            raise ValueError("position_ids must be non-negative")
        if bool(torch.equal(pos, torch.arange(S, device=device))):
            return None
        return pos


class LlamaDecoderLayer(FlatDecoderLayer):
    """LlamaDecoderLayer (models/llama_simple.py:391-487) over one flat
    parameter.  ``dtype`` is accepted for signature compatibility (the
    reference uses it only to pick the attention class); parameters are
    created in ``param_dtype``: fp32 (the nn.Linear default) for the
    profiler's autocast protocol, or bf16 / fp16 for the pipeline's mixed
    precision, where the optimizer keeps the fp32 master."""

    ORIG_NAMES = {"q": "self_attn.q_proj.weight", "k": "self_attn.k_proj.weight",
                  "v": "self_attn.v_proj.weight", "o": "self_attn.o_proj.weight",
                  "gate": "mlp.gate_proj.weight", "up": "mlp.up_proj.weight",
                  "down": "mlp.down_proj.weight", "ln1": "input_layernorm.weight",
                  "ln2": "post_attention_layernorm.weight"}

    def __init__(self, config, layer_idx: int, dtype=torch.float32, *,
                 sliding_window=None, device=None, param_dtype=torch.float32,
                 init_std: float | None = None, generator: torch.Generator | None = None):
        super().__init__(spec_from_config(config, sliding_window), device=device,
                         param_dtype=param_dtype)
        self.hidden_size = self.spec.hidden
        self.layer_idx = layer_idx
        self.self_attn = LlamaAttention(self, self.spec, layer_idx)
        self.mlp = LlamaMLP(self, self.spec)
        self.input_layernorm = FlatRMSNorm(self, "ln1", self.spec.hidden, self.spec.eps)
        self.post_attention_layernorm = FlatRMSNorm(self, "ln2", self.spec.hidden,
                                                    self.spec.eps)
        self.reset_parameters(init_std, generator)

    def forward(self, hidden_states, attention_mask=None, position_ids=None,
                past_key_value=None, output_attentions=False, use_cache=False,
                cache_position=None, **kwargs):
        if attention_mask is not None:
            raise NotImplementedError("explicit attention masks are not supported; the "
                                      "layer applies the causal / sliding-window mask itself")
        if past_key_value is not None or use_cache or output_attentions:
            raise NotImplementedError("KV caches and attention weights are not produced")
        pos = self._positions(position_ids, hidden_states.shape[1], hidden_states.device)
        return (self._run(hidden_states, pos),)


class Block(nn.Module):
    """models/llama_simple.py:490-518: caches position_ids = arange(S)[None]
    and returns the decoder layer's hidden states."""

    def __init__(self, config, layer_idx, dtype=torch.float32, **layer_kw):
        super().__init__()
        self.block = LlamaDecoderLayer(config, layer_idx, dtype, **layer_kw)
        self.register_buffer("cached_position_ids", None)

    def forward(self, x):
        seq_length = x.size(1)
        if self.cached_position_ids is None or self.cached_position_ids.size(1) != seq_length:
            self.cached_position_ids = torch.arange(0, seq_length, device=x.device,
                                                    dtype=torch.long).unsqueeze(0)
            # the layer takes these ids as 0 .. S-1 without checking them
            self.block._arange_ids = self.cached_position_ids
        return self.block(x, attention_mask=None, position_ids=self.cached_position_ids)[0]


class NoOp(nn.Module):
    """models/common.py:6-15 -- identity placeholder layer with one zero
    dummy parameter."""

    def __init__(self):
        super().__init__()
        self.dummy_param = nn.Parameter(torch.zeros(1))

    def forward(self, x):
        return x


class DeepspeedLlama(nn.Module):
    """models/llama_simple.py:524-585."""

    def __init__(self, vocab_size=49152, seq_length=2048, hidden_size=2048,
                 intermediate_size=5632, num_hidden_layers=22, num_attention_heads=32,
                 insert_noop=False, dtype=torch.float32, num_key_value_heads=None,
                 rope_theta=10000.0, rms_norm_eps=1e-6, sliding_window=None, **layer_kw):
        super().__init__()
        config = llama_config(vocab_size=vocab_size, max_position_embeddings=seq_length,
                              hidden_size=hidden_size, num_attention_heads=num_attention_heads,
                              num_hidden_layers=num_hidden_layers,
                              intermediate_size=intermediate_size,
                              num_key_value_heads=num_key_value_heads, rope_theta=rope_theta,
                              rms_norm_eps=rms_norm_eps)
        self.config = config
        self.padding_idx = config.pad_token_id
        self.vocab_size = config.vocab_size
        self.embed_tokens = nn.Embedding(config.vocab_size, config.hidden_size, self.padding_idx)
        layers = []
        for i in range(config.num_hidden_layers):
            layers.append(Block(config, i, dtype, sliding_window=sliding_window, **layer_kw))
            if insert_noop:
                layers.append(NoOp())
        self.layers = nn.ModuleList(layers)
        self.norm = LlamaRMSNorm(config.hidden_size, eps=config.rms_norm_eps)
        self.lm_head = nn.Linear(config.hidden_size, config.vocab_size, bias=False)
        self.output_layer = nn.Sequential(self.norm, self.lm_head)

    def forward(self, x, labels=None):
        if self.embed_tokens:
            x = self.embed_tokens(x)
        for block in self.layers:
            x = block(x)
        if self.output_layer:
            x = self.output_layer(x)
        return x

    def join_layers(self):
        out = []
        if self.embed_tokens:
            out.append(self.embed_tokens)
        out.extend(self.layers)
        if self.output_layer:
            out.append(self.output_layer)
        return out


MODEL_SHAPES = {
    # models/llama_simple.py:598-636
    "deepspeedllama_tiny": (2048, 5632, 22, 32),
    "deepspeedllama_3b": (3200, 8640, 26, 32),
    "deepspeedllama_7b": (4096, 11008, 32, 32),
    "deepspeedllama_13b": (5120, 13824, 40, 40),
    "deepspeedllama_33b": (6656, 17920, 60, 52),
    "deepspeedllama_65b": (8192, 22016, 80, 64),
}


def get_model(model_name, vocab_size=49152, seq_length=2048, layers=None,
              insert_noop=False, dtype=torch.float32, **kw):
    """models/llama_simple.py:588-652."""
    if model_name not in MODEL_SHAPES:
        raise ValueError(f"Unsupported model: {model_name}")
    hidden, inter, n_layers, heads = MODEL_SHAPES[model_name]
    if layers:
        n_layers = layers
    model = DeepspeedLlama(vocab_size=vocab_size, seq_length=seq_length, hidden_size=hidden,
                           intermediate_size=inter, num_hidden_layers=n_layers,
                           num_attention_heads=heads, insert_noop=insert_noop, dtype=dtype, **kw)
    model._hidden_size = hidden
    return model
