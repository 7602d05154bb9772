"""zorse_amd -- MI355X (gfx950) kernels and drop-in modules for the decoder-layer
hot path of benson-guo/zorse: RMSNorm, RoPE + GQA causal / sliding-window flash
attention, the SwiGLU MLP activation and the fused AdamW step on a layer's
flat parameter shard.

The kernels live in ``libzorse_amd.so`` (sources in ``csrc/``, C ABI in
``include/zorse_amd.h``); ``kernels`` wraps them for torch tensors,
``functional`` / ``layer`` add autograd, ``llama_simple`` / ``mistral_simple``
mirror the reference's model classes and ``optim`` its optimizer.
There is no CPU fallback: the library and a GPU are required to compute.
"""
from .layer import DecoderLayerFunction, LayerSpec  # noqa: F401

__all__ = ["LayerSpec", "DecoderLayerFunction"]
