"""One-GPU pipeline-stage runner: the per-layer call order of the reference's
stage executor with the optimizer stepped inside the backward.

Reference behaviour reproduced (single GPU, no communication):
  * forward: each layer called in order on the micro-batch
    (zorse_utils/pipeline_schedule_v2.py:138-155, ``_forward_layer``);
  * backward: ``out.backward(grad)``, and as soon as a layer's flat gradient
    is complete its optimizer steps on a dedicated optimizer stream that first
    waits for the compute stream (utils/patch.py:76-154, the
    ``--optimizer_in_backwards`` path built at zorse_utils/pipeline.py:
    150-181), then the gradient is released;
  * with ``transposed_weights`` (the default) each bf16 / fp16 layer's step
    also writes transposed copies of its projection weights, which the next
    backward's input-gradient GEMMs read along their reduction;
  * ``recompute=True`` re-runs each layer's forward inside the backward, as
    ``_backward_layer`` does (zorse_utils/pipeline_schedule_v2.py:157-200);
    with ``cache_attention`` (the default) the first forward keeps each
    layer's attention output and LSE and the re-run skips the attention
    forward kernel.

All streams are created at the default priority.
"""
from __future__ import annotations

from typing import Sequence

import torch
import torch.nn as nn

from . import layer as _layer_mod
from .layer import AttentionCache
from .optim import FusedAdamW


def _call(layer: nn.Module, x: torch.Tensor) -> torch.Tensor:
    """Blocks return a tensor, bare decoder layers a tuple (hidden, ...)."""
    y = layer(x)
    return y[0] if isinstance(y, tuple) else y


class StageRunner:
    def __init__(self, layers: Sequence[nn.Module], lr=1e-4, betas=(0.9, 0.95), eps=1e-8,
                 weight_decay=0.1, optimizer_in_backwards=True, recompute=False,
                 cache_attention=True, optimizer_overlap="attention", transposed_weights=True):
        if optimizer_overlap not in ("attention", "immediate"):
            raise ValueError(f"optimizer_overlap {optimizer_overlap!r}: 'attention' or 'immediate'")
        self.layers = list(layers)
        self.optimizer_in_backwards = optimizer_in_backwards
        # "immediate": a layer's step is enqueued as soon as its gradient is
        # complete; "attention": it is held until the next layer's attention
        # backward starts, so that it overlaps that kernel instead of GEMMs
        self.optimizer_overlap = optimizer_overlap
        self._pending = []
        self.recompute = recompute
        # one attention cache per fused decoder layer (recompute mode only)
        self.attn_caches = []
        if recompute and cache_attention:
            for layer in self.layers:
                for m in layer.modules():
                    if hasattr(m, "attn_cache") and hasattr(m, "flat_param"):
                        m.attn_cache = AttentionCache()
                        self.attn_caches.append(m.attn_cache)
        self.optimizers = []
        self._hooks = []
        dev = next(self.layers[0].parameters()).device
        self.optimizer_stream = torch.cuda.Stream(device=dev) if dev.type == "cuda" else None
        for layer in self.layers:
            params = [p for p in layer.parameters() if p.requires_grad]
            opt = FusedAdamW(params, lr=lr, betas=betas, eps=eps, weight_decay=weight_decay)
            self.optimizers.append(opt)
            if transposed_weights:
                # the step also writes W^T of the projections for the next
                # backward's input-gradient GEMMs (bf16 / fp16 parameters)
                for m in layer.modules():
                    if hasattr(m, "enable_transposed_weights") and \
                            m.flat_param.dtype in (torch.bfloat16, torch.float16):
                        m.enable_transposed_weights(opt)
            if optimizer_in_backwards:
                for p in params:
                    self._hooks.append(p.register_post_accumulate_grad_hook(
                        self._make_hook(opt)))

    def _make_hook(self, opt: FusedAdamW):
        def hook(p: torch.Tensor):
            if self.optimizer_overlap == "attention":
                self._pending.append((opt, p))
            else:
                self._step_on_side_stream(opt, p)
        return hook

    def _launch_pending(self):
        pending, self._pending = self._pending, []
        for opt, p in pending:
            self._step_on_side_stream(opt, p)

    def _step_on_side_stream(self, opt: FusedAdamW, p: torch.Tensor):
        cur = torch.cuda.current_stream(p.device)
        side = self.optimizer_stream
        side.wait_stream(cur)
        with torch.cuda.stream(side):
            grad = p.grad
            opt.step()
            grad.record_stream(side)
            p.grad = None

    def wait_optimizer(self):
        """Make the compute stream wait for every optimizer step enqueued so
        far (call before the next forward touches the parameters)."""
        if self.optimizer_stream is not None:
            torch.cuda.current_stream(self.optimizer_stream.device).wait_stream(
                self.optimizer_stream)

    def forward(self, x: torch.Tensor):
        self.wait_optimizer()
        if self.recompute:
            self._inputs = []
            with torch.no_grad():
                for layer in self.layers:
                    self._inputs.append(x)
                    x = _call(layer, x)
            return x
        for layer in self.layers:
            x = _call(layer, x)
        return x

    def backward(self, out: torch.Tensor, grad: torch.Tensor):
        hook = self._launch_pending
        _layer_mod.BEFORE_ATTENTION_BACKWARD.append(hook)
        try:
            if not self.recompute:
                out.backward(grad)
            else:
                g = grad
                for layer, x in zip(reversed(self.layers), reversed(self._inputs)):
                    xr = x.detach().requires_grad_(True)
                    y = _call(layer, xr)
                    y.backward(g)
                    g = xr.grad
                self._inputs = []
                for c in self.attn_caches:  # entries of forwards never recomputed
                    c.clear()
        finally:
            _layer_mod.BEFORE_ATTENTION_BACKWARD.remove(hook)
        self._launch_pending()  # the last layer's step: nothing left to overlap
        if not self.optimizer_in_backwards:
            for opt in self.optimizers:
                opt.step()
                opt.zero_grad(set_to_none=True)

    def step(self, x: torch.Tensor, grad: torch.Tensor):
        """One stage step: forward, backward, per-layer AdamW."""
        out = self.forward(x)
        if self.recompute:
            out = out.detach()
        self.backward(out, grad)
        return out
