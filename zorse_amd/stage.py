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
  * ``offload_inputs=True`` (recompute mode) keeps each layer's input in
    pinned host memory between the two forwards: D2H during the forward and
    H2D one layer ahead during the backward, on a copy stream (the
    reference's mem_copy_stream and CPU activation buffers,
    zorse_utils/pipeline_schedule_v2.py:119-136,
    zorse_utils/pipeline_schedule_zero2.py:246-270, 391-470);
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

from . import kernels as K
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
                 cache_attention=True, optimizer_overlap="attention", offload_inputs=False):
        if optimizer_overlap not in ("attention", "immediate"):
            raise ValueError(f"optimizer_overlap {optimizer_overlap!r}: 'attention' or 'immediate'")
        if offload_inputs and not recompute:
            raise ValueError("offload_inputs keeps the layer inputs on the host between the two "
                             "forwards of recompute mode: it needs recompute=True")
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
        # the attention caches of each layer (for the micro-batch tokens of offload mode)
        self._layer_caches = [[m.attn_cache for m in layer.modules()
                               if getattr(m, "attn_cache", None) is not None]
                              for layer in self.layers]
        self.optimizers = []
        self._hooks = []
        dev = next(self.layers[0].parameters()).device
        self.optimizer_stream = torch.cuda.Stream(device=dev) if dev.type == "cuda" else None
        # offload mode: each layer's input goes to pinned host memory during the
        # forward and comes back, one layer ahead, during the backward -- both
        # copies on their own stream (the reference's mem_copy_stream)
        self.offload_inputs = offload_inputs
        self.copy_stream = torch.cuda.Stream(device=dev) if offload_inputs else None
        self._host = []   # pinned host buffer per layer input, reused across steps
        # both copies as zk_copy_to_host / zk_copy_from_host kernels from this
        # many workgroups (0: hipMemcpyAsync, whose device-to-host kernel holds
        # every CU for the transfer and whose host-to-device call can block the
        # host until the copy stream's wait on the compute stream resolves)
        self.copy_blocks = 2
        self._step_no = 0
        for layer in self.layers:
            params = [p for p in layer.parameters() if p.requires_grad]
            opt = FusedAdamW(params, lr=lr, betas=betas, eps=eps, weight_decay=weight_decay)
            self.optimizers.append(opt)
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
            # this parameter only: a layer with several parameters gets one
            # hook call per parameter, and each must be stepped exactly once
            opt.step_param(p)
            grad.record_stream(side)
            p.grad = None

    def wait_optimizer(self):
        """Make the compute stream wait for every optimizer step enqueued so
        far (call before the next forward touches the parameters)."""
        if self.optimizer_stream is not None:
            torch.cuda.current_stream(self.optimizer_stream.device).wait_stream(
                self.optimizer_stream)

    def _set_tokens(self, li):
        for c in self._layer_caches[li]:
            c.token = (self._step_no, li)

    def _store(self, li: int, x: torch.Tensor):
        """D2H copy of layer li's input into its pinned host buffer."""
        while len(self._host) <= li:
            self._host.append(None)
        host = self._host[li]
        if host is None or host.shape != x.shape or host.dtype != x.dtype:
            host = torch.empty(x.shape, dtype=x.dtype, pin_memory=True)
            self._host[li] = host
        self.copy_stream.wait_stream(torch.cuda.current_stream(x.device))
        with torch.cuda.stream(self.copy_stream):
            if self.copy_blocks:
                K.copy_to_host(host, x.contiguous(), blocks=self.copy_blocks)
            else:
                host.copy_(x, non_blocking=True)
        x.record_stream(self.copy_stream)  # keep x's memory until the copy is done
        return host, x.device

    def _load(self, i: int, after_compute: bool = False):
        """H2D copy of layer i's input (after its D2H: same stream).  With
        ``after_compute`` the copy also waits for the compute enqueued so far,
        so a prefetch starts with the layer it overlaps, however far ahead
        the host runs, and at most two inputs are back on the device."""
        host, dev = self._inputs[i]
        if after_compute:
            self.copy_stream.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(self.copy_stream):
            # allocated on the copy stream, so the allocator orders its reuse
            # after this copy; record_stream covers the compute stream's use
            buf = torch.empty(host.shape, dtype=host.dtype, device=dev)
            if self.copy_blocks:
                K.copy_from_host(buf, host, blocks=self.copy_blocks)
            else:
                buf.copy_(host, non_blocking=True)
        buf.record_stream(torch.cuda.current_stream(dev))
        done = torch.cuda.Event()
        done.record(self.copy_stream)
        return buf, done

    def forward(self, x: torch.Tensor):
        self.wait_optimizer()
        if self.recompute:
            self._inputs = []
            self._step_no += 1
            with torch.no_grad():
                last = len(self.layers) - 1
                for li, layer in enumerate(self.layers):
                    if self.offload_inputs:
                        self._set_tokens(li)
                    if self.offload_inputs and li < last:
                        self._inputs.append(self._store(li, x))
                    else:  # the last layer's input is the backward's first: it stays
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
            elif self.offload_inputs:
                g = grad
                n = len(self.layers)
                nxt = (self._inputs[n - 1], None)
                for li in range(n - 1, -1, -1):
                    buf, done = nxt
                    if li > 0:  # prefetch during this layer's backward
                        nxt = self._load(li - 1, after_compute=True)
                    if done is not None:
                        torch.cuda.current_stream(buf.device).wait_event(done)
                    self._set_tokens(li)
                    xr = buf.detach().requires_grad_(True)
                    y = _call(self.layers[li], xr)
                    y.backward(g)
                    g = xr.grad
                self._inputs = []
                for c in self.attn_caches:
                    c.clear()
                    c.token = None
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
