"""Output layer + cross-entropy of the last pipeline stage, chunked over the
vocabulary.

Replaces ``output_layer = Sequential(norm, lm_head)`` (models/llama_simple.py:
559-561) followed by ``F.cross_entropy(out.flatten(0, 1), target.flatten(0,
1))`` (zorse_utils/pipeline_schedule_v2.py:181-184).  The reference
materialises [tokens, vocab] logits (and their fp32 softmax under autocast);
here the vocabulary is processed in chunks of ``chunk`` columns:
  forward   per chunk: logits_c = x W_c^T (zk_gemm), then zk_ce_fwd_chunk
            folds it into a running log-sum-exp and picks the label logit;
            loss = mean over non-ignored tokens of (lse - label logit);
  backward  per chunk: logits_c is recomputed, zk_ce_bwd_chunk turns it in
            place into g (softmax - onehot) / n_valid, then dx += dlogits_c
            W_c (fp32 accumulator) and dW_c = dlogits_c^T x, both products on
            zk_gemm with the operands as stored.
Only [tokens, chunk] logits and fp32 per-token vectors are ever live.  With
``chunk >= vocab`` the one chunk's logits are kept from the forward instead
(the [tokens, vocab] buffer the reference also holds): the backward then
skips the recomputation, a quarter of the head's MFMA work, and forms dx in
one product.
"""
from __future__ import annotations

import torch

from . import kernels as K
from ._abi import check, dtype_code, lib, ptr, stream_handle
from .functional import rms_norm


def _fwd_chunk(logits, labels, col0, run_max, run_sum, target):
    check(lib().zk_ce_fwd_chunk(ptr(logits), logits.shape[0], logits.shape[1], logits.stride(0),
                                ptr(labels), col0, ptr(run_max), ptr(run_sum), ptr(target),
                                dtype_code(logits.dtype), stream_handle(logits.device)),
          "zk_ce_fwd_chunk")


def _bwd_chunk(logits, labels, col0, lse, scale):
    check(lib().zk_ce_bwd_chunk(ptr(logits), logits.shape[0], logits.shape[1], logits.stride(0),
                                ptr(labels), col0, ptr(lse), float(scale),
                                dtype_code(logits.dtype), stream_handle(logits.device)),
          "zk_ce_bwd_chunk")


class LMHeadCrossEntropyFunction(torch.autograd.Function):
    """loss = mean_t CE(x_t W^T, label_t) over tokens whose label is not
    ``ignore_index`` -- F.cross_entropy's semantics: every other label must
    lie in [0, V) (checked on the host; an out-of-range label raises
    ValueError as F.cross_entropy raises on it)."""

    @staticmethod
    def forward(ctx, x, weight, labels, chunk, ignore_index=-100):
        K._require_gpu(x, weight, labels)
        if x.dim() != 2 or weight.dim() != 2 or x.shape[1] != weight.shape[1]:
            raise ValueError("x must be [T, h] and weight [V, h]")
        if labels.dtype != torch.int64 or labels.shape != (x.shape[0],):
            raise ValueError("labels must be int64 [T]")
        x = x.contiguous()
        w = weight if weight.dtype == x.dtype else weight.to(x.dtype)
        T, V = x.shape[0], w.shape[0]
        ignored = labels == ignore_index
        if bool((~ignored & ((labels < 0) | (labels >= V))).any()):
            raise ValueError(f"labels must lie in [0, {V}) or equal ignore_index "
                             f"({ignore_index})")
        # the kernels skip rows whose label is negative
        labels = torch.where(ignored, torch.full_like(labels, -1), labels).contiguous()
        run_max = torch.full((T,), float("-inf"), device=x.device, dtype=torch.float32)
        run_sum = torch.zeros(T, device=x.device, dtype=torch.float32)
        target = torch.zeros(T, device=x.device, dtype=torch.float32)
        for c0 in range(0, V, chunk):
            logits = K.gemm(x, w[c0:c0 + chunk])
            _fwd_chunk(logits, labels, c0, run_max, run_sum, target)
        lse = run_max + torch.log(run_sum)
        valid = labels >= 0
        n_valid = valid.sum()
        loss = torch.where(valid, lse - target, torch.zeros_like(lse)).sum() / n_valid.clamp(min=1)
        ctx.save_for_backward(x, w, labels, lse, n_valid)
        ctx.chunk = chunk
        ctx.weight_dtype = weight.dtype
        # one chunk covered the vocabulary: keep its logits for the backward
        ctx.logits = logits if chunk >= V else None
        return loss

    @staticmethod
    def backward(ctx, g):
        x, w, labels, lse, n_valid = ctx.saved_tensors
        chunk = ctx.chunk
        T, V = x.shape[0], w.shape[0]
        scale = (g / n_valid.clamp(min=1)).item()
        if ctx.logits is not None:
            # the forward's logits, overwritten in place by their gradient (a
            # second backward through a retained graph recomputes them)
            dlog, ctx.logits = ctx.logits, None
            _bwd_chunk(dlog, labels, 0, lse, scale)
            dx = K.gemm(dlog, w, b_kmajor=True)
            dw = K.gemm(dlog, x, a_kmajor=True, b_kmajor=True)
            if dw.dtype != ctx.weight_dtype:
                dw = dw.to(ctx.weight_dtype)
            return dx, dw, None, None, None
        dx = torch.zeros(x.shape, device=x.device, dtype=torch.float32)
        dw = torch.empty_like(w)
        for c0 in range(0, V, chunk):
            wc = w[c0:c0 + chunk]
            dlog = K.gemm(x, wc)
            _bwd_chunk(dlog, labels, c0, lse, scale)
            dx.add_(K.gemm(dlog, wc, b_kmajor=True))
            K.gemm(dlog, x, a_kmajor=True, b_kmajor=True, out=dw[c0:c0 + chunk])
        if dw.dtype != ctx.weight_dtype:
            dw = dw.to(ctx.weight_dtype)
        return dx.to(x.dtype), dw, None, None, None


# Default chunking: the whole vocabulary in one chunk (logits kept for the
# backward) while the [tokens, vocab] logits take at most this many bytes,
# else chunks of 8192 columns.  Measured at 4096 tokens, hidden 4096, vocab
# 49152 (403 MB of bf16 logits), fwd + bwd: 3.85 ms in one chunk, 5.11 ms in
# 8192-column chunks, 5.40 ms for F.linear + F.cross_entropy.
SINGLE_CHUNK_BYTES = 1 << 30


def default_chunk(tokens: int, vocab: int, dtype: torch.dtype) -> int:
    elem = torch.empty((), dtype=dtype).element_size()
    return vocab if tokens * vocab * elem <= SINGLE_CHUNK_BYTES else 8192


def lm_head_cross_entropy(x, weight, labels, chunk: int | None = None, ignore_index: int = -100):
    """Mean cross-entropy of logits x W^T against labels, skipping tokens whose
    label is ``ignore_index`` (F.cross_entropy's default -100); x [..., h] is
    flattened over its leading dims.  ``chunk``: vocabulary columns per pass
    (default: default_chunk)."""
    h = x.shape[-1]
    x2 = x.reshape(-1, h)
    if chunk is None:
        chunk = default_chunk(x2.shape[0], weight.shape[0], x.dtype)
    return LMHeadCrossEntropyFunction.apply(x2, weight, labels.reshape(-1), int(chunk),
                                            int(ignore_index))


class OutputLayerLoss(torch.nn.Module):
    """norm -> lm_head -> cross-entropy, the last stage's tail, returning only
    the loss (the logits are kept whole for the backward only while they take
    at most SINGLE_CHUNK_BYTES, see default_chunk): wraps an existing ``norm``
    (RMSNorm module) and ``lm_head`` (nn.Linear without bias)."""

    def __init__(self, norm, lm_head, chunk: int | None = None):
        super().__init__()
        self.norm, self.lm_head, self.chunk = norm, lm_head, chunk

    def forward(self, x, labels):
        y = rms_norm(x, self.norm.weight, self.norm.variance_epsilon)
        return lm_head_cross_entropy(y, self.lm_head.weight, labels, self.chunk)
