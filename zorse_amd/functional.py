"""Autograd functions over the HIP kernels (RMSNorm, RoPE + flash attention,
SwiGLU), usable on their own; the fused decoder layer lives in ``layer.py``.

RoPE tables are built once per (S, d, theta, pairing, dtype, device) with the
reference's formula (models/llama_simple.py:75-81, 115-137: inv_freq and the
position product in fp32, cos/sin rounded to the activation dtype for the
half-split pairing; models/llama_v2.py:102-122 for the interleaved pairing,
which stays fp32) and handed to the kernel as fp32 [S, d/2] tables.
"""
from __future__ import annotations

import math
import threading

import torch

from . import kernels as K


# ------------------------------------------------------------- RoPE tables --

_rope_cache: dict = {}
_rope_lock = threading.Lock()


def rope_tables(seq: int, head_dim: int, theta: float, dtype: torch.dtype,
                device: torch.device, interleaved: bool = False):
    """fp32 cos / sin tables [seq, head_dim/2] holding exactly the values the
    reference multiplies by (rounded to ``dtype`` for the half-split form)."""
    key = (seq, head_dim, float(theta), dtype, str(device), interleaved)
    with _rope_lock:
        hit = _rope_cache.get(key)
    if hit is not None:
        return hit
    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.int64).float() / head_dim))
    pos = torch.arange(seq, dtype=torch.int64).float()
    freqs = torch.outer(pos, inv_freq)  # fp32 on the host: deterministic tables
    cos, sin = freqs.cos(), freqs.sin()
    if not interleaved and dtype != torch.float32:
        cos, sin = cos.to(dtype).float(), sin.to(dtype).float()
    tab = (cos.contiguous().to(device), sin.contiguous().to(device))
    with _rope_lock:
        _rope_cache[key] = tab
    return tab


# ---------------------------------------------------------------- RMSNorm --

class RMSNormFunction(torch.autograd.Function):
    """y = w * round(x * rsqrt(mean(x^2) + eps)) -- HF LlamaRMSNorm.forward
    (imported at models/llama_simple.py:9)."""

    @staticmethod
    def forward(ctx, x, weight, eps):
        shape = x.shape
        x2 = x.contiguous().view(-1, shape[-1])
        y, rstd, _ = K.rmsnorm_fwd(x2, weight.contiguous(), eps)
        ctx.save_for_backward(x2, weight, rstd)
        out_dtype = torch.promote_types(x.dtype, weight.dtype)
        y = y.view(shape)
        return y if out_dtype == y.dtype else y.to(out_dtype)

    @staticmethod
    def backward(ctx, dy):
        x2, weight, rstd = ctx.saved_tensors
        dy2 = dy.to(x2.dtype).contiguous().view_as(x2)
        dx, dw = K.rmsnorm_bwd(dy2, x2, weight.contiguous(), rstd,
                               dw_dtype=weight.dtype)
        return dx.view(dy.shape), dw, None


def rms_norm(x, weight, eps=1e-6):
    return RMSNormFunction.apply(x, weight, eps)


# ----------------------------------------------------------------- SwiGLU --

class SwiGLUFunction(torch.autograd.Function):
    """z = silu(g) * u on [T, F] (HF LlamaMLP's activation, models/
    llama_simple.py:418)."""

    @staticmethod
    def forward(ctx, g, u):
        g2 = g.contiguous().view(-1, g.shape[-1])
        u2 = u.contiguous().view(-1, u.shape[-1])
        z = K.swiglu_fwd(g2, u2)
        ctx.save_for_backward(g2, u2)
        return z.view(g.shape)

    @staticmethod
    def backward(ctx, dz):
        g2, u2 = ctx.saved_tensors
        dz2 = dz.contiguous().view_as(g2)
        dg, du = torch.empty_like(g2), torch.empty_like(u2)
        K.swiglu_bwd(dz2, g2, u2, dg, du)
        return dg.view(dz.shape), du.view(dz.shape)


def swiglu(g, u):
    return SwiGLUFunction.apply(g, u)


# -------------------------------------------------------------- Attention --

class FlashAttentionFunction(torch.autograd.Function):
    """Causal / sliding-window GQA attention with RoPE applied to Q and K
    first; [B, S, H, d] in and out.  The attention core replaces
    models/llama_simple.py:320-342 (and the FA2 / SDPA classes chosen at
    :376-416); RoPE replaces apply_rotary_pos_emb (:34-58)."""

    @staticmethod
    def forward(ctx, q, k, v, causal, window, scale, rope_theta, interleaved):
        B, S, Hq, d = q.shape
        if rope_theta is not None:
            cos, sin = rope_tables(S, d, rope_theta, q.dtype, q.device, interleaved)
            q = q.contiguous().clone()
            k = k.contiguous().clone()
            K.rope_(q, k, cos, sin, interleaved=interleaved)
        o, lse = K.attn_fwd(q, k, v, causal=causal, window=window, scale=scale)
        ctx.save_for_backward(q, k, v, o, lse)
        ctx.cfg = (causal, window, scale, rope_theta, interleaved)
        return o

    @staticmethod
    def backward(ctx, do):
        q, k, v, o, lse = ctx.saved_tensors
        causal, window, scale, rope_theta, interleaved = ctx.cfg
        do = do.contiguous()
        if do.stride() != o.stride():
            do = do.view(o.shape)
        rope = None
        if rope_theta is not None:
            B, S, Hq, d = q.shape
            cos, sin = rope_tables(S, d, rope_theta, q.dtype, q.device, interleaved)
            rope = (cos, sin, None, interleaved)
        # with RoPE the kernels also apply the rotation's transpose to dq / dk
        dq, dk, dv = K.attn_bwd(q, k, v, o, do, lse, causal=causal, window=window,
                                scale=scale, rope=rope)
        return dq, dk, dv, None, None, None, None, None


def flash_attention(q, k, v, *, causal=True, window=0, scale=None, rope_theta=None,
                    interleaved=False):
    """Autograd entry: q [B,S,Hq,d], k / v [B,S,Hkv,d] (bf16 / fp16 / fp32)."""
    if scale is None:
        scale = 1.0 / math.sqrt(q.shape[-1])
    return FlashAttentionFunction.apply(q, k, v, bool(causal), int(window or 0),
                                        float(scale), rope_theta, bool(interleaved))
