"""Fused decoder-layer forward / backward over one flat parameter buffer.

One autograd node per layer: the whole of LlamaDecoderLayer.forward
(models/llama_simple.py:456-479) -- RMSNorm, the q|k|v projection as ONE GEMM,
RoPE, flash attention (GQA, causal / sliding window), o_proj, the residual
add fused into the second RMSNorm, gate|up as ONE GEMM with SwiGLU in its
epilogue, down with the residual folded into the GEMM -- and its backward, which
writes every weight gradient straight into one flat gradient buffer laid out like the flat
parameter (q, k, v, o, gate, up, down, ln1, ln2 -- the registration order the
reference's FSDP flat parameter uses, zorse_utils/pipeline.py:120-148).

Because q, k, v (and gate, up) are adjacent in that order, the fused
projection weights are plain views of the flat buffer, and their gradients
are single GEMMs into adjacent slices: no concatenation, no gradient copies.
"""
from __future__ import annotations

import math
import os
from dataclasses import dataclass

import torch

from . import kernels as K
from .functional import rope_tables

PARAM_ORDER = ("q", "k", "v", "o", "gate", "up", "down", "ln1", "ln2")


@dataclass(frozen=True)
class LayerSpec:
    hidden: int
    heads: int
    kv_heads: int
    head_dim: int
    ffn: int
    eps: float = 1e-6
    rope_theta: float = 1e4
    causal: bool = True
    window: int = 0
    interleaved_rope: bool = False

    def __post_init__(self):
        if self.heads % self.kv_heads:
            raise ValueError(f"heads={self.heads} not a multiple of kv_heads={self.kv_heads}")
        if self.head_dim % 2:
            raise ValueError("head_dim must be even")

    @property
    def q_dim(self) -> int:
        return self.heads * self.head_dim

    @property
    def kv_dim(self) -> int:
        return self.kv_heads * self.head_dim

    @property
    def qkv_dim(self) -> int:
        return self.q_dim + 2 * self.kv_dim

    def shapes(self) -> dict[str, tuple[int, ...]]:
        h, F = self.hidden, self.ffn
        return {"q": (self.q_dim, h), "k": (self.kv_dim, h), "v": (self.kv_dim, h),
                "o": (h, self.q_dim), "gate": (F, h), "up": (F, h), "down": (h, F),
                "ln1": (h,), "ln2": (h,)}

    def offsets(self) -> dict[str, tuple[int, int]]:
        out, off = {}, 0
        for k, shp in self.shapes().items():
            n = math.prod(shp)
            out[k] = (off, off + n)
            off += n
        return out

    @property
    def numel(self) -> int:
        return sum(math.prod(s) for s in self.shapes().values())


class FlatViews:
    """Named views of a flat buffer laid out as LayerSpec.offsets()."""

    def __init__(self, spec: LayerSpec, flat: torch.Tensor):
        o = spec.offsets()
        h, F = spec.hidden, spec.ffn

        def v(a, b, shp):
            return flat[a:b].view(shp)

        self.qkv = v(o["q"][0], o["v"][1], (spec.qkv_dim, h))
        self.o = v(*o["o"], (h, spec.q_dim))
        self.gu = v(o["gate"][0], o["up"][1], (2 * F, h))
        self.down = v(*o["down"], (h, F))
        self.ln1 = flat[o["ln1"][0]:o["ln1"][1]]
        self.ln2 = flat[o["ln2"][0]:o["ln2"][1]]


# Every projection product runs on the hand-written GEMMs (zk_gemm) with the
# operands as the layer holds them: the forward x W^T and the backward's
# input gradients dY W (W read K-major) and weight gradients dY^T X (both
# token-major activations read K-major; for gate|up and q|k|v, dY^T as the
# SwiGLU / attention backward kernels also write it from their epilogues) --
# no transpose pass, and no product goes to a library GEMM.


def _linear(x, w, residual=None):
    """x W^T (+ residual, one rounding): the nn.Linear forward."""
    return K.gemm(x, w, residual=residual)


def _dgrad(dy, w):
    """dy W: the input gradient of y = x W^T, W [out, in] read as stored."""
    return K.gemm(dy, w, b_kmajor=True)


def _wgrad(dy, x, out, dyt=None):
    """out = dy^T x: the weight gradient of y = x W^T, from the token-major
    dy [T, out] and x [T, in] as stored -- or, when the kernel that produced
    dy also wrote ``dyt`` = dy^T [out, T] from its epilogue, from dyt read
    along the reduction.  The second form runs the GEMM with one K-major
    operand instead of two, ~25 % faster at the 7B shapes (the two-K-major
    form runs at ~55 % MFMA-busy against ~75 %)."""
    if dyt is not None:
        K.gemm(dyt, x, b_kmajor=True, out=out)
    else:
        K.gemm(dy, x, a_kmajor=True, b_kmajor=True, out=out)


# The gate|up and q|k|v weight gradients dY^T X read dY either K-major as the
# input-gradient chain holds it (both operands K-major) or from a dY^T that the
# SwiGLU / attention backward kernels also write from their epilogues (the
# input-gradient form).  The K-major form of those two products is only 1-3 %
# slower (alone, 7B shapes), and in the 7B stage (one process, alternating,
# three rounds, on two boxes) the two arrangements measured equal: 42.30-42.48
# ms/step without the transposed copies against 42.37-42.56 with them; with
# those two products in order on the compute stream, 40.87-40.91 without
# against 40.95-41.10 with (one box, four alternating rounds).  On by default,
# which keeps the input-gradient form the stage's dominant kernel;
# set_transposed_wgrad(False) or ZORSE_TRANSPOSED_WGRAD=0 writes no copies
# (280 MB less written and allocated per layer backward).
_transposed_wgrad = os.environ.get("ZORSE_TRANSPOSED_WGRAD", "1") != "0"


def set_transposed_wgrad(enable: bool) -> bool:
    """Take the gate|up and q|k|v weight gradients from the dY^T the SwiGLU /
    attention backward write (True) or from dY as stored (False); returns the
    previous setting."""
    global _transposed_wgrad
    prev, _transposed_wgrad = _transposed_wgrad, bool(enable)
    return prev


def _transposed_outputs(t):
    """True when the SwiGLU / attention backward kernels are to write their
    result transposed as well (enabled, 2-byte types, token counts multiples
    of 8)."""
    return (_transposed_wgrad and t.dtype in (torch.bfloat16, torch.float16)
            and t.shape[0] % 8 == 0)


# The four weight-gradient GEMMs of a layer's backward are off its critical
# path: nothing in the layer's backward reads them.  Those of down_proj and
# o_proj run on a side stream beside the input-gradient chain (the down
# input-gradient GEMM and the SwiGLU backward; the attention backward), so the
# partial last round of one GEMM's tiles fills with work of the other instead
# of idling; those of gate|up and q|k|v run in order on the compute stream.
# The layer's backward joins the side stream before it returns its gradient,
# and a cross-stream wait costs ~25 us on this GPU before the waiting queue's
# next kernel starts: with q|k|v's product last on the side stream, the join
# waited for it every layer.  7B stage, one process, alternating, two boxes:
# 41.39-41.54 ms/step this way, 41.52-41.68 with all four on the side stream,
# 41.98-42.03 with all four in order, 41.54-41.66 with only gate|up in order.
# ZORSE_WGRAD_STREAM=0 or set_wgrad_stream(False) runs all four in order on the
# compute stream.
_wgrad_side = os.environ.get("ZORSE_WGRAD_STREAM", "1") != "0"
_side_streams: dict = {}


def set_wgrad_stream(enable: bool) -> bool:
    """Run the weight-gradient GEMMs on a side stream (True) or in order on the
    compute stream; returns the previous setting."""
    global _wgrad_side
    prev, _wgrad_side = _wgrad_side, bool(enable)
    return prev


class _WeightGrads:
    """Enqueues a layer backward's weight-gradient GEMMs on a default-priority
    side stream (after the compute stream's work so far) or, when disabled,
    on the compute stream; join() makes the compute stream wait for them."""

    def __init__(self, device, grad_flat):
        self.main = torch.cuda.current_stream(device)
        self.side = None
        if _wgrad_side:
            self.side = _side_streams.get(device)
            if self.side is None:
                self.side = _side_streams[device] = torch.cuda.Stream(device=device)
            grad_flat.record_stream(self.side)

    def __call__(self, dy, x, out, dyt=None, in_order=False):
        if self.side is None or in_order:
            _wgrad(dy, x, out, dyt)
            return
        self.side.wait_stream(self.main)
        with torch.cuda.stream(self.side):
            _wgrad(dy, x, out, dyt)
        # the compute stream may free and reuse dy / dyt / x before the side
        # stream has read them
        for t in (dy, x, dyt):
            if t is not None:
                t.record_stream(self.side)

    def join(self):
        if self.side is not None:
            self.main.wait_stream(self.side)


# gate|up GEMM with the SwiGLU activation in its epilogue (zk_gemm_swiglu:
# writes g, u and z in one pass) for 2-byte types; otherwise the GEMM and a
# separate SwiGLU pass.  On by default: in the 7B stage it measured equal to
# the GEMM plus the SwiGLU pass; ZORSE_FUSED_MLP=0 or set_fused_gate_up(False)
# turns it off (the separate pass computes SiLU with the IEEE exp and
# division, the fused epilogue with the hardware exp2 and reciprocal).
_fused_gate_up = os.environ.get("ZORSE_FUSED_MLP", "1") != "0"


def set_fused_gate_up(enable: bool) -> bool:
    """Enable / disable the fused gate|up + SwiGLU GEMM; returns the previous setting."""
    global _fused_gate_up
    prev, _fused_gate_up = _fused_gate_up, bool(enable)
    return prev


def _fused_gate_up_takes(n2, F):
    """zk_gemm_swiglu's conditions: 2-byte type, K a multiple of 64, tokens
    and F multiples of 8."""
    T, h = n2.shape
    return (_fused_gate_up and n2.dtype in (torch.bfloat16, torch.float16)
            and h % 64 == 0 and T % 8 == 0 and F % 8 == 0)


# Head dims the MFMA attention kernels do not take (they take 64 and 128; the
# fp32 kernels any head dim up to 128): q, k, v are zero-padded to the next of
# those, attention runs with the real head dim's scale -- the padded
# coordinates add nothing to Q K^T, P V or any gradient -- and the results are
# sliced back.  RoPE rotates the real coordinates in place before (forward),
# and its transpose is applied to dq / dk after the backward.  The padding
# copies are torch copies into zeroed buffers (head dims 48 - 110 of the
# smaller llama_* HF-factory models only).
def _attn_padded_dim(spec, dtype):
    d = spec.head_dim
    if dtype == torch.float32 or d in (64, 128):
        return None
    if d < 64:
        return 64
    if d < 128:
        return 128
    raise NotImplementedError(f"head_dim {d}: the attention kernels take head dims up to 128")


def _pad_heads(t, dp):
    """[B, S, H, d] -> a zero-padded [B, S, H, dp] copy."""
    out = t.new_zeros(*t.shape[:3], dp)
    out[..., :t.shape[3]].copy_(t)
    return out


def _rope_for(S, spec, dtype, device, positions):
    """RoPE tables covering positions 0 .. S-1, or 0 .. max(positions) when
    explicit positions are given (int64 [S] on the device)."""
    n_pos = S
    if positions is not None:
        n_pos = max(S, int(positions.max().item()) + 1)
    return rope_tables(n_pos, spec.head_dim, spec.rope_theta, dtype, device,
                       spec.interleaved_rope)


def layer_forward(x: torch.Tensor, w: FlatViews, spec: LayerSpec, attn_cache=None,
                  positions: torch.Tensor | None = None):
    """Forward on compute-dtype tensors; returns (out, saved tuple).

    ``attn_cache`` (optional) is an AttentionCache: a hit supplies the
    attention output and LSE of an earlier forward of the same input and
    weights, so the attention forward is skipped (the recompute of the
    reference's pipeline backward); a miss computes them and records them.
    ``positions`` (optional): int64 [S] token positions for RoPE, shared by
    the batch (default 0 .. S-1)."""
    B, S, h = x.shape
    T = B * S
    d, Hq, Hkv = spec.head_dim, spec.heads, spec.kv_heads
    x2 = x.reshape(T, h)
    n1, rstd1, _ = K.rmsnorm_fwd(x2, w.ln1, spec.eps)
    # q|k|v [T, (Hq + 2 Hkv) d] with RoPE applied to the q and k heads in the
    # GEMM's epilogue (zk_gemm_rope; the same values as the product followed
    # by the rotation pass)
    cos, sin = _rope_for(S, spec, x.dtype, x.device, positions)
    qkv = K.gemm_rope(n1, w.qkv, seq_len=S, rot_cols=spec.q_dim + spec.kv_dim, head_dim=d,
                      cos=cos, sin=sin, positions=positions, interleaved=spec.interleaved_rope)
    q = qkv[:, :spec.q_dim].view(B, S, Hq, d)
    k = qkv[:, spec.q_dim:spec.q_dim + spec.kv_dim].view(B, S, Hkv, d)
    v = qkv[:, spec.q_dim + spec.kv_dim:].view(B, S, Hkv, d)
    hit = attn_cache.take() if attn_cache is not None else None
    if hit is not None:
        o, lse = hit
    else:
        dp = _attn_padded_dim(spec, x.dtype)
        if dp is None:
            o, lse = K.attn_fwd(q, k, v, causal=spec.causal, window=spec.window)
        else:
            o, lse = K.attn_fwd(_pad_heads(q, dp), _pad_heads(k, dp), _pad_heads(v, dp),
                                causal=spec.causal, window=spec.window,
                                scale=1.0 / math.sqrt(d))
            o = o[..., :d].contiguous()
        if attn_cache is not None:
            attn_cache.put(o, lse)
    o2 = o.view(T, spec.q_dim)
    # o_proj, then residual add fused into the second RMSNorm (one pass writes
    # hdn = x + round(o_proj) and its normalisation, the reference's order)
    attn_out = _linear(o2, w.o)
    n2, rstd2, hdn = K.rmsnorm_fwd(attn_out, w.ln2, spec.eps, residual=x2)
    F = spec.ffn
    if _fused_gate_up_takes(n2, F):
        # one GEMM writes gate | up (kept for the backward) and z
        gu, z = K.gemm_swiglu(n2, w.gu[:F], w.gu[F:])
    else:
        gu = _linear(n2, w.gu)                       # [T, 2F] = gate | up
        z = K.swiglu_fwd(gu[:, :F], gu[:, F:])
    out = _linear(z, w.down, residual=hdn)           # residual + down(z)
    saved = (x2, n1, rstd1, qkv, o2, lse, hdn, n2, rstd2, gu, z, positions)
    return out.view(B, S, h), saved


# Host callbacks run right before a layer's attention backward is enqueued
# (the stage runner starts the previous layer's optimizer step there, so the
# HBM-bound update runs beside the LDS-bound attention kernels rather than
# beside the projection GEMMs).
BEFORE_ATTENTION_BACKWARD: list = []


def layer_backward(dout: torch.Tensor, saved, w: FlatViews, spec: LayerSpec,
                   grad_flat: torch.Tensor) -> torch.Tensor:
    """Backward of layer_forward; writes weight grads into ``grad_flat``
    (compute dtype, flat layout) and returns dx."""
    x2, n1, rstd1, qkv, o2, lse, hdn, n2, rstd2, gu, z, positions = saved
    T, h = x2.shape
    B = dout.shape[0]
    S = T // B
    d, Hq, Hkv, F = spec.head_dim, spec.heads, spec.kv_heads, spec.ffn
    g = FlatViews(spec, grad_flat)
    dout2 = dout.reshape(T, h)
    wgrad = _WeightGrads(dout.device, grad_flat)

    # MLP: out = hdn + z W_down^T
    wgrad(dout2, z, g.down)
    dz = _dgrad(dout2, w.down)                       # [T, F]
    dgu = torch.empty_like(gu)
    dgut = None
    if _transposed_outputs(gu) and F % 8 == 0:
        # dgu^T [2F, T] from the same pass, for the gate|up weight gradient
        dgut = torch.empty(2 * F, T, device=gu.device, dtype=gu.dtype)
        K.swiglu_bwd_t(dz, gu[:, :F], gu[:, F:], dgu[:, :F], dgu[:, F:], dgut[:F], dgut[F:])
    else:
        K.swiglu_bwd(dz, gu[:, :F], gu[:, F:], dgu[:, :F], dgu[:, F:])
    del dz
    wgrad(dgu, n2, g.gu, dgut, in_order=True)
    dn2 = _dgrad(dgu, w.gu)                          # [T, h]
    del dgu, dgut
    dh, _ = K.rmsnorm_bwd(dn2, hdn, w.ln2, rstd2, dres=dout2, dw=g.ln2)
    del dn2

    # attention: hdn = x + o W_o^T
    wgrad(dh, o2, g.o)
    do2 = _dgrad(dh, w.o)                            # [T, Hq d]
    q = qkv[:, :spec.q_dim].view(B, S, Hq, d)
    k = qkv[:, spec.q_dim:spec.q_dim + spec.kv_dim].view(B, S, Hkv, d)
    v = qkv[:, spec.q_dim + spec.kv_dim:].view(B, S, Hkv, d)
    dqkv = torch.empty_like(qkv)
    dq = dqkv[:, :spec.q_dim].view(B, S, Hq, d)
    dk = dqkv[:, spec.q_dim:spec.q_dim + spec.kv_dim].view(B, S, Hkv, d)
    dv = dqkv[:, spec.q_dim + spec.kv_dim:].view(B, S, Hkv, d)
    for fn in list(BEFORE_ATTENTION_BACKWARD):
        fn()
    cos, sin = _rope_for(S, spec, dout.dtype, dout.device, positions)
    dp = _attn_padded_dim(spec, dout.dtype)
    dqkvt = None
    if dp is None:
        # the attention backward also takes dq / dk back through RoPE's
        # rotation, and writes dqkv^T [(Hq + 2 Hkv) d, T] from its epilogues
        # for the q|k|v weight gradient
        if _transposed_outputs(qkv) and S % 8 == 0:
            dqkvt = torch.empty(qkv.shape[1], T, device=qkv.device, dtype=qkv.dtype)
        kv0, kv1 = spec.q_dim, spec.q_dim + spec.kv_dim
        K.attn_bwd(q, k, v, o2.view(B, S, Hq, d), do2.view(B, S, Hq, d), lse,
                   causal=spec.causal, window=spec.window, dq=dq, dk=dk, dv=dv,
                   rope=(cos, sin, positions, spec.interleaved_rope),
                   transposed=None if dqkvt is None else
                   (dqkvt[:kv0], dqkvt[kv0:kv1], dqkvt[kv1:]))
    else:
        grads = K.attn_bwd(*(_pad_heads(t, dp) for t in (q, k, v, o2.view(B, S, Hq, d),
                                                         do2.view(B, S, Hq, d))), lse,
                           causal=spec.causal, window=spec.window, scale=1.0 / math.sqrt(d))
        for dst, src in zip((dq, dk, dv), grads):
            dst.copy_(src[..., :d])
        del grads
        K.rope_(dq, dk, cos, sin, positions=positions, interleaved=spec.interleaved_rope,
                inverse=True)
    del do2
    wgrad(dqkv, n1, g.qkv, dqkvt, in_order=True)
    dn1 = _dgrad(dqkv, w.qkv)                        # [T, h]
    del dqkv, dqkvt
    dx, _ = K.rmsnorm_bwd(dn1, x2, w.ln1, rstd1, dres=dh, dw=g.ln1)
    wgrad.join()
    return dx.view(B, S, h)


class AttentionCache:
    """Attention outputs of forwards that will be recomputed.

    The reference's pipeline runs every layer forward twice per micro-batch:
    once without autograd, and again inside the backward to rebuild the
    activations (zorse_utils/pipeline_schedule_v2.py:157-200).  Between the
    two the input and the weights are unchanged, so the attention output O
    and its LSE can be kept from the first forward and the second skips the
    attention kernel.  Entries are keyed by the input's storage address,
    offset, shape, strides and version counter plus the weights' address and
    version counters; an entry keeps the input's storage alive, so no other
    tensor can take that address while the entry exists.  A caller that moves
    the input between the two forwards (host offload) sets ``token`` to an
    identifier of the micro-batch and layer instead.  A forward whose key has
    no entry computes attention and records it; an entry is removed when it
    is used."""

    def __init__(self):
        self._entries = {}
        self._key = None
        self._storage = None
        # Set by a caller that moves the input between the two forwards (the
        # stage runner's host offload): identifies the micro-batch and layer
        # in place of the input's storage.
        self.token = None

    def __len__(self):
        return len(self._entries)

    def clear(self):
        self._entries.clear()
        self._key = self._storage = None

    def bind(self, x, flat_param, w_flat):
        wkey = (flat_param._version, w_flat.data_ptr(), w_flat._version)
        if self.token is not None:
            self._storage = None
            self._key = ("token", self.token, tuple(x.shape)) + wkey
            return
        st = x.untyped_storage()
        self._storage = st
        self._key = (st.data_ptr(), x.storage_offset(), tuple(x.shape), tuple(x.stride()),
                     x._version) + wkey

    def take(self):
        """(o, lse) of the bound key's entry, removed, or None."""
        hit = self._entries.pop(self._key, None)
        if hit is None:
            return None
        self._storage = None  # the input's storage is no longer needed here
        return hit[1:]

    def put(self, o, lse):
        """Records O and its LSE."""
        self._entries[self._key] = (self._storage, o, lse)


class DecoderLayerFunction(torch.autograd.Function):
    """autograd node of one decoder layer: inputs (x, flat_param)."""

    @staticmethod
    def forward(ctx, x, flat_param, spec, weights_lowp, attn_cache=None, positions=None):
        w_flat = weights_lowp if weights_lowp is not None else flat_param
        w = FlatViews(spec, w_flat)
        if attn_cache is not None:
            attn_cache.bind(x, flat_param, w_flat)
        with torch.autocast("cuda", enabled=False):
            out, saved = layer_forward(x.contiguous(), w, spec, attn_cache, positions)
        ctx.spec = spec
        ctx.param_dtype = flat_param.dtype
        ctx.positions = saved[-1]
        ctx.save_for_backward(w_flat, *saved[:-1])
        return out

    @staticmethod
    def backward(ctx, dout):
        w_flat, *saved = ctx.saved_tensors
        saved = (*saved, ctx.positions)
        spec = ctx.spec
        w = FlatViews(spec, w_flat)
        dout = dout.to(w_flat.dtype).contiguous()
        grad_flat = torch.empty(spec.numel, device=dout.device, dtype=w_flat.dtype)
        with torch.autocast("cuda", enabled=False):
            dx = layer_backward(dout, saved, w, spec, grad_flat)
        if ctx.param_dtype != grad_flat.dtype:
            grad_flat = grad_flat.to(ctx.param_dtype)
        return dx, grad_flat, None, None, None, None
