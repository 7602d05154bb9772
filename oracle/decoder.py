"""Plain-PyTorch CPU restatement of one Llama / Mistral decoder layer.

Test infrastructure only (see ``oracle/__init__.py``).  Tensors are in the
[B, S, H, d] ("BSHD") layout the GPU path uses; the reference transposes to
[B, H, S, d] (models/llama_simple.py:297-305), which changes no value.

Every function computes in the dtype of its inputs, so passing fp64 tensors
gives the golden fp64 result and passing fp32 tensors gives the CPU baseline.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch
import torch.nn.functional as F


# ----------------------------------------------------------------- config --

@dataclass(frozen=True)
class LayerShape:
    """Shape of one decoder layer (names follow HF LlamaConfig / MistralConfig)."""

    hidden: int
    heads: int
    kv_heads: int
    head_dim: int
    ffn: int
    eps: float = 1e-6
    theta: float = 1e4
    causal: bool = True
    window: int = 0           # 0: no sliding window

    @property
    def n_rep(self) -> int:
        return self.heads // self.kv_heads


# Order in which the reference registers a decoder layer's parameters, which
# is also the order of FSDP's flat parameter (use_orig_params=False):
# self_attn.{q,k,v,o}_proj (models/llama_simple.py:206-221), mlp.{gate,up,down}
# (HF LlamaMLP, built at models/llama_simple.py:418), input_layernorm,
# post_attention_layernorm (models/llama_simple.py:419-422).
PARAM_ORDER = ("q", "k", "v", "o", "gate", "up", "down", "ln1", "ln2")


def param_shapes(s: LayerShape) -> dict[str, tuple[int, ...]]:
    qd, kd = s.heads * s.head_dim, s.kv_heads * s.head_dim
    return {
        "q": (qd, s.hidden), "k": (kd, s.hidden), "v": (kd, s.hidden),
        "o": (s.hidden, qd), "gate": (s.ffn, s.hidden), "up": (s.ffn, s.hidden),
        "down": (s.hidden, s.ffn), "ln1": (s.hidden,), "ln2": (s.hidden,),
    }


def flat_numel(s: LayerShape) -> int:
    return sum(math.prod(v) for v in param_shapes(s).values())


def flatten(p: dict[str, torch.Tensor]) -> torch.Tensor:
    return torch.cat([p[k].reshape(-1) for k in PARAM_ORDER])


def unflatten(flat: torch.Tensor, s: LayerShape) -> dict[str, torch.Tensor]:
    out, off = {}, 0
    for k, shp in param_shapes(s).items():
        n = math.prod(shp)
        out[k] = flat[off:off + n].view(shp)
        off += n
    return out


def init_params(s: LayerShape, gen: torch.Generator, dtype=torch.float32,
                std: float = 0.02, random_norm: bool = False) -> dict[str, torch.Tensor]:
    """Linear weights N(0, std); norm weights ones (the module default) or
    1 + N(0, 0.1) when ``random_norm``."""
    p = {}
    for k in PARAM_ORDER:
        shp = param_shapes(s)[k]
        if k.startswith("ln"):
            w = torch.ones(shp, dtype=torch.float32)
            if random_norm:
                w = w + 0.1 * torch.randn(shp, generator=gen, dtype=torch.float32)
        else:
            w = std * torch.randn(shp, generator=gen, dtype=torch.float32)
        p[k] = w.to(dtype)
    return p


# ---------------------------------------------------------------- RMSNorm --

def rmsnorm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    """HF LlamaRMSNorm.forward (imported at models/llama_simple.py:9, built at
    :419-422; transformers modeling_llama.py LlamaRMSNorm): variance in fp32 (or
    wider), normalised value cast back to the input dtype, then times w."""
    acc = torch.float64 if x.dtype == torch.float64 else torch.float32
    h = x.to(acc)
    var = h.pow(2).mean(-1, keepdim=True)
    h = h * torch.rsqrt(var + eps)
    return w * h.to(x.dtype)


def rmsnorm_rstd(x: torch.Tensor, eps: float) -> torch.Tensor:
    """The per-row factor rsqrt(mean(x^2) + eps) of rmsnorm (HF LlamaRMSNorm's
    ``torch.rsqrt(variance + eps)``), fp32 (fp64 for fp64 input): the value the
    GPU forward saves for the backward."""
    acc = torch.float64 if x.dtype == torch.float64 else torch.float32
    return torch.rsqrt(x.to(acc).pow(2).mean(-1) + eps)


def rmsnorm_bwd(dy, x, w, eps):
    """Closed-form gradient of rmsnorm (fp32/fp64 throughout):
    xh = x r, g = dy w; dx = r (g - xh mean(g xh)); dw = sum_rows dy xh."""
    acc = torch.float64 if x.dtype == torch.float64 else torch.float32
    xf, dyf, wf = x.to(acc), dy.to(acc), w.to(acc)
    r = torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    xh = xf * r
    g = dyf * wf
    dx = r * (g - xh * (g * xh).mean(-1, keepdim=True))
    dw = (dyf * xh).reshape(-1, x.shape[-1]).sum(0)
    return dx, dw


# ------------------------------------------------------------------- RoPE --

def rope_inv_freq(head_dim: int, theta: float) -> torch.Tensor:
    """inv_freq[i] = 1 / theta^(2i/d) in fp32 (models/llama_simple.py:75-81)."""
    return 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.int64).float() / head_dim))


def rope_cos_sin(seq: int, head_dim: int, theta: float, dtype=torch.float32,
                 positions: torch.Tensor | None = None):
    """cos / sin tables [S, d] of LlamaRotaryEmbedding.forward
    (models/llama_simple.py:115-137): freqs = inv_freq x position in fp32 with
    autocast off, emb = cat(freqs, freqs), cos/sin cast to the activation
    dtype."""
    pos = torch.arange(seq, dtype=torch.int64) if positions is None else positions
    freqs = torch.outer(pos.float(), rope_inv_freq(head_dim, theta))
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos().to(dtype), emb.sin().to(dtype)


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    """models/llama_simple.py:27-31 -- cat(-x2, x1) over the last dim."""
    h = x.shape[-1] // 2
    return torch.cat((-x[..., h:], x[..., :h]), dim=-1)


def apply_rope_half(q: torch.Tensor, k: torch.Tensor, cos: torch.Tensor,
                    sin: torch.Tensor):
    """apply_rotary_pos_emb (models/llama_simple.py:34-58) on BSHD tensors:
    cos/sin [S, d] broadcast over batch and heads."""
    c = cos[None, :, None, :]
    s = sin[None, :, None, :]
    return q * c + rotate_half(q) * s, k * c + rotate_half(k) * s


def rope_freqs_cis(head_dim: int, end: int, theta: float) -> torch.Tensor:
    """precompute_freqs_cis (models/llama_v2.py:102-122): complex64 [end, d/2]."""
    freqs = 1.0 / (theta ** (torch.arange(0, head_dim, 2)[: head_dim // 2].float() / head_dim))
    t = torch.arange(end, device=freqs.device)
    freqs = torch.outer(t, freqs).float()
    return torch.polar(torch.ones_like(freqs), freqs)


def apply_rope_interleaved(xq: torch.Tensor, xk: torch.Tensor, freqs_cis: torch.Tensor):
    """apply_rotary_emb (models/llama_v2.py:151-177): adjacent pairs (2i, 2i+1)
    rotated as complex numbers in fp32 (fp64 inputs stay fp64), cast back."""
    S = xq.shape[1]
    fc = freqs_cis[:S]
    if xq.dtype == torch.float64:
        fc = fc.to(torch.complex128)
        cq, ck = xq, xk
    else:
        cq, ck = xq.float(), xk.float()
    q_ = torch.view_as_complex(cq.reshape(*xq.shape[:-1], -1, 2).contiguous())
    k_ = torch.view_as_complex(ck.reshape(*xk.shape[:-1], -1, 2).contiguous())
    f = fc[None, :, None, :]
    return (torch.view_as_real(q_ * f).flatten(3).type_as(xq),
            torch.view_as_real(k_ * f).flatten(3).type_as(xk))


# -------------------------------------------------------------- attention --

def repeat_kv(x: torch.Tensor, n_rep: int) -> torch.Tensor:
    """repeat_kv on BSHD (models/llama_v2.py:180-189; HF repeat_kv, used at
    models/llama_simple.py:320-321, is the same on BHSD): head j of the result
    is KV head j // n_rep."""
    if n_rep == 1:
        return x
    B, S, H, d = x.shape
    return x[:, :, :, None, :].expand(B, S, H, n_rep, d).reshape(B, S, H * n_rep, d)


def attn_mask(sq: int, skv: int, causal: bool, window: int, device=None) -> torch.Tensor:
    """Boolean [Sq, Skv] visibility: causal keeps key j <= query i; a sliding
    window W additionally keeps j > i - W (W keys including self), the
    convention of HF's sliding-window mask (transformers masking_utils)."""
    i = torch.arange(sq, device=device)[:, None]
    j = torch.arange(skv, device=device)[None, :]
    vis = torch.ones(sq, skv, dtype=torch.bool, device=device)
    if causal:
        vis &= j <= i
    if window and window > 0:
        vis &= j > i - window
    return vis


def attention(q, k, v, causal=True, window=0, scale=None):
    """softmax(Q K^T * scale + mask) V with GQA, BSHD in and out.

    Eager attention of models/llama_simple.py:320-342: scores in the input
    precision, softmax upcast to fp32 (or kept fp64) and cast back before PV
    (:336-338); scale 1/sqrt(d) (:323-325).  Returns (out [B,S,Hq,d],
    lse [B,Hq,S] natural-log logsumexp of the scaled masked scores)."""
    B, Sq, Hq, d = q.shape
    Hkv = k.shape[2]
    scale = 1.0 / math.sqrt(d) if scale is None else scale
    kk = repeat_kv(k, Hq // Hkv).transpose(1, 2)
    vv = repeat_kv(v, Hq // Hkv).transpose(1, 2)
    qq = q.transpose(1, 2)
    s = torch.matmul(qq, kk.transpose(-1, -2)) * scale
    acc = torch.float64 if q.dtype == torch.float64 else torch.float32
    s = s.to(acc)
    vis = attn_mask(Sq, k.shape[1], causal, window, q.device)
    s = s.masked_fill(~vis, float("-inf"))
    lse = torch.logsumexp(s, dim=-1)
    p = torch.softmax(s, dim=-1)
    p = torch.nan_to_num(p, nan=0.0).to(q.dtype)
    out = torch.matmul(p, vv).transpose(1, 2)
    return out, lse


def attention_bwd(q, k, v, do, causal=True, window=0, scale=None):
    """Closed-form attention gradient (FlashAttention-2 recurrences, Dao 2023):
    P = softmax(S), dV = P^T dO, dP = dO V^T, dS = P (dP - rowsum(dO o O)),
    dQ = scale dS K, dK = scale dS^T Q; GQA sums dK / dV over the group."""
    B, Sq, Hq, d = q.shape
    Hkv = k.shape[2]
    n_rep = Hq // Hkv
    scale = 1.0 / math.sqrt(d) if scale is None else scale
    kk = repeat_kv(k, n_rep).transpose(1, 2)
    vv = repeat_kv(v, n_rep).transpose(1, 2)
    qq = q.transpose(1, 2)
    dd = do.transpose(1, 2)
    s = torch.matmul(qq, kk.transpose(-1, -2)) * scale
    vis = attn_mask(Sq, k.shape[1], causal, window, q.device)
    s = s.masked_fill(~vis, float("-inf"))
    p = torch.nan_to_num(torch.softmax(s, dim=-1), nan=0.0)
    o = torch.matmul(p, vv)
    dv = torch.matmul(p.transpose(-1, -2), dd)
    dp = torch.matmul(dd, vv.transpose(-1, -2))
    delta = (dd * o).sum(-1, keepdim=True)
    ds = p * (dp - delta)
    dq = torch.matmul(ds, kk) * scale
    dk = torch.matmul(ds.transpose(-1, -2), qq) * scale
    Skv = k.shape[1]
    dk = dk.view(B, Hkv, n_rep, Skv, d).sum(2).transpose(1, 2)
    dv = dv.view(B, Hkv, n_rep, Skv, d).sum(2).transpose(1, 2)
    return dq.transpose(1, 2), dk, dv


def flash_attention_lowp(q, k, v, causal=True, window=0, scale=None):
    """Attention with the rounding points of the flash kernels the reference
    runs for its bf16 / fp16 layers (HF LlamaFlashAttention2 -> flash-attn, or
    LlamaSdpaAttention -> SDPA's flash backend, chosen at
    models/llama_simple.py:396-416; FlashAttention-2, Dao 2023):
      forward  S = scale Q K^T and the softmax in fp32; the unnormalised
               probabilities exp(S - rowmax) rounded to the storage dtype for
               the P V product (fp32 accumulation), divided by the fp32 row sum,
               O rounded;
      backward P = exp(S - lse) in fp32; dV = round(P)^T dO; dP = dO V^T;
               dS = P (dP - rowsum(dO o O)) rounded to the storage dtype for
               dQ = scale dS K and dK = scale dS^T Q (fp32 accumulation);
               with GQA each query head's dK / dV is rounded and the group is
               then summed (flash-attn's dk_expanded sum, or the autograd of
               repeat_kv on the SDPA path).
    Q/K/V in a 16-bit dtype (fp32 / fp64 inputs: no rounding at all, i.e.
    ``attention``).  Differentiable; returns O only."""
    return _FlashLowp.apply(q, k, v, bool(causal), int(window or 0), scale)


def _round(t, dtype):
    return t.to(dtype).to(t.dtype)


class _FlashLowp(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, causal, window, scale):
        dt = q.dtype
        acc = torch.float64 if dt == torch.float64 else torch.float32
        B, Sq, Hq, d = q.shape
        Hkv = k.shape[2]
        sc = 1.0 / math.sqrt(d) if scale is None else scale
        kk = repeat_kv(k, Hq // Hkv).transpose(1, 2).to(acc)
        vv = repeat_kv(v, Hq // Hkv).transpose(1, 2).to(acc)
        qq = q.transpose(1, 2).to(acc)
        s = torch.matmul(qq, kk.transpose(-1, -2).contiguous()) * sc
        vis = attn_mask(Sq, k.shape[1], causal, window, q.device)
        s = s.masked_fill(~vis, float("-inf"))
        m = s.amax(-1, keepdim=True)
        m = torch.where(torch.isfinite(m), m, torch.zeros_like(m))
        p = torch.exp(s - m)
        lsum = p.sum(-1, keepdim=True)
        o = torch.matmul(_round(p, dt), vv) / torch.where(lsum > 0, lsum, torch.ones_like(lsum))
        lse = (m + torch.log(lsum)).squeeze(-1)
        out = o.transpose(1, 2).to(dt)
        ctx.save_for_backward(q, k, v, out, lse)
        ctx.cfg = (causal, window, sc)
        return out

    @staticmethod
    def backward(ctx, do):
        q, k, v, out, lse = ctx.saved_tensors
        causal, window, sc = ctx.cfg
        dt = q.dtype
        acc = torch.float64 if dt == torch.float64 else torch.float32
        B, Sq, Hq, d = q.shape
        Skv, Hkv = k.shape[1], k.shape[2]
        n_rep = Hq // Hkv
        kk = repeat_kv(k, n_rep).transpose(1, 2).to(acc)
        vv = repeat_kv(v, n_rep).transpose(1, 2).to(acc)
        qq = q.transpose(1, 2).to(acc)
        dd = do.to(dt).transpose(1, 2).to(acc)
        s = torch.matmul(qq, kk.transpose(-1, -2).contiguous()) * sc
        vis = attn_mask(Sq, Skv, causal, window, q.device)
        p = torch.exp(s - lse[..., None]).masked_fill(~vis, 0.0)
        del s
        dv = torch.matmul(_round(p, dt).transpose(-1, -2).contiguous(), dd)
        dp = torch.matmul(dd, vv.transpose(-1, -2).contiguous())
        delta = (dd * out.transpose(1, 2).to(acc)).sum(-1, keepdim=True)
        ds = _round(p * (dp - delta), dt)
        del p, dp
        dq = (torch.matmul(ds, kk) * sc).transpose(1, 2).to(dt)
        dk = torch.matmul(ds.transpose(-1, -2).contiguous(), qq) * sc
        # per-query-head gradients in the storage dtype, then the group sum
        dk = dk.to(dt).to(acc).view(B, Hkv, n_rep, Skv, d).sum(2).transpose(1, 2).to(dt)
        dv = dv.to(dt).to(acc).view(B, Hkv, n_rep, Skv, d).sum(2).transpose(1, 2).to(dt)
        return dq, dk, dv, None, None, None


# -------------------------------------------------------------------- MLP --

def silu(x: torch.Tensor) -> torch.Tensor:
    """ACT2FN["silu"] of HF LlamaMLP (nn.SiLU): x * sigmoid(x), one rounding
    in a 16-bit dtype."""
    return F.silu(x)


def swiglu(g: torch.Tensor, u: torch.Tensor) -> torch.Tensor:
    """act_fn(gate(x)) * up(x) of HF LlamaMLP.forward (built at
    models/llama_simple.py:418; torchtitan FeedForward, models/llama_v2.py:
    319-320)."""
    return silu(g) * u


def swiglu_bwd(dz, g, u):
    """dz -> (dg, du): du = dz silu(g); dg = dz u sigma(g)(1 + g(1 - sigma(g)))."""
    sg = torch.sigmoid(g)
    return dz * u * sg * (1 + g * (1 - sg)), dz * g * sg


def mlp(x, wg, wu, wd):
    """HF LlamaMLP.forward: down(silu(gate(x)) * up(x)), no biases."""
    return F.linear(swiglu(F.linear(x, wg), F.linear(x, wu)), wd)


# ------------------------------------------------------------------ layer --

def decoder_layer(x: torch.Tensor, p: dict[str, torch.Tensor], s: LayerShape,
                  rope: str = "half", positions: torch.Tensor | None = None,
                  attn: str = "eager") -> torch.Tensor:
    """LlamaDecoderLayer.forward (models/llama_simple.py:456-479):
        h   = x + o_proj(Attn(RoPE(q_proj(n1)), RoPE(k_proj(n1)), v_proj(n1)))
        out = h + down(silu(gate(n2)) * up(n2)),   n1 = RMSNorm1(x), n2 = RMSNorm2(h)
    with the attention of a-7 (causal, optional sliding window, GQA).  The
    Mistral layer (HF MistralDecoderLayer via models/mistral_simple.py:13-41)
    is the same composition.  rope="interleaved" uses the llama_v2 pairing
    (models/llama_v2.py:151-177, TransformerBlock :328-399).  attn="flash"
    takes the attention through flash_attention_lowp (the flash kernels'
    rounding points; the same value in fp32 / fp64).  ``positions``: int64
    [S] token positions for RoPE (default 0 .. S-1)."""
    B, S, h = x.shape
    T = B * S
    n1 = rmsnorm(x, p["ln1"], s.eps).reshape(T, h)
    q = F.linear(n1, p["q"]).view(B, S, s.heads, s.head_dim)
    k = F.linear(n1, p["k"]).view(B, S, s.kv_heads, s.head_dim)
    v = F.linear(n1, p["v"]).view(B, S, s.kv_heads, s.head_dim)
    if rope == "half":
        cos, sin = rope_cos_sin(S, s.head_dim, s.theta, x.dtype,
                                None if positions is None else positions.cpu())
        q, k = apply_rope_half(q, k, cos.to(x.device), sin.to(x.device))
    else:
        q, k = apply_rope_interleaved(q, k, rope_freqs_cis(s.head_dim, S, s.theta).to(x.device))
    if attn == "flash":
        a = flash_attention_lowp(q, k, v, s.causal, s.window)
    else:
        a, _ = attention(q, k, v, s.causal, s.window)
    hdn = x + F.linear(a.reshape(T, s.heads * s.head_dim), p["o"]).view(B, S, h)
    n2 = rmsnorm(hdn, p["ln2"], s.eps).reshape(T, h)
    return hdn + mlp(n2, p["gate"], p["up"], p["down"]).view(B, S, h)


def layer_fwd_bwd(x, p, s: LayerShape, dout, rope: str = "half", attn: str = "eager",
                  positions: torch.Tensor | None = None):
    """Output, input gradient and parameter gradients of decoder_layer via
    autograd (the reference's backward is torch autograd over the same graph,
    models/llama_simple.py:456-479).  Returns (out, dx, {name: grad}).

    With x, p and dout in bf16 / fp16 and attn="flash" this is the layer as
    plain PyTorch computes it at that precision -- the reference's own bf16 /
    fp16 layer up to GEMM summation order: every op rounds to the storage
    dtype where the reference's does (RMSNorm's fp32 upcast, bf16 RoPE
    tables, nn.SiLU, the residual adds) and attention has the flash kernels'
    rounding points."""
    xr = x.detach().clone().requires_grad_(True)
    pr = {k: t.detach().clone().requires_grad_(True) for k, t in p.items()}
    out = decoder_layer(xr, pr, s, rope, positions=positions, attn=attn)
    out.backward(dout)
    return out.detach(), xr.grad, {k: t.grad for k, t in pr.items()}


def lm_head_ce(x, norm_w, head_w, labels, eps):
    """Last-stage output layer + loss: Sequential(norm, lm_head)
    (models/llama_simple.py:559-561) and F.cross_entropy over flattened tokens
    (zorse_utils/pipeline_schedule_v2.py:181-184)."""
    logits = F.linear(rmsnorm(x, norm_w, eps), head_w)
    return F.cross_entropy(logits.flatten(0, 1).to(torch.float64 if x.dtype == torch.float64
                                                   else torch.float32),
                           labels.flatten(0, 1))


# ------------------------------------------------------------------ AdamW --

def adamw_step(p, g, m, v, step, lr, beta1, beta2, eps, weight_decay):
    """One AdamW step, in place, in the dtype of p (torch.optim.AdamW's
    documented algorithm, Loshchilov & Hutter): decoupled decay
    p <- p (1 - lr wd); m <- b1 m + (1-b1) g; v <- b2 v + (1-b2) g^2;
    p <- p - lr/(1-b1^t) * m / (sqrt(v)/sqrt(1-b2^t) + eps).
    weight_decay 0 is torch.optim.Adam, the reference's optimizer
    (zorse_utils/pipeline.py:176-179) applied to the flat shard in the
    reduce-grad callback with the grad cast to the param dtype
    (utils/patch.py:115-138)."""
    g = g.to(p.dtype)
    p.mul_(1 - lr * weight_decay)
    m.lerp_(g, 1 - beta1)
    v.mul_(beta2).addcmul_(g, g, value=1 - beta2)
    bc1 = 1 - beta1 ** step
    bc2 = 1 - beta2 ** step
    denom = v.sqrt() / math.sqrt(bc2) + eps
    p.addcdiv_(m, denom, value=-lr / bc1)
    return p, m, v


def adamw_step_scalar(p: list[float], g: list[float], m: list[float], v: list[float],
                      step, lr, beta1, beta2, eps, weight_decay):
    """Element-by-element restatement of adamw_step in Python floats (fp64),
    for brute-force checks on tiny shards."""
    bc1 = 1 - beta1 ** step
    bc2 = 1 - beta2 ** step
    for i in range(len(p)):
        p[i] *= 1 - lr * weight_decay
        m[i] = beta1 * m[i] + (1 - beta1) * g[i]
        v[i] = beta2 * v[i] + (1 - beta2) * g[i] * g[i]
        p[i] -= (lr / bc1) * m[i] / (math.sqrt(v[i]) / math.sqrt(bc2) + eps)
    return p, m, v
