"""Algorithmic work of the hot path -- the single definition the benchmark's
throughput and roofline figures use.

* Attention: fwd = 4 B Hq d P, with P the number of visible (query, key)
  pairs per (batch, head): causal S(S+1)/2, sliding window sum_i min(i+1, W);
  bwd = 2.5 x fwd (the five d-length contractions of the backward vs two).
* Projections: fwd = 2 T N_lin, bwd = 4 T N_lin, with
  N_lin = h Hq d + 2 h Hkv d + Hq d h + 3 h F (T = B S tokens).
* RMSNorm bytes: fwd 2 T h e + 4 h + 4 T (read x, write y, weight, rstd);
  bwd 3 T h e + 4 T + 4 h (read dy, x, write dx).
* AdamW bytes per element: read p, g, m, v and write p, m, v:
  12 + g_bytes + 12 (+ 2 for a low-precision copy of p).
"""
from __future__ import annotations


def visible_pairs(sq: int, skv: int, causal: bool, window: int) -> int:
    if not causal and not window:
        return sq * skv
    if not window:
        n = min(sq, skv)
        return n * (n + 1) // 2
    w = window
    full = max(0, sq - w)          # rows with W visible keys
    head = min(sq, w)              # rows 0..W-1 see i+1 keys
    return head * (head + 1) // 2 + full * w


def attn_fwd_flops(B, Hq, d, sq, skv, causal=True, window=0) -> float:
    return 4.0 * B * Hq * d * visible_pairs(sq, skv, causal, window)


def attn_bwd_flops(B, Hq, d, sq, skv, causal=True, window=0) -> float:
    return 2.5 * attn_fwd_flops(B, Hq, d, sq, skv, causal, window)


def n_lin(spec) -> int:
    h = spec.hidden
    return (h * spec.heads * spec.head_dim + 2 * h * spec.kv_heads * spec.head_dim
            + spec.heads * spec.head_dim * h + 3 * h * spec.ffn)


def gemm_fwd_flops(spec, B, S) -> float:
    return 2.0 * B * S * n_lin(spec)


def layer_fwd_flops(spec, B, S) -> float:
    return gemm_fwd_flops(spec, B, S) + attn_fwd_flops(B, spec.heads, spec.head_dim, S, S,
                                                       spec.causal, spec.window)


def layer_fwd_bwd_flops(spec, B, S) -> float:
    attn = attn_fwd_flops(B, spec.heads, spec.head_dim, S, S, spec.causal, spec.window)
    return 3.0 * gemm_fwd_flops(spec, B, S) + 3.5 * attn


def rmsnorm_fwd_bytes(T, h, e=2) -> int:
    return 2 * T * h * e + 4 * h + 4 * T


def rmsnorm_bwd_bytes(T, h, e=2) -> int:
    return 3 * T * h * e + 4 * T + 4 * h


def adamw_bytes(n, grad_bytes=4, lowp_copy=False) -> int:
    return n * (24 + grad_bytes + (2 if lowp_copy else 0))


def attn_fwd_bytes(B, S, Hq, Hkv, d, e=2) -> int:
    """Compulsory HBM bytes of the attention forward: read Q, K, V, write O
    (storage type, e bytes) and the fp32 LSE."""
    return e * B * S * d * (2 * Hq + 2 * Hkv) + 4 * B * Hq * S


def attn_bwd_bytes(B, S, Hq, Hkv, d, e=2) -> int:
    """Compulsory HBM bytes of the attention backward: read Q, K, V, O, dO and
    the LSE, write dQ, dK, dV, plus the fp32 delta / log2-LSE workspace
    (written once, read by both gradient kernels)."""
    return e * B * S * d * (3 * Hq + 2 * Hkv) + e * B * S * d * (Hq + 2 * Hkv) \
        + 4 * B * Hq * S + 2 * 3 * 4 * B * Hq * S
