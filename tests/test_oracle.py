"""Pins the CPU oracle (oracle/decoder.py) before anything is compared to it.

Each check is chosen so that a plausible slip in the oracle -- a dropped
term, a wrong sign or index, a transposed operand, the wrong RoPE pairing, an
off-by-one window -- fails at least one of them:
  * the golden fixtures written by the transformers modules the reference
    composes its layer from (tests/golden/make_golden.py);
  * library routines (HF LlamaRMSNorm / LlamaMLP / rotary embedding, torch
    SDPA, torch.optim.AdamW / Adam);
  * closed forms, invariants and brute force on tiny inputs.
"""
import math
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import decoder as O

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
torch.set_num_threads(min(8, os.cpu_count() or 1))


def _load(name):
    z = np.load(os.path.join(GOLDEN, name + ".npz"))
    hidden, heads, kv, hd, ffn, B, S, theta, window, seed = z["meta"]
    shape = O.LayerShape(hidden=int(hidden), heads=int(heads), kv_heads=int(kv),
                         head_dim=int(hd), ffn=int(ffn), theta=float(theta),
                         window=int(window))
    t = {k: torch.from_numpy(z[k]).double() for k in z.files if k != "meta"}
    return shape, t


# ------------------------------------------------------------ golden layer --

@pytest.mark.parametrize("name", ["llama_gqa_d16", "llama_mha_d64", "mistral_swa_d64"])
def test_oracle_layer_matches_transformers_golden(name):
    shape, t = _load(name)
    p = {k: t["w_" + k] for k in O.PARAM_ORDER}
    out, dx, grads = O.layer_fwd_bwd(t["x"], p, shape, t["dout"])
    # fixtures are stored in fp32: compare at fp32 storage precision
    assert torch.allclose(out, t["out"], rtol=1e-5, atol=1e-5)
    assert torch.allclose(dx, t["dx"], rtol=1e-5, atol=1e-5)
    for k in O.PARAM_ORDER:
        ref = t["g_" + k]
        assert torch.allclose(grads[k], ref, rtol=1e-5, atol=1e-5 * ref.abs().max().item()), k


def test_golden_window_is_active():
    """The Mistral fixture's window (16) is shorter than its sequence (40):
    the non-windowed oracle must disagree with it."""
    shape, t = _load("mistral_swa_d64")
    assert shape.window < t["x"].shape[1]
    p = {k: t["w_" + k] for k in O.PARAM_ORDER}
    causal_only = O.LayerShape(**{**shape.__dict__, "window": 0})
    out = O.decoder_layer(t["x"], p, causal_only)
    assert not torch.allclose(out, t["out"], atol=1e-3)


# ---------------------------------------------------------------- RMSNorm --

def test_rmsnorm_matches_hf():
    from transformers.models.llama.modeling_llama import LlamaRMSNorm
    g = torch.Generator().manual_seed(0)
    m = LlamaRMSNorm(96, eps=1e-6)
    with torch.no_grad():
        m.weight.copy_(torch.randn(96, generator=g))
    for dt in (torch.float32, torch.bfloat16, torch.float16):
        x = torch.randn(5, 7, 96, generator=g).to(dt)
        ref = m.to(dt)(x)
        got = O.rmsnorm(x, m.weight, 1e-6)
        assert got.dtype == ref.dtype
        assert torch.equal(got, ref)


def test_rmsnorm_invariants():
    g = torch.Generator().manual_seed(1)
    x = torch.randn(9, 64, generator=g, dtype=torch.float64)
    y = O.rmsnorm(x, torch.ones(64, dtype=torch.float64), 0.0)
    assert torch.allclose(y.pow(2).mean(-1), torch.ones(9, dtype=torch.float64))
    y2 = O.rmsnorm(7.5 * x, torch.ones(64, dtype=torch.float64), 0.0)
    assert torch.allclose(y, y2)


def test_rmsnorm_bwd_closed_form_vs_autograd():
    g = torch.Generator().manual_seed(2)
    x = torch.randn(6, 48, generator=g, dtype=torch.float64, requires_grad=True)
    w = torch.randn(48, generator=g, dtype=torch.float64, requires_grad=True)
    dy = torch.randn(6, 48, generator=g, dtype=torch.float64)
    O.rmsnorm(x, w, 1e-6).backward(dy)
    dx, dw = O.rmsnorm_bwd(dy, x.detach(), w.detach(), 1e-6)
    assert torch.allclose(dx, x.grad) and torch.allclose(dw, w.grad)


def test_rmsnorm_rstd_matches_hf_variance_and_closed_forms():
    """rmsnorm_rstd is the factor HF LlamaRMSNorm multiplies by: with a unit
    weight in fp64 the module's output divided by its input is rstd in every
    element; a constant row c gives 1 / sqrt(c^2 + eps); a one-hot row gives
    1 / sqrt(1 / h + eps); and mean((x rstd)^2) = m / (m + eps) with
    m = mean(x^2).  A slip to sum, to sqrt, or a dropped eps fails."""
    from transformers.models.llama.modeling_llama import LlamaRMSNorm
    g = torch.Generator().manual_seed(21)
    h, eps = 40, 1e-2
    m = LlamaRMSNorm(h, eps=eps).double()
    x = torch.randn(6, h, generator=g, dtype=torch.float64)
    r = O.rmsnorm_rstd(x, eps)
    assert r.shape == (6,) and r.dtype == torch.float64
    # (HF upcasts to fp32 internally, hence fp32-level agreement)
    assert torch.allclose(m(x) / x, r[:, None].expand(6, h), rtol=1e-6, atol=0)
    c = torch.full((1, h), 0.3, dtype=torch.float64)
    assert math.isclose(O.rmsnorm_rstd(c, eps).item(), 1 / math.sqrt(0.09 + eps), rel_tol=1e-14)
    e = torch.zeros(1, h, dtype=torch.float64)
    e[0, 7] = 1.0
    assert math.isclose(O.rmsnorm_rstd(e, eps).item(), 1 / math.sqrt(1 / h + eps), rel_tol=1e-14)
    ms = x.pow(2).mean(-1)
    assert torch.allclose((x * r[:, None]).pow(2).mean(-1), ms / (ms + eps), rtol=1e-13)
    # fp32 / bf16 input: fp32 result from the fp32-upcast variance (HF's order)
    xb = x.to(torch.bfloat16)
    rb = O.rmsnorm_rstd(xb, eps)
    assert rb.dtype == torch.float32
    assert torch.equal(rb, torch.rsqrt(xb.float().pow(2).mean(-1) + eps))


# ------------------------------------------------------------------- RoPE --

def test_rope_matches_hf():
    from transformers import LlamaConfig
    from transformers.models.llama.modeling_llama import (LlamaRotaryEmbedding,
                                                          apply_rotary_pos_emb)
    for d, theta in ((64, 1e4), (128, 5e5), (128, 1e6)):
        cfg = LlamaConfig(hidden_size=4 * d, num_attention_heads=4, head_dim=d,
                          rope_theta=theta, max_position_embeddings=64)
        rope = LlamaRotaryEmbedding(cfg)
        g = torch.Generator().manual_seed(d)
        for dt in (torch.float32, torch.bfloat16):
            q = torch.randn(2, 4, 33, d, generator=g).to(dt)   # BHSD for HF
            k = torch.randn(2, 2, 33, d, generator=g).to(dt)
            pos = torch.arange(33)[None].expand(2, 33)
            cos, sin = rope(q, pos)
            rq, rk = apply_rotary_pos_emb(q, k, cos, sin)
            c2, s2 = O.rope_cos_sin(33, d, theta, dt)
            assert torch.equal(c2, cos[0]) and torch.equal(s2, sin[0])
            oq, ok = O.apply_rope_half(q.transpose(1, 2), k.transpose(1, 2), c2, s2)
            assert torch.equal(oq.transpose(1, 2), rq) and torch.equal(ok.transpose(1, 2), rk)


def test_rope_invariants():
    g = torch.Generator().manual_seed(3)
    d, S = 64, 40
    cos, sin = O.rope_cos_sin(S, d, 1e4, torch.float64)
    q = torch.randn(1, S, 1, d, generator=g, dtype=torch.float64)
    k = torch.randn(1, S, 1, d, generator=g, dtype=torch.float64)
    rq, rk = O.apply_rope_half(q, k, cos, sin)
    # per-pair (i, i + d/2) norms preserved
    pn = lambda t: t[..., : d // 2] ** 2 + t[..., d // 2:] ** 2  # noqa: E731
    assert torch.allclose(pn(rq), pn(q))
    # <R_m q, R_n k> depends only on m - n: rotate the same q, k at shifted positions
    q0 = q[:, :1].expand(1, S, 1, d)
    k0 = k[:, :1].expand(1, S, 1, d)
    rq0, rk0 = O.apply_rope_half(q0, k0, cos, sin)
    dots = torch.einsum("bshd,bthd->st", rq0, rk0)
    for off in (0, 3, -5):
        diag = torch.diagonal(dots, off)
        assert torch.allclose(diag, diag[0].expand_as(diag))
    # pairing matters: the interleaved form differs from the half-split one
    iq, _ = O.apply_rope_interleaved(q, k, O.rope_freqs_cis(d, S, 1e4))
    assert not torch.allclose(iq, rq)
    assert torch.allclose(pn(rq), pn(q))


def test_rope_interleaved_is_complex_rotation():
    g = torch.Generator().manual_seed(4)
    d, S = 16, 9
    q = torch.randn(1, S, 2, d, generator=g, dtype=torch.float64)
    fc = O.rope_freqs_cis(d, S, 1e4)
    rq, _ = O.apply_rope_interleaved(q, q, fc)
    for s in range(S):
        for i in range(d // 2):
            ang = s * (1e4 ** (-(2 * i) / d))
            a, b = q[0, s, 0, 2 * i].item(), q[0, s, 0, 2 * i + 1].item()
            assert math.isclose(rq[0, s, 0, 2 * i].item(), a * math.cos(ang) - b * math.sin(ang),
                                abs_tol=1e-6)
            assert math.isclose(rq[0, s, 0, 2 * i + 1].item(),
                                a * math.sin(ang) + b * math.cos(ang), abs_tol=1e-6)


# -------------------------------------------------------------- attention --

def test_attention_matches_sdpa_causal_gqa():
    g = torch.Generator().manual_seed(5)
    B, S, Hq, Hkv, d = 2, 37, 4, 2, 32
    q = torch.randn(B, S, Hq, d, generator=g, dtype=torch.float64)
    k = torch.randn(B, S, Hkv, d, generator=g, dtype=torch.float64)
    v = torch.randn(B, S, Hkv, d, generator=g, dtype=torch.float64)
    out, lse = O.attention(q, k, v, causal=True)
    ref = F.scaled_dot_product_attention(
        q.transpose(1, 2), O.repeat_kv(k, 2).transpose(1, 2), O.repeat_kv(v, 2).transpose(1, 2),
        is_causal=True).transpose(1, 2)
    assert torch.allclose(out, ref, atol=1e-10)
    # GQA == explicitly expanded MHA
    out2, _ = O.attention(q, O.repeat_kv(k, 2), O.repeat_kv(v, 2), causal=True)
    assert torch.allclose(out, out2, atol=1e-12)
    assert lse.shape == (B, Hq, S)


def test_attention_brute_force_window():
    g = torch.Generator().manual_seed(6)
    S, d, W = 12, 8, 4
    q = torch.randn(1, S, 1, d, generator=g, dtype=torch.float64)
    k = torch.randn(1, S, 1, d, generator=g, dtype=torch.float64)
    v = torch.randn(1, S, 1, d, generator=g, dtype=torch.float64)
    out, lse = O.attention(q, k, v, causal=True, window=W)
    for i in range(S):
        js = [j for j in range(S) if i - W < j <= i]
        assert len(js) == min(i + 1, W)
        sc = [sum(q[0, i, 0, e].item() * k[0, j, 0, e].item() for e in range(d)) / math.sqrt(d)
              for j in js]
        m = max(sc)
        ws = [math.exp(s - m) for s in sc]
        z = sum(ws)
        assert math.isclose(lse[0, 0, i].item(), m + math.log(z), rel_tol=1e-12)
        for e in range(d):
            ref = sum(w * v[0, j, 0, e].item() for w, j in zip(ws, js)) / z
            assert math.isclose(out[0, i, 0, e].item(), ref, abs_tol=1e-12)


def test_attention_ignores_future_and_out_of_window_keys():
    g = torch.Generator().manual_seed(7)
    S, d, W = 20, 16, 5
    q = torch.randn(1, S, 2, d, generator=g, dtype=torch.float64)
    k = torch.randn(1, S, 2, d, generator=g, dtype=torch.float64)
    v = torch.randn(1, S, 2, d, generator=g, dtype=torch.float64)
    out, _ = O.attention(q, k, v, causal=True, window=W)
    i = 11
    k2, v2 = k.clone(), v.clone()
    k2[:, i + 1:] += 5.0
    v2[:, : i - W + 1] -= 3.0
    out2, _ = O.attention(q, k2, v2, causal=True, window=W)
    assert torch.allclose(out[:, i], out2[:, i])
    assert not torch.allclose(out[:, i + 1:], out2[:, i + 1:])


def test_attention_mask_matches_transformers_mask_functions():
    from transformers.masking_utils import (causal_mask_function,
                                            sliding_window_causal_mask_function)
    qi = torch.arange(30)[:, None]
    kj = torch.arange(30)[None, :]
    assert torch.equal(O.attn_mask(30, 30, True, 0), causal_mask_function(0, 0, qi, kj))
    for W in (1, 7, 29, 64):
        assert torch.equal(O.attn_mask(30, 30, True, W),
                           sliding_window_causal_mask_function(W)(0, 0, qi, kj))


def test_attention_bwd_closed_form_vs_autograd():
    g = torch.Generator().manual_seed(8)
    B, S, Hq, Hkv, d = 1, 19, 4, 1, 8
    q = torch.randn(B, S, Hq, d, generator=g, dtype=torch.float64, requires_grad=True)
    k = torch.randn(B, S, Hkv, d, generator=g, dtype=torch.float64, requires_grad=True)
    v = torch.randn(B, S, Hkv, d, generator=g, dtype=torch.float64, requires_grad=True)
    do = torch.randn(B, S, Hq, d, generator=g, dtype=torch.float64)
    for W in (0, 6):
        for t in (q, k, v):
            t.grad = None
        out, _ = O.attention(q, k, v, causal=True, window=W)
        out.backward(do)
        dq, dk, dv = O.attention_bwd(q.detach(), k.detach(), v.detach(), do, causal=True,
                                     window=W)
        assert torch.allclose(dq, q.grad) and torch.allclose(dk, k.grad)
        assert torch.allclose(dv, v.grad)


def test_attention_rows_sum_to_one():
    g = torch.Generator().manual_seed(9)
    q = torch.randn(1, 10, 1, 4, generator=g, dtype=torch.float64)
    k = torch.randn(1, 10, 1, 4, generator=g, dtype=torch.float64)
    ones = torch.ones(1, 10, 1, 4, dtype=torch.float64)
    out, _ = O.attention(q, k, ones, causal=True, window=3)
    assert torch.allclose(out, ones)


def test_flash_attention_lowp_is_attention_without_rounding():
    """In fp64 (no storage rounding) the flash-rounding attention is the eager
    attention, forward and closed-form backward (GQA 4:1, causal, window):
    this pins its indexing, scale, mask, LSE use and the GQA group sum."""
    g = torch.Generator().manual_seed(22)
    B, S, Hq, Hkv, d = 2, 23, 4, 1, 8
    q = torch.randn(B, S, Hq, d, generator=g, dtype=torch.float64, requires_grad=True)
    k = torch.randn(B, S, Hkv, d, generator=g, dtype=torch.float64, requires_grad=True)
    v = torch.randn(B, S, Hkv, d, generator=g, dtype=torch.float64, requires_grad=True)
    do = torch.randn(B, S, Hq, d, generator=g, dtype=torch.float64)
    for W in (0, 5):
        for t in (q, k, v):
            t.grad = None
        out = O.flash_attention_lowp(q, k, v, causal=True, window=W)
        ref, _ = O.attention(q.detach(), k.detach(), v.detach(), causal=True, window=W)
        assert torch.allclose(out, ref, atol=1e-13)
        out.backward(do)
        dq, dk, dv = O.attention_bwd(q.detach(), k.detach(), v.detach(), do, causal=True,
                                     window=W)
        assert torch.allclose(q.grad, dq, atol=1e-12)
        assert torch.allclose(k.grad, dk, atol=1e-12)
        assert torch.allclose(v.grad, dv, atol=1e-12)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_flash_attention_lowp_error_matches_sdpa(dtype):
    """At 16-bit storage the flash-rounding attention is as accurate as torch's
    own SDPA in that dtype (CPU flash kernel: fp32 softmax, 16-bit P): output
    and gradient errors against fp64 within a factor 2 of SDPA's, and the
    16-bit rounding is really applied (errors far above fp32's)."""
    g = torch.Generator().manual_seed(23)
    B, S, H, d = 1, 96, 2, 64
    q64 = torch.randn(B, S, H, d, generator=g, dtype=torch.float64)
    k64 = torch.randn(B, S, H, d, generator=g, dtype=torch.float64)
    v64 = torch.randn(B, S, H, d, generator=g, dtype=torch.float64)
    do64 = torch.randn(B, S, H, d, generator=g, dtype=torch.float64)
    q, k, v, do = (t.to(dtype) for t in (q64, k64, v64, do64))
    # the fp64 truth on the rounded inputs
    refs = [t.double().requires_grad_(True) for t in (q, k, v)]
    ro, _ = O.attention(*refs, causal=True)
    ro.backward(do.double())
    mine = [t.clone().requires_grad_(True) for t in (q, k, v)]
    mo = O.flash_attention_lowp(*mine, causal=True)
    mo.backward(do)
    lib = [t.clone().transpose(1, 2).requires_grad_(True) for t in (q, k, v)]
    lo = F.scaled_dot_product_attention(*lib, is_causal=True)
    lo.backward(do.transpose(1, 2))
    lo = lo.transpose(1, 2)

    def e(a, b):
        return (a.double() - b.double()).abs().max().item()

    pairs = [("o", mo, lo, ro)] + [(n, a.grad, b.grad.transpose(1, 2), c.grad)
                                   for n, a, b, c in zip("qkv", mine, lib, refs)]
    for name, got, sdpa, ref in pairs:
        em, es = e(got, ref), e(sdpa, ref)
        assert em <= 2.0 * es, (name, em, es)
        assert em > 1e-5 * ref.abs().max().item(), (name, em)


def test_layer_flash_path_is_the_eager_layer_in_fp64():
    """layer_fwd_bwd(attn="flash") and the eager composition agree in fp64
    (output, dx and all nine weight gradients), on the Mistral golden shape."""
    shape, t = _load("mistral_swa_d64")
    p = {k: t["w_" + k] for k in O.PARAM_ORDER}
    a = O.layer_fwd_bwd(t["x"], p, shape, t["dout"])
    b = O.layer_fwd_bwd(t["x"], p, shape, t["dout"], attn="flash")
    assert torch.allclose(a[0], b[0], atol=1e-12) and torch.allclose(a[1], b[1], atol=1e-12)
    for k in O.PARAM_ORDER:
        assert torch.allclose(a[2][k], b[2][k], atol=1e-12), k


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_layer_lowp_is_transformers_layer_precision(dtype):
    """The compute-precision layer (attn="flash" on 16-bit tensors) is as
    accurate as transformers' own LlamaDecoderLayer run in that dtype with SDPA
    attention (the reference's non-flash-attn path): every output / gradient
    error against fp64 within a factor 2 (+1 ulp) of the transformers layer's."""
    from transformers import LlamaConfig
    from transformers.models.llama.modeling_llama import LlamaDecoderLayer, LlamaRotaryEmbedding
    hidden, heads, kv, hd, ffn, S = 128, 4, 2, 32, 256, 80
    cfg = LlamaConfig(hidden_size=hidden, num_attention_heads=heads, num_key_value_heads=kv,
                      head_dim=hd, intermediate_size=ffn, rms_norm_eps=1e-6,
                      max_position_embeddings=S, rope_theta=1e4, attention_dropout=0.0)
    cfg._attn_implementation = "sdpa"
    layer = LlamaDecoderLayer(cfg, 0)
    g = torch.Generator().manual_seed(24)
    names = {"q": layer.self_attn.q_proj.weight, "k": layer.self_attn.k_proj.weight,
             "v": layer.self_attn.v_proj.weight, "o": layer.self_attn.o_proj.weight,
             "gate": layer.mlp.gate_proj.weight, "up": layer.mlp.up_proj.weight,
             "down": layer.mlp.down_proj.weight, "ln1": layer.input_layernorm.weight,
             "ln2": layer.post_attention_layernorm.weight}
    with torch.no_grad():
        for k_, w in names.items():
            w.copy_(1 + 0.1 * torch.randn(w.shape, generator=g) if k_.startswith("ln")
                    else 0.05 * torch.randn(w.shape, generator=g))
    layer = layer.to(dtype)
    x = torch.randn(1, S, hidden, generator=g).to(dtype)
    dout = torch.randn(1, S, hidden, generator=g).to(dtype)
    rope = LlamaRotaryEmbedding(cfg)
    pos = torch.arange(S)[None]
    xr = x.clone().requires_grad_(True)
    cos, sin = rope(xr, pos)
    hf_out = layer(xr, attention_mask=None, position_ids=pos,
                   position_embeddings=(cos.to(dtype), sin.to(dtype)))
    hf_out = hf_out[0] if isinstance(hf_out, tuple) else hf_out
    hf_out.backward(dout)
    p = {k_: w.detach() for k_, w in names.items()}
    shape = O.LayerShape(hidden=hidden, heads=heads, kv_heads=kv, head_dim=hd, ffn=ffn)
    ref = O.layer_fwd_bwd(x.double(), {k_: w.double() for k_, w in p.items()}, shape,
                          dout.double())
    low = O.layer_fwd_bwd(x, p, shape, dout, attn="flash")
    ulp = {torch.bfloat16: 2.0 ** -7, torch.float16: 2.0 ** -10}[dtype]
    cases = [("out", low[0], hf_out, ref[0]), ("dx", low[1], xr.grad, ref[1])]
    cases += [("d" + k_, low[2][k_], names[k_].grad, ref[2][k_]) for k_ in O.PARAM_ORDER]
    for name, mine, hf, r in cases:
        em = (mine.double() - r).abs().max().item()
        eh = (hf.double() - r).abs().max().item()
        floor = ulp * 2.0 ** math.floor(math.log2(r.abs().max().item()))
        assert em <= 2.0 * eh + floor, (name, em, eh)


# -------------------------------------------------------------------- MLP --

def test_mlp_matches_hf_and_closed_form_bwd():
    from transformers import LlamaConfig
    from transformers.models.llama.modeling_llama import LlamaMLP
    cfg = LlamaConfig(hidden_size=24, intermediate_size=40, num_attention_heads=4)
    m = LlamaMLP(cfg).double()
    g = torch.Generator().manual_seed(10)
    x = torch.randn(3, 24, generator=g, dtype=torch.float64)
    ref = m(x)
    got = O.mlp(x, m.gate_proj.weight, m.up_proj.weight, m.down_proj.weight)
    assert torch.allclose(got, ref, atol=1e-12)
    gg = torch.randn(5, 7, generator=g, dtype=torch.float64, requires_grad=True)
    uu = torch.randn(5, 7, generator=g, dtype=torch.float64, requires_grad=True)
    dz = torch.randn(5, 7, generator=g, dtype=torch.float64)
    O.swiglu(gg, uu).backward(dz)
    dg, du = O.swiglu_bwd(dz, gg.detach(), uu.detach())
    assert torch.allclose(dg, gg.grad) and torch.allclose(du, uu.grad)


# ------------------------------------------------------------------ AdamW --

def test_adamw_matches_torch_multi_step():
    g = torch.Generator().manual_seed(11)
    n = 1000
    p0 = torch.randn(n, generator=g)
    grads = [torch.randn(n, generator=g) for _ in range(5)]
    for wd in (0.0, 0.1):
        ref = p0.clone().requires_grad_(True)
        opt = torch.optim.AdamW([ref], lr=1e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=wd,
                                foreach=False)
        p, m, v = p0.clone(), torch.zeros(n), torch.zeros(n)
        for t, gr in enumerate(grads, 1):
            ref.grad = gr.clone()
            opt.step()
            O.adamw_step(p, gr, m, v, t, 1e-3, 0.9, 0.95, 1e-8, wd)
        assert torch.allclose(p, ref.detach(), rtol=0, atol=1e-6)


def test_adamw_wd0_is_torch_adam():
    g = torch.Generator().manual_seed(12)
    p0 = torch.randn(300, generator=g, dtype=torch.float64)
    ref = p0.clone().requires_grad_(True)
    opt = torch.optim.Adam([ref], foreach=False)   # the reference's optimizer, defaults
    p, m, v = p0.clone(), torch.zeros_like(p0), torch.zeros_like(p0)
    for t in range(1, 4):
        gr = torch.randn(300, generator=g, dtype=torch.float64)
        ref.grad = gr.clone()
        opt.step()
        O.adamw_step(p, gr, m, v, t, 1e-3, 0.9, 0.999, 1e-8, 0.0)
    assert torch.allclose(p, ref.detach(), rtol=0, atol=1e-12)


def test_adamw_first_step_closed_form_and_scalar_loop():
    g = torch.Generator().manual_seed(13)
    p0 = torch.randn(50, generator=g, dtype=torch.float64)
    gr = torch.randn(50, generator=g, dtype=torch.float64)
    lr, wd, eps = 1e-2, 0.1, 1e-8
    p = p0.clone()
    O.adamw_step(p, gr, torch.zeros(50, dtype=torch.float64), torch.zeros(50, dtype=torch.float64),
                 1, lr, 0.9, 0.95, eps, wd)
    closed = p0 * (1 - lr * wd) - lr * gr / (gr.abs() + eps)
    assert torch.allclose(p, closed, atol=1e-12)
    ps, ms, vs = p0.tolist(), [0.0] * 50, [0.0] * 50
    p2, m2, v2 = p0.clone(), torch.zeros(50, dtype=torch.float64), torch.zeros(50, dtype=torch.float64)
    for t in range(1, 4):
        gt = torch.randn(50, generator=g, dtype=torch.float64)
        O.adamw_step_scalar(ps, gt.tolist(), ms, vs, t, lr, 0.9, 0.95, eps, wd)
        O.adamw_step(p2, gt, m2, v2, t, lr, 0.9, 0.95, eps, wd)
    assert torch.allclose(p2, torch.tensor(ps, dtype=torch.float64), atol=1e-12)


# ---------------------------------------------------------- flat param layout --

def test_flat_numel_matches_reference_model_stats():
    """data/model_stats.json:92,104 -- per-layer flat-shard numel of
    deepspeedllama_tiny and deepspeedllama_7b."""
    tiny = O.LayerShape(hidden=2048, heads=32, kv_heads=32, head_dim=64, ffn=5632)
    l7b = O.LayerShape(hidden=4096, heads=32, kv_heads=32, head_dim=128, ffn=11008)
    assert O.flat_numel(tiny) == 51_384_320
    assert O.flat_numel(l7b) == 202_383_360
    cfg3 = O.LayerShape(hidden=2048, heads=32, kv_heads=8, head_dim=64, ffn=8192)
    assert O.flat_numel(cfg3) == 60_821_504
    g = torch.Generator().manual_seed(0)
    s = O.LayerShape(hidden=8, heads=2, kv_heads=1, head_dim=4, ffn=12)
    p = O.init_params(s, g)
    assert all(torch.equal(a, b) for a, b in zip(O.unflatten(O.flatten(p), s).values(),
                                                  (p[k] for k in O.PARAM_ORDER)))
