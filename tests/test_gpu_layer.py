"""GPU parity of the drop-in decoder layer, the stage runner and the fused
AdamW-in-backward, against the oracle and the transformers golden fixtures.

Layer configs are the BASELINE configs scaled down so the fp64 oracle
finishes in seconds (same head_dim, GQA ratio, RoPE theta, dtype and mask
kind); the full-size shapes are exercised by tests/test_gpu_fullsize.py.
"""
import os

import numpy as np
import pytest
import torch

from oracle import decoder as O
from tests._tol import assert_close, assert_loss, assert_matched

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _layer(spec_kw, dev, param_dtype=torch.float32, seed=0, std=0.02, window=None):
    from zorse_amd import llama_simple as L
    cfg = L.llama_config(**spec_kw)
    g = torch.Generator().manual_seed(seed)
    layer = L.LlamaDecoderLayer(cfg, 0, sliding_window=window, init_std=std, generator=g)
    with torch.no_grad():
        ln = layer.param_view("ln1")
        ln.copy_(1 + 0.1 * torch.randn(ln.shape, generator=g))
        ln = layer.param_view("ln2")
        ln.copy_(1 + 0.1 * torch.randn(ln.shape, generator=g))
    return layer.to(device=dev, dtype=param_dtype)


def _oracle_params(layer, dtype):
    """The layer's weights as the GPU computes with them (rounded to the
    compute dtype), in fp64 on the CPU."""
    return {short: layer.param_view(short).detach().to(dtype).double().cpu()
            for short in O.PARAM_ORDER}


def _oracle_shape(layer):
    s = layer.spec
    return O.LayerShape(hidden=s.hidden, heads=s.heads, kv_heads=s.kv_heads,
                        head_dim=s.head_dim, ffn=s.ffn, eps=s.eps, theta=s.rope_theta,
                        window=s.window)


def _check_layer(layer, x, dout, dtype, what, rope="half"):
    """Output, dx and all nine weight gradients against the fp64 oracle; for
    16-bit layers also against the same layer computed by plain PyTorch in
    that dtype (the precision-matched bar of tests/_tol.py) and the loss
    <out, dout>."""
    xg = x.to(layer.flat_param.device).requires_grad_(True)
    out = layer(xg)[0]
    assert out.dtype == dtype and out.shape == x.shape
    out.backward(dout.to(xg.device))
    return _compare_layer(layer, x, xg, out, dout, dtype, what, rope)


def _compare_layer(layer, x, xg, out, dout, dtype, what, rope="half"):
    """The checks of _check_layer on a forward / backward already run (out,
    xg.grad, the layer's flat gradient)."""
    p = _oracle_params(layer, dtype)
    shape = _oracle_shape(layer)
    rout, rdx, rgrads = O.layer_fwd_bwd(x.double(), p, shape, dout.double(), rope=rope)
    grad = layer.flat_param.grad
    offs = layer.spec.offsets()
    got = {"out": out, "dx": xg.grad}
    got.update({"d" + k: grad[offs[k][0]:offs[k][1]].view(rgrads[k].shape)
                for k in O.PARAM_ORDER})
    ref = {"out": rout, "dx": rdx}
    ref.update({"d" + k: rgrads[k] for k in O.PARAM_ORDER})
    if dtype == torch.float32:
        for k in got:
            assert_close(got[k], ref[k], dtype, f"{what} {k}")
        return out, rout
    lout, ldx, lgrads = O.layer_fwd_bwd(x, {k: v.to(dtype) for k, v in p.items()}, shape, dout,
                                        rope=rope, attn="flash")
    low = {"out": lout, "dx": ldx}
    low.update({"d" + k: lgrads[k] for k in O.PARAM_ORDER})
    for k in got:
        assert_matched(got[k], ref[k], low[k], dtype, f"{what} {k}")
    assert_loss(out, rout, lout, dout, f"{what} loss")
    return out, rout


# ------------------------------------------------------------ golden fixtures --

@pytest.mark.parametrize("name", ["llama_gqa_d16", "llama_mha_d64", "mistral_swa_d64"])
def test_layer_fp32_matches_transformers_golden(dev, name):
    from zorse_amd import llama_simple as L
    z = np.load(os.path.join(GOLDEN, name + ".npz"))
    hidden, heads, kv, hd, ffn, B, S, theta, window, seed = (float(v) for v in z["meta"])
    cfg = L.llama_config(hidden_size=int(hidden), num_attention_heads=int(heads),
                         num_key_value_heads=int(kv), head_dim=int(hd), intermediate_size=int(ffn),
                         rope_theta=theta)
    layer = L.LlamaDecoderLayer(cfg, 0, sliding_window=int(window) or None).to(dev)
    layer.load_named({k: torch.from_numpy(z["w_" + k]) for k in O.PARAM_ORDER})
    x = torch.from_numpy(z["x"]).to(dev).requires_grad_(True)
    out = layer(x)[0]
    out.backward(torch.from_numpy(z["dout"]).to(dev))
    assert_close(out, torch.from_numpy(z["out"]), torch.float32, "out")
    assert_close(x.grad, torch.from_numpy(z["dx"]), torch.float32, "dx")
    offs = layer.spec.offsets()
    for k in O.PARAM_ORDER:
        a, b = offs[k]
        ref = torch.from_numpy(z["g_" + k])
        assert_close(layer.flat_param.grad[a:b].view(ref.shape), ref, torch.float32, "d" + k)


def test_layer_bf16_matches_transformers_golden(dev):
    from zorse_amd import llama_simple as L
    z = np.load(os.path.join(GOLDEN, "mistral_swa_d64.npz"))
    hidden, heads, kv, hd, ffn, B, S, theta, window, seed = (float(v) for v in z["meta"])
    cfg = L.llama_config(hidden_size=int(hidden), num_attention_heads=int(heads),
                         num_key_value_heads=int(kv), head_dim=int(hd), intermediate_size=int(ffn),
                         rope_theta=theta)
    layer = L.LlamaDecoderLayer(cfg, 0, sliding_window=int(window), param_dtype=torch.bfloat16)
    layer = layer.to(dev)
    layer.load_named({k: torch.from_numpy(z["w_" + k]) for k in O.PARAM_ORDER})
    x = torch.from_numpy(z["x"]).to(torch.bfloat16)
    out = layer(x.to(dev))[0]
    shape = O.LayerShape(hidden=int(hidden), heads=int(heads), kv_heads=int(kv), head_dim=int(hd),
                         ffn=int(ffn), theta=theta, window=int(window))
    wb = {k: torch.from_numpy(z["w_" + k]).to(torch.bfloat16) for k in O.PARAM_ORDER}
    with torch.no_grad():
        lout = O.decoder_layer(x, wb, shape, attn="flash")
        rout = O.decoder_layer(x.double(), {k: v.double() for k, v in wb.items()}, shape)
    assert_close(out, torch.from_numpy(z["out"]), torch.bfloat16, "out vs golden")
    assert_matched(out, rout, lout, torch.bfloat16, "out")


# ------------------------------------------------------------ scaled configs --

CONFIGS = {
    # BASELINE cfg1 exactly (fp32, tiny): hidden 256, 4 x 64, FFN 688, B 2, S 128
    "cfg1_fp32": (dict(hidden_size=256, num_attention_heads=4, intermediate_size=688,
                       rope_theta=1e4), None, torch.float32, (2, 128)),
    # cfg3 scaled: GQA 4:1, d 64, theta 5e5, fp16
    "cfg3_fp16_gqa": (dict(hidden_size=512, num_attention_heads=8, num_key_value_heads=2,
                           intermediate_size=1024, rope_theta=5e5), None, torch.float16, (2, 256)),
    # cfg4 scaled: MHA d 128, theta 1e4, bf16
    "cfg4_bf16": (dict(hidden_size=512, num_attention_heads=4, intermediate_size=1376,
                       rope_theta=1e4), None, torch.bfloat16, (1, 384)),
    # cfg5 scaled: GQA 4:1, d 128, SWA, theta 1e6, bf16
    "cfg5_bf16_swa": (dict(hidden_size=512, num_attention_heads=4, num_key_value_heads=1,
                           intermediate_size=1792, rope_theta=1e6), 160, torch.bfloat16, (1, 512)),
}


@pytest.mark.parametrize("name", list(CONFIGS))
def test_layer_fwd_bwd_vs_oracle(dev, name):
    kw, window, dtype, (B, S) = CONFIGS[name]
    print(f"layer {name}", flush=True)
    layer = _layer(kw, dev, param_dtype=dtype, window=window,
                   seed=list(CONFIGS).index(name) + 100)
    g = torch.Generator().manual_seed(7)
    x = torch.randn(B, S, kw["hidden_size"], generator=g).to(dtype)
    dout = torch.randn(B, S, kw["hidden_size"], generator=g).to(dtype)
    _check_layer(layer, x, dout, dtype, name)


# Sequence lengths that are not multiples of 8 (and token counts off the
# GEMM pipeline's 256 grid): every projection product then runs on the masked
# general GEMM kernel, and the fused gate|up GEMM on its ragged-tile kernel
# where the token count is a multiple of 8.
RAGGED_LONG = {
    "cfg4_bf16_S1100": ("cfg4_bf16", None, (1, 1100)),
    "cfg3_fp16_S516x2": ("cfg3_fp16_gqa", None, (2, 516)),
    "cfg5_bf16_swa_S1027": ("cfg5_bf16_swa", 160, (1, 1027)),
}


@pytest.mark.parametrize("name", list(RAGGED_LONG))
def test_layer_ragged_long_sequence(dev, name):
    from zorse_amd import layer as LY
    base, window, (B, S) = RAGGED_LONG[name]
    kw, _, dtype, _ = CONFIGS[base]
    assert S % 8 != 0 and (B * S) % 256 != 0
    print(f"layer {name}", flush=True)
    layer = _layer(kw, dev, param_dtype=dtype, window=window, seed=211)
    g = torch.Generator().manual_seed(17)
    x = torch.randn(B, S, kw["hidden_size"], generator=g).to(dtype)
    dout = torch.randn(B, S, kw["hidden_size"], generator=g).to(dtype)
    _check_layer(layer, x, dout, dtype, name)


# Layers whose every projection GEMM is on the MFMA pipeline's grid (tokens,
# hidden, q|k|v width and FFN multiples of 256).
HIP_GEMM = {
    "cfg3_fp16_gqa": (CONFIGS["cfg3_fp16_gqa"][0], None, torch.float16, (2, 256)),
    "cfg4_bf16_F1536": (dict(hidden_size=512, num_attention_heads=4, intermediate_size=1536,
                             rope_theta=1e4), None, torch.bfloat16, (1, 512)),
    "cfg5_bf16_swa": (CONFIGS["cfg5_bf16_swa"][0], 160, torch.bfloat16, (1, 512)),
}


def _forbid_library_products(monkeypatch):
    """Make every torch GEMM entry point the layer could reach raise."""
    def forbidden(name):
        def fn(*a, **k):
            raise AssertionError(f"torch.{name} called on the layer's path")
        return fn
    for name in ("mm", "addmm", "matmul", "bmm", "baddbmm"):
        monkeypatch.setattr(torch, name, forbidden(name))
    monkeypatch.setattr(torch.Tensor, "__matmul__", forbidden("Tensor.__matmul__"))


@pytest.mark.parametrize("transposed", [False, True], ids=["dY", "dYt"])
@pytest.mark.parametrize("name", list(HIP_GEMM))
def test_layer_every_product_hand_written(dev, name, transposed, monkeypatch):
    """All twelve projection products of a layer step go through the
    hand-written GEMMs -- the four forward ones (q|k|v with RoPE in its
    epilogue, gate|up with the SwiGLU epilogue), the four input gradients
    dY W on W as stored, and the four
    weight gradients dY^T X (o and down on the token-major dY, X as stored;
    gate|up and q|k|v on the dY^T the SwiGLU / attention backward kernels
    write from their epilogues, or with set_transposed_wgrad(False) on dY as
    stored too) -- each on the
    MFMA pipeline (zk_gemm_path "tiled"); no torch GEMM, no transpose pass
    and no separate RoPE pass is called.  Parity against the fp64 oracle as
    every layer test."""
    from zorse_amd import kernels as K
    from zorse_amd import layer as LY
    kw, window, dtype, (B, S) = HIP_GEMM[name]
    print(f"layer {name} (every product hand-written)", flush=True)
    layer = _layer(kw, dev, param_dtype=dtype, window=window, seed=307)
    g = torch.Generator().manual_seed(29)
    x = torch.randn(B, S, kw["hidden_size"], generator=g).to(dtype)
    dout = torch.randn(B, S, kw["hidden_size"], generator=g).to(dtype)
    calls = []
    real_gemm, real_swiglu, real_rope_gemm = K.gemm, K.gemm_swiglu, K.gemm_rope

    def gemm(a, b, *, a_kmajor=False, b_kmajor=False, residual=None, out=None):
        M, Kd = (a.shape[1], a.shape[0]) if a_kmajor else a.shape
        N = b.shape[1] if b_kmajor else b.shape[0]
        ldc = out.stride(0) if out is not None else N
        calls.append(("gemm", a_kmajor, b_kmajor,
                      K.gemm_path(M, N, Kd, a.stride(0), b.stride(0), ldc, a.dtype, a_kmajor,
                                  b_kmajor, residual.stride(0) if residual is not None else -1)))
        return real_gemm(a, b, a_kmajor=a_kmajor, b_kmajor=b_kmajor, residual=residual, out=out)

    def gemm_swiglu(*a, **k):
        calls.append(("gemm_swiglu", False, False,
                      "tiled" if K.gemm_nt_supported(a[0].shape[0], 2 * a[1].shape[0],
                                                     a[0].shape[1]) else "general"))
        return real_swiglu(*a, **k)

    def gemm_rope(x, w, **k):
        # the epilogue takes launches on the tiled grid with head dim 64 / 128
        # and whole 128-column blocks of rotated heads
        on = (K.gemm_path(x.shape[0], w.shape[0], x.shape[1], x.stride(0), w.stride(0),
                          w.shape[0], x.dtype) == "tiled" and k["head_dim"] in (64, 128)
              and k["rot_cols"] % 128 == 0)
        calls.append(("gemm_rope", False, False, "tiled" if on else "general"))
        return real_rope_gemm(x, w, **k)

    def no_transpose(*a, **k):
        raise AssertionError("zk_transpose called on the layer's path")

    def no_rope(*a, **k):
        raise AssertionError("a separate RoPE pass called on the layer's path")

    monkeypatch.setattr(K, "gemm", gemm)
    monkeypatch.setattr(K, "gemm_swiglu", gemm_swiglu)
    monkeypatch.setattr(K, "gemm_rope", gemm_rope)
    monkeypatch.setattr(K, "transpose", no_transpose)
    monkeypatch.setattr(K, "rope_", no_rope)
    xg = x.to(dev).requires_grad_(True)
    with monkeypatch.context() as m:
        _forbid_library_products(m)
        prev = LY.set_fused_gate_up(True)
        prev_t = LY.set_transposed_wgrad(transposed)
        try:
            out = layer(xg)[0]
            out.backward(dout.to(dev))
            torch.cuda.synchronize()
        finally:
            LY.set_fused_gate_up(prev)
            LY.set_transposed_wgrad(prev_t)
    _compare_layer(layer, x, xg, out, dout, dtype,
                   f"{name} hand-written GEMMs" + (" (dY^T)" if transposed else ""))
    # the layer step itself: 4 forward + 8 backward products (the oracle runs
    # on the CPU, outside these wrappers)
    assert len(calls) == 12, calls
    assert sum(c[0] == "gemm_swiglu" for c in calls) == 1, calls
    assert sum(c[0] == "gemm_rope" for c in calls) == 1, calls
    # dY W (4), plus the gate|up / q|k|v weight gradients when they read the
    # dY^T their producers wrote (2); the other weight gradients on dY, X as
    # stored
    assert sum(c[1:3] == (False, True) for c in calls) == (6 if transposed else 4), calls
    assert sum(c[1:3] == (True, True) for c in calls) == (2 if transposed else 4), calls
    assert all(c[3] == "tiled" for c in calls), calls


def test_cfg1_head_and_cross_entropy_loss(dev):
    """BASELINE cfg1 end to end: layer + final RMSNorm + linear head + CE over
    integer labels (vocab 1000), fp32, all on this build's kernels (chunked
    vocabulary CE); loss agreement 1e-3 (relative 1e-4 on the fp32 path)."""
    from zorse_amd import llama_simple as L
    kw, _, dtype, (B, S) = CONFIGS["cfg1_fp32"]
    layer = _layer(kw, dev, seed=0)
    norm = L.LlamaRMSNorm(256).to(dev)
    g = torch.Generator().manual_seed(0)
    head = (0.02 * torch.randn(1000, 256, generator=g))
    x = torch.randn(B, S, 256, generator=g)
    labels = torch.randint(0, 1000, (B, S), generator=g)
    xg = x.to(dev).requires_grad_(True)
    lm_head = torch.nn.Linear(256, 1000, bias=False).to(dev)
    with torch.no_grad():
        lm_head.weight.copy_(head)
    hw = lm_head.weight
    from zorse_amd.lm_head import OutputLayerLoss
    loss = OutputLayerLoss(norm, lm_head, chunk=384)(layer(xg)[0], labels.to(dev))
    loss.backward()
    p = _oracle_params(layer, torch.float32)
    xr = x.double().requires_grad_(True)
    pr = {k: v.clone().requires_grad_(True) for k, v in p.items()}
    hr = head.double().requires_grad_(True)
    rl = O.lm_head_ce(O.decoder_layer(xr, pr, _oracle_shape(layer)),
                      torch.ones(256, dtype=torch.float64), hr, labels, 1e-6)
    rl.backward()
    assert abs(loss.item() - rl.item()) <= 1e-3 * max(1.0, abs(rl.item()))
    assert abs(loss.item() - rl.item()) <= 1e-4 * abs(rl.item())
    assert_close(xg.grad, xr.grad, torch.float32, "dx")
    assert_close(hw.grad, hr.grad, torch.float32, "dhead")
    offs = layer.spec.offsets()
    for k in O.PARAM_ORDER:
        a, b = offs[k]
        assert_close(layer.flat_param.grad[a:b].view(pr[k].shape), pr[k].grad, torch.float32, k)


def test_block_and_profiler_protocol(dev):
    """Block.forward(x) as the layer profiler calls it
    (utils/runtime_estimator.py:216-243): fp32 params under fp16 autocast,
    fp16 input, then two backward passes with retain_graph=True; weight
    gradients accumulate (2x)."""
    from zorse_amd import llama_simple as L
    cfg = L.llama_config(hidden_size=256, num_attention_heads=4, intermediate_size=512)
    blk = L.Block(cfg, 0, torch.float16, init_std=0.02,
                  generator=torch.Generator().manual_seed(1)).to(dev)
    x = torch.randn(2, 64, 256, device=dev).to(torch.float16).requires_grad_(True)
    with torch.autocast("cuda", dtype=torch.float16):
        out = blk(x)
    assert out.dtype == torch.float16 and blk.cached_position_ids.shape == (1, 64)
    gr = torch.rand(out.shape, device=dev, dtype=out.dtype)
    out.backward(gr, retain_graph=True)
    g1 = blk.block.flat_param.grad.clone()
    assert g1.dtype == torch.float32
    out.backward(gr, retain_graph=True)
    assert torch.allclose(blk.block.flat_param.grad, 2 * g1, rtol=1e-6, atol=1e-7)
    layer = blk.block
    p = _oracle_params(layer, torch.float16)
    xc, grc = x.detach().cpu(), gr.cpu()
    rout, _, rg = O.layer_fwd_bwd(xc.double(), p, _oracle_shape(layer), grc.double())
    lout, _, lg = O.layer_fwd_bwd(xc, {k: v.half() for k, v in p.items()}, _oracle_shape(layer),
                                  grc, attn="flash")
    assert_matched(out, rout, lout, torch.float16, "out")
    a, b = layer.spec.offsets()["q"]
    assert_matched(g1[a:b].view(rg["q"].shape), rg["q"], lg["q"], torch.float16, "dq_proj")


def test_deepspeed_llama_model_forward(dev):
    from zorse_amd import llama_simple as L
    torch.manual_seed(0)
    model = L.get_model("deepspeedllama_tiny", vocab_size=512, seq_length=64, layers=2).to(dev)
    ids = torch.randint(0, 512, (1, 64), device=dev)
    logits = model(ids)
    assert logits.shape == (1, 64, 512) and torch.isfinite(logits).all()
    logits.float().sum().backward()
    assert all(torch.isfinite(b.block.flat_param.grad).all() for b in model.layers)


def test_layer_position_ids(dev):
    """position_ids other than 0 .. S-1, given as a device tensor, rotate q / k
    by those positions (forward and backward) -- against the oracle with the
    same positions; the Block's cached arange and an explicit arange give the
    plain result bit for bit; ids that differ between batch rows, negative
    ids and a length mismatch are rejected."""
    from zorse_amd import llama_simple as L
    kw = dict(hidden_size=256, num_attention_heads=2, num_key_value_heads=1,
              intermediate_size=512, rope_theta=1e4)
    dtype = torch.bfloat16
    layer = _layer(kw, dev, param_dtype=dtype, seed=31)
    g = torch.Generator().manual_seed(32)
    B, S = 2, 192
    x = torch.randn(B, S, 256, generator=g).to(dtype)
    dout = torch.randn(B, S, 256, generator=g).to(dtype)
    pos = 3 * torch.arange(S) + 11          # gaps and an offset: tables past S
    xg = x.to(dev).requires_grad_(True)
    out = layer(xg, position_ids=pos[None].expand(B, S).to(dev))[0]
    out.backward(dout.to(dev))
    p = _oracle_params(layer, dtype)
    shape = _oracle_shape(layer)
    rout, rdx, rg = O.layer_fwd_bwd(x.double(), p, shape, dout.double(), positions=pos)
    lout, ldx, lg = O.layer_fwd_bwd(x, {k: v.to(dtype) for k, v in p.items()}, shape, dout,
                                    attn="flash", positions=pos)
    assert_matched(out, rout, lout, dtype, "out")
    assert_matched(xg.grad, rdx, ldx, dtype, "dx")
    offs = layer.spec.offsets()
    for k in ("q", "k", "o"):
        a, b = offs[k]
        assert_matched(layer.flat_param.grad[a:b].view(rg[k].shape), rg[k], lg[k], dtype, "d" + k)
    # plain positions: three ways, one result
    with torch.no_grad():
        plain = layer(x.to(dev))[0]
        explicit = layer(x.to(dev), position_ids=torch.arange(S, device=dev)[None])[0]
        blk = L.Block(L.llama_config(**kw), 0, param_dtype=dtype).to(dev)
        blk.block.flat_param.copy_(layer.flat_param)
        viablock = blk(x.to(dev))
        shifted = layer(x.to(dev), position_ids=pos[None].to(dev))[0]
    assert torch.equal(plain, explicit) and torch.equal(plain, viablock)
    assert not torch.equal(plain, shifted)
    with pytest.raises(NotImplementedError):
        layer(x.to(dev), position_ids=torch.stack([torch.arange(S), pos]).to(dev))
    with pytest.raises(ValueError):
        layer(x.to(dev), position_ids=(torch.arange(S) - 1)[None].to(dev))
    with pytest.raises(ValueError):
        layer(x.to(dev), position_ids=torch.arange(S - 1)[None].to(dev))


def test_cross_entropy_ignore_index_and_label_range(dev):
    """The chunked-vocabulary CE ignores exactly ignore_index (-100) like
    F.cross_entropy -- loss and gradients against it in fp64 with a third of
    the labels ignored -- and rejects labels outside [0, V) with ValueError
    rather than computing a wrong loss."""
    from zorse_amd.lm_head import lm_head_cross_entropy
    g = torch.Generator().manual_seed(33)
    T, h, V = 96, 64, 500
    x = torch.randn(T, h, generator=g)
    w = 0.1 * torch.randn(V, h, generator=g)
    labels = torch.randint(0, V, (T,), generator=g)
    labels[::3] = -100
    xg, wg = x.to(dev).requires_grad_(True), w.to(dev).requires_grad_(True)
    loss = lm_head_cross_entropy(xg, wg, labels.to(dev), chunk=128)
    loss.backward()
    xr, wr = x.double().requires_grad_(True), w.double().requires_grad_(True)
    ref = torch.nn.functional.cross_entropy(xr @ wr.t(), labels)
    ref.backward()
    assert abs(loss.item() - ref.item()) <= 1e-4 * abs(ref.item())
    assert_close(xg.grad, xr.grad, torch.float32, "dx")
    assert_close(wg.grad, wr.grad, torch.float32, "dw")
    for bad in (-1, V, V + 7):
        lab = labels.clone()
        lab[5] = bad
        with pytest.raises(ValueError):
            lm_head_cross_entropy(xg, wg, lab.to(dev), chunk=128)


# ----------------------------------------------------------- stage + AdamW --

def test_stage_runner_optimizer_in_backwards(dev):
    """Two bf16 layers with fp32 master weights; AdamW (lr 1e-4, betas 0.9 /
    0.95, wd 0.1) stepped per layer inside the backward on the optimizer
    stream.  Checks: each layer's gradient (captured by a hook that runs just
    before the optimizer's) matches the oracle's; the fp32 master equals the
    oracle's AdamW applied to that gradient; the bf16 parameter is the rounded
    master; the gradient is released."""
    from zorse_amd.stage import StageRunner
    kw = dict(hidden_size=256, num_attention_heads=2, intermediate_size=512, rope_theta=1e4)
    dtype = torch.bfloat16
    layers = [_layer(kw, dev, param_dtype=dtype, seed=s) for s in (1, 2)]
    before = [_oracle_params(l, dtype) for l in layers]
    shape = _oracle_shape(layers[0])
    captured = {}
    for i, l in enumerate(layers):
        l.flat_param.register_post_accumulate_grad_hook(
            lambda p, i=i: captured.__setitem__(i, p.grad.detach().clone()))
    runner = StageRunner(layers, lr=1e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1)
    g = torch.Generator().manual_seed(3)
    x = torch.randn(1, 256, 256, generator=g).to(dtype)
    dout = torch.randn(1, 256, 256, generator=g).to(dtype)
    runner.step(x.to(dev), dout.to(dev))
    runner.wait_optimizer()
    torch.cuda.synchronize()
    assert sorted(captured) == [0, 1]
    xr = x.double().requires_grad_(True)
    prs = [{k: v.clone().requires_grad_(True) for k, v in p.items()} for p in before]
    y = O.decoder_layer(O.decoder_layer(xr, prs[0], shape), prs[1], shape)
    y.backward(dout.double())
    # the same two-layer stack as plain PyTorch computes it in bf16
    pls = [{k: v.to(dtype).requires_grad_(True) for k, v in p.items()} for p in before]
    yl = O.decoder_layer(O.decoder_layer(x, pls[0], shape, attn="flash"), pls[1], shape,
                         attn="flash")
    yl.backward(dout)
    for i, (layer, pr, opt) in enumerate(zip(layers, prs, runner.optimizers)):
        gref = O.flatten({k: v.grad for k, v in pr.items()})
        glow = O.flatten({k: v.grad for k, v in pls[i].items()})
        assert_matched(captured[i], gref, glow, dtype, f"layer {i} grad")
        flat0 = O.flatten(before[i]).clone()
        m, v = torch.zeros_like(flat0), torch.zeros_like(flat0)
        O.adamw_step(flat0, captured[i].double().cpu(), m, v, 1, 1e-4, 0.9, 0.95, 1e-8, 0.1)
        master = opt.master_param(layer.flat_param)
        assert_close(master, flat0, torch.float32, f"layer {i} master")
        assert torch.equal(layer.flat_param.detach().cpu(), master.cpu().to(dtype))
        assert layer.flat_param.grad is None


def test_stage_steps_each_parameter_once(dev):
    """A stage layer with several parameters (the last stage's output layer
    is Sequential(norm, lm_head), models/llama_simple.py:559-561): each
    parameter's post-accumulate hook steps that parameter alone, so every
    parameter gets exactly one AdamW update per step in both overlap modes --
    the same weights as torch.optim.AdamW applied once to the captured
    gradients."""
    from zorse_amd.stage import StageRunner
    torch.manual_seed(34)
    x = torch.randn(2, 16, 64, device=dev)
    dout = torch.randn(2, 16, 64, device=dev)
    init = torch.nn.Sequential(torch.nn.Linear(64, 64, bias=False),
                               torch.nn.Linear(64, 64, bias=False)).to(dev)
    results = {}
    for mode in ("attention", "immediate"):
        layer = torch.nn.Sequential(torch.nn.Linear(64, 64, bias=False),
                                    torch.nn.Linear(64, 64, bias=False)).to(dev)
        layer.load_state_dict(init.state_dict())
        grads = {}
        for name, p in layer.named_parameters():
            p.register_post_accumulate_grad_hook(
                lambda t, name=name: grads.__setitem__(name, t.grad.detach().clone()))
        runner = StageRunner([layer], lr=1e-2, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1,
                             optimizer_overlap=mode)
        runner.step(x, dout)
        runner.wait_optimizer()
        torch.cuda.synchronize()
        steps = {n: runner.optimizers[0].state[p]["step"] for n, p in layer.named_parameters()}
        assert steps == {"0.weight": 1, "1.weight": 1}, (mode, steps)
        ref = {n: p.detach().clone().requires_grad_(True) for n, p in init.named_parameters()}
        opt = torch.optim.AdamW(list(ref.values()), lr=1e-2, betas=(0.9, 0.95), eps=1e-8,
                                weight_decay=0.1, foreach=False)
        for n, p in ref.items():
            p.grad = grads[n]
        opt.step()
        for n, p in layer.named_parameters():
            assert_close(p, ref[n], torch.float32, f"{mode} {n}")
        results[mode] = [p.detach().clone() for p in layer.parameters()]
    for a, b in zip(results["attention"], results["immediate"]):
        assert torch.equal(a, b)


def test_stage_no_transposes_no_library_gemm(dev, monkeypatch):
    """Two 2-layer stage steps at 1024 tokens with AdamW in the backward: no
    transpose pass and no torch GEMM anywhere on the path (forward, backward,
    optimizer step), and the step runs twice without error."""
    from zorse_amd import kernels as K
    from zorse_amd.stage import StageRunner
    kw = dict(hidden_size=256, num_attention_heads=2, intermediate_size=512, rope_theta=1e4)
    dtype = torch.bfloat16
    g = torch.Generator().manual_seed(9)
    x = torch.randn(1, 1024, 256, generator=g).to(dtype).to(dev)
    dout = torch.randn(1, 1024, 256, generator=g).to(dtype).to(dev)
    layers = [_layer(kw, dev, param_dtype=dtype, seed=s) for s in (1, 2)]
    runner = StageRunner(layers, lr=1e-4)

    def no_transpose(*a, **k):
        raise AssertionError("zk_transpose called on the stage's path")

    monkeypatch.setattr(K, "transpose", no_transpose)
    before = [l.flat_param.detach().clone() for l in layers]
    with monkeypatch.context() as m:
        _forbid_library_products(m)
        for _ in range(2):
            runner.step(x, dout)
        runner.wait_optimizer()
        torch.cuda.synchronize()
    for b, l in zip(before, layers):
        assert torch.isfinite(l.flat_param).all() and not torch.equal(b, l.flat_param)


def _check_stack_against_oracle(layers, before, xs, douts, captured, masters, dtype, what,
                                lr=1e-4, betas=(0.9, 0.95), eps=1e-8, wd=0.1):
    """A stack of layers run by the stage runner over len(xs) steps, against
    the fp64 oracle: per step, layer and each of the nine parameter slices,
    the gradient the optimizer consumed (``captured[step][i]``) against the
    oracle's gradient of the stack at the weights that step saw
    (``before[step][i]``, oracle parameter dicts), with the precision-matched
    bar (plain PyTorch in ``dtype`` as the reference layer); after the last
    step each fp32 master against the oracle's AdamW applied to the captured
    gradients."""
    shape = _oracle_shape(layers[0])
    offs = layers[0].spec.offsets()
    for step, (x, dout) in enumerate(zip(xs, douts)):
        x, dout = x.detach().cpu(), dout.detach().cpu()
        xr = x.double().requires_grad_(True)
        prs = [{k: v.clone().requires_grad_(True) for k, v in p.items()} for p in before[step]]
        pls = [{k: v.to(dtype).requires_grad_(True) for k, v in p.items()} for p in before[step]]
        y, yl = xr, x
        for pr, pl in zip(prs, pls):
            y = O.decoder_layer(y, pr, shape)
            yl = O.decoder_layer(yl, pl, shape, attn="flash")
        y.backward(dout.double())
        yl.backward(dout)
        for i in range(len(layers)):
            got = captured[step][i]
            for k in O.PARAM_ORDER:
                a, b = offs[k]
                assert_matched(got[a:b].view(prs[i][k].shape), prs[i][k].grad, pls[i][k].grad,
                               dtype, f"{what} step {step + 1} layer {i} d{k}")
    for i, master in enumerate(masters):
        p = O.flatten(before[0][i]).clone()
        m, v = torch.zeros_like(p), torch.zeros_like(p)
        for t in range(len(xs)):
            O.adamw_step(p, captured[t][i].double().cpu(), m, v, t + 1, lr, betas[0], betas[1],
                         eps, wd)
        assert_close(master, p, torch.float32, f"{what} layer {i} master")


@pytest.mark.parametrize("S", [256, 1024])
def test_stage_recompute_attention_cache(dev, S):
    """Recompute mode (the reference pipeline's second forward inside the
    backward, zorse_utils/pipeline_schedule_v2.py:157-200): with the attention
    cache the re-forward launches no attention kernel, and every layer
    gradient is bit-identical to recompute without the cache and to the
    single-forward path (the kernels are deterministic); and the cached
    recompute's gradients (each parameter slice) and fp32 masters against the
    fp64 oracle.  1024 tokens run every GEMM on the tiled pipeline, 256 on
    the masked kernel for the token-sized dimensions."""
    from zorse_amd import layer as L
    from zorse_amd.stage import StageRunner
    kw = dict(hidden_size=256, num_attention_heads=2, intermediate_size=512, rope_theta=1e4)
    dtype = torch.bfloat16
    g = torch.Generator().manual_seed(5)
    x = torch.randn(1, S, 256, generator=g).to(dtype).to(dev)
    dout = torch.randn(1, S, 256, generator=g).to(dtype).to(dev)
    calls = {"n": 0}
    real = L.K.attn_fwd

    def counting(*a, **k):
        calls["n"] += 1
        return real(*a, **k)

    results = {}
    try:
        L.K.attn_fwd = counting
        for name, rc, cache in (("plain", False, False), ("recompute", True, False),
                                ("cached", True, True)):
            layers = [_layer(kw, dev, param_dtype=dtype, seed=s) for s in (1, 2)]
            before = [_oracle_params(l, dtype) for l in layers]
            grads = {}
            for i, l in enumerate(layers):
                l.flat_param.register_post_accumulate_grad_hook(
                    lambda p, i=i: grads.__setitem__(i, p.grad.detach().clone()))
            runner = StageRunner(layers, lr=1e-4, recompute=rc, cache_attention=cache)
            calls["n"] = 0
            runner.step(x, dout)
            runner.wait_optimizer()
            torch.cuda.synchronize()
            masters = [o.master_param(l.flat_param) for o, l in zip(runner.optimizers, layers)]
            results[name] = (grads, calls["n"], [len(c) for c in runner.attn_caches], layers,
                             before, masters)
    finally:
        L.K.attn_fwd = real
    assert results["plain"][1] == 2 and results["recompute"][1] == 4
    assert results["cached"][1] == 2, "the recompute forward ran attention again"
    assert results["cached"][2] == [0, 0], "cache entries left after the backward"
    for i in (0, 1):
        assert torch.equal(results["cached"][0][i], results["recompute"][0][i])
        assert torch.equal(results["cached"][0][i], results["plain"][0][i])
    # and against the oracle, not only against the plain path
    grads, _, _, layers, before, masters = results["cached"]
    _check_stack_against_oracle(layers, [before], [x], [dout], [grads], masters, dtype,
                                f"recompute S={S}")


def test_stage_offload_inputs(dev):
    """Host offload in recompute mode (the reference pipeline's CPU activation
    buffers on mem_copy_stream, zorse_utils/pipeline_schedule_v2.py:119-136):
    each layer input goes D2H to pinned memory in the forward and returns H2D
    one layer ahead in the backward.  Over two steps the gradients and weights
    are bit-identical to recompute without offload, the attention cache still
    hits across the round trip (one attention forward per layer), and the
    gradients of both steps (each parameter slice) and the fp32 masters agree
    with the fp64 oracle of the three-layer stack."""
    from zorse_amd import layer as L
    from zorse_amd.stage import StageRunner
    kw = dict(hidden_size=256, num_attention_heads=2, intermediate_size=512, rope_theta=1e4)
    dtype = torch.bfloat16
    g = torch.Generator().manual_seed(15)
    xs = [torch.randn(1, 256, 256, generator=g).to(dtype).to(dev) for _ in range(2)]
    douts = [torch.randn(1, 256, 256, generator=g).to(dtype).to(dev) for _ in range(2)]
    calls = {"n": 0}
    real = L.K.attn_fwd

    def counting(*a, **k):
        calls["n"] += 1
        return real(*a, **k)

    results = {}
    try:
        L.K.attn_fwd = counting
        for name, off in (("recompute", False), ("offload", True)):
            layers = [_layer(kw, dev, param_dtype=dtype, seed=s) for s in (1, 2, 3)]
            grads = {}
            for i, l in enumerate(layers):
                l.flat_param.register_post_accumulate_grad_hook(
                    lambda p, i=i: grads.__setitem__(i, p.grad.detach().clone()))
            runner = StageRunner(layers, lr=1e-4, recompute=True, cache_attention=True,
                                 offload_inputs=off)
            per_step, weights_seen = [], []
            for x, dout in zip(xs, douts):
                weights_seen.append([_oracle_params(l, dtype) for l in layers])
                calls["n"] = 0
                torch.cuda.synchronize()
                before = torch.cuda.memory_allocated()
                y = runner.forward(x)
                torch.cuda.synchronize()
                held = torch.cuda.memory_allocated() - before
                runner.backward(y.detach(), dout)
                del y
                runner.wait_optimizer()
                torch.cuda.synchronize()
                per_step.append(({i: t.clone() for i, t in grads.items()}, calls["n"], held))
            weights = [l.flat_param.detach().clone() for l in layers]
            masters = [o.master_param(l.flat_param) for o, l in zip(runner.optimizers, layers)]
            results[name] = (per_step, weights, runner, layers, weights_seen, masters)
    finally:
        L.K.attn_fwd = real
    off = results["offload"][2]
    # the first two inputs went to the host; the last layer's stays resident
    assert len(off._host) == 2 and all(h.is_pinned() and h.device.type == "cpu"
                                      for h in off._host)
    assert [len(c) for c in off.attn_caches] == [0, 0, 0]
    assert all(c.token is None for c in off.attn_caches)
    nbytes = xs[0].numel() * xs[0].element_size()
    for step in range(2):
        (g_ref, n_ref, held_ref), (g_off, n_off, held_off) = (results["recompute"][0][step],
                                                              results["offload"][0][step])
        assert n_ref == 3 and n_off == 3, (n_ref, n_off)
        # between the forwards the input of layer 1 lives on the host (layer 0's
        # is the caller's tensor, layer 2's stays for the backward's start)
        assert held_ref - held_off >= nbytes, (held_ref, held_off, nbytes)
        for i in range(3):
            assert torch.equal(g_off[i], g_ref[i]), (step, i)
    for a, b in zip(results["offload"][1], results["recompute"][1]):
        assert torch.equal(a, b)
    # and against the oracle: both steps' gradients and the masters after them
    per_step, _, _, layers, weights_seen, masters = results["offload"]
    _check_stack_against_oracle(layers, weights_seen, xs, douts, [g for g, _, _ in per_step],
                                masters, dtype, "offload")
    with pytest.raises(ValueError):
        StageRunner([_layer(kw, dev, param_dtype=dtype, seed=1)], offload_inputs=True)


# ------------------------------------------------------------- llama_v2 block --

@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_llama_v2_block_vs_oracle(dev, dtype):
    """torchtitan-style TransformerBlock (models/llama_v2.py:328-399):
    interleaved complex RoPE, RMSNorm eps 1e-5, GQA 2:1, causal."""
    from zorse_amd import llama_v2 as V
    args = V.ModelArgs(dim=256, n_heads=2, n_kv_heads=1, n_layers=4, vocab_size=64,
                       multiple_of=128, rope_theta=1e4)
    blk = V.TransformerBlock(2, args, generator=torch.Generator().manual_seed(5),
                             param_dtype=dtype).to(dev)
    with torch.no_grad():
        for k in ("ln1", "ln2"):
            blk.param_view(k).copy_(1 + 0.1 * torch.randn(256, generator=torch.Generator().manual_seed(6)))
    g = torch.Generator().manual_seed(8)
    x = torch.randn(1, 200, 256, generator=g).to(dtype)
    dout = torch.randn(1, 200, 256, generator=g).to(dtype)
    xg = x.to(dev).requires_grad_(True)
    out = blk(xg)
    out.backward(dout.to(dev))
    s = blk.spec
    shape = O.LayerShape(hidden=s.hidden, heads=s.heads, kv_heads=s.kv_heads, head_dim=s.head_dim,
                         ffn=s.ffn, eps=s.eps, theta=s.rope_theta)
    p = _oracle_params(blk, dtype)
    rout, rdx, rg = O.layer_fwd_bwd(x.double(), p, shape, dout.double(), rope="interleaved")
    offs = s.offsets()
    got = [("out", out, rout), ("dx", xg.grad, rdx)]
    got += [("d" + k, blk.flat_param.grad[offs[k][0]:offs[k][1]].view(rg[k].shape), rg[k])
            for k in O.PARAM_ORDER]
    if dtype == torch.float32:
        for name, a, r in got:
            assert_close(a, r, dtype, name)
        return
    lout, ldx, lg = O.layer_fwd_bwd(x, {k: v.to(dtype) for k, v in p.items()}, shape, dout,
                                    rope="interleaved", attn="flash")
    low = {"out": lout, "dx": ldx, **{"d" + k: lg[k] for k in O.PARAM_ORDER}}
    for name, a, r in got:
        assert_matched(a, r, low[name], dtype, name)
    assert_loss(out, rout, lout, dout)


def test_profiler_protocol_small(dev):
    """The layer-profiler counterpart runs its protocol end to end on a small
    layer: positive kernel times per batch size, a line fit, and the
    optimizer latency for several shard counts."""
    from zorse_amd import llama_simple as L
    from zorse_amd import profiler as P
    cfg = L.llama_config(hidden_size=256, num_attention_heads=2, intermediate_size=512)
    layer = L.Block(cfg, 0).to(dev)
    times = [P.get_compute_latency(layer, bs, 128, 256, torch.bfloat16, vocab_size=512,
                                   num_iterations=3, delay=0.0) for bs in (1, 2)]
    assert all(f > 0 and b > 0 for f, b in times)
    assert P.get_optimizer_latency(layer, 1, num_iterations=3) > 0
    assert P.get_optimizer_latency(layer, 4, num_iterations=3) > 0
    assert P.gpu_name() == "mi355x"


# ------------------------------------------------------------- HF-factory routes --

def test_hf_llama_route_vs_oracle(dev):
    """The llama_* route (models/llama.py:5-56 through models/hub.py): the
    factory's model form -- LlamaConfig defaults, FFN = 4 x hidden, HF's
    attribute layout (model.model.layers, .embed_tokens, .norm, .lm_head) --
    at a scaled shape (hidden 512, 4 heads x 128, 2 layers, vocab 1000, seq
    128, batch 2), fp32 parameters.  forward(input_ids, labels) gives HF's
    causal-LM loss (position t predicts label t + 1) through the chunked
    vocabulary head; the loss and every parameter gradient (embedding, each
    layer's nine slices, final norm, head) against the fp64 oracle of the same
    composition (fp32 bar: 1e-4 normwise; loss 1e-4 relative)."""
    from zorse_amd import hf_models as H
    from zorse_amd.llama_simple import llama_config
    cfg = llama_config(vocab_size=1000, max_position_embeddings=128, hidden_size=512,
                       num_hidden_layers=2, num_attention_heads=4, intermediate_size=4 * 512)
    torch.manual_seed(21)
    model = H.CausalLM(cfg, init_std=0.02, generator=torch.Generator().manual_seed(22))
    with torch.no_grad():   # norm weights other than one
        for l in model.model.layers:
            for ln in ("ln1", "ln2"):
                l.param_view(ln).copy_(1 + 0.1 * torch.randn(512))
        model.model.norm.weight.copy_(1 + 0.1 * torch.randn(512))
    model = model.to(dev)
    assert isinstance(H.get_layers(model), torch.nn.ModuleList) and len(model.model.layers) == 2
    g = torch.Generator().manual_seed(23)
    ids = torch.randint(0, 1000, (2, 128), generator=g)
    labels = torch.randint(0, 1000, (2, 128), generator=g)
    labels[0, 17] = -100
    out = model(ids.to(dev), labels=labels.to(dev))
    out.loss.backward()
    # the oracle, fp64 on the CPU
    emb = model.model.embed_tokens.weight.detach().double().cpu().requires_grad_(True)
    ps = [{k: v.clone().requires_grad_(True) for k, v in _oracle_params(l, torch.float32).items()}
          for l in model.model.layers]
    nw = model.model.norm.weight.detach().double().cpu().requires_grad_(True)
    hw = model.lm_head.weight.detach().double().cpu().requires_grad_(True)
    x = emb[ids]
    shape = _oracle_shape(model.model.layers[0])
    for p in ps:
        x = O.decoder_layer(x, p, shape)
    rl = O.lm_head_ce(x[:, :-1], nw, hw, labels[:, 1:], 1e-6)
    rl.backward()
    print(f"  HF llama route loss: hip {out.loss.item():.8f} fp64 {rl.item():.8f}", flush=True)
    assert abs(out.loss.item() - rl.item()) <= 1e-4 * abs(rl.item())
    assert_close(model.model.embed_tokens.weight.grad, emb.grad, torch.float32, "d embed")
    assert_close(model.model.norm.weight.grad, nw.grad, torch.float32, "d norm")
    assert_close(model.lm_head.weight.grad, hw.grad, torch.float32, "d lm_head")
    offs = model.model.layers[0].spec.offsets()
    for i, (l, p) in enumerate(zip(model.model.layers, ps)):
        for k in O.PARAM_ORDER:
            a, b = offs[k]
            assert_close(l.flat_param.grad[a:b].view(p[k].shape), p[k].grad, torch.float32,
                         f"layer {i} d{k}")
    # without labels: the logits of the same forward (hand-written GEMM head)
    with torch.no_grad():
        logits = model(ids.to(dev)).logits
        rlog = torch.nn.functional.linear(O.rmsnorm(x.detach(), nw.detach(), 1e-6), hw.detach())
    assert logits.shape == (2, 128, 1000)
    assert_close(logits, rlog, torch.float32, "logits")


def test_hf_mistral_route_layer_and_profiler_protocol(dev):
    """The mistral_* route (models/mistral.py:5-35): MistralConfig's form
    (8 KV heads, sliding window 4096, FFN as given) at a scaled shape (hidden
    512, 4 q-heads / 1 kv-head of 128, window 96, seq 160, bf16 parameters):
    a layer of model.model.layers against the oracle with the precision-matched
    bar, then the layer profiler's protocol on it (utils/runtime_estimator.py:
    187-253: forward under autocast, backward with retain_graph)."""
    from zorse_amd import hf_models as H
    from zorse_amd import profiler as P
    from zorse_amd.mistral_simple import mistral_config
    cfg = mistral_config(vocab_size=1000, max_position_embeddings=160, hidden_size=512,
                         num_hidden_layers=1, num_attention_heads=4, num_key_value_heads=1,
                         intermediate_size=1536, sliding_window=96)
    model = H.CausalLM(cfg, sliding_window=cfg.sliding_window, init_std=0.02,
                       generator=torch.Generator().manual_seed(31),
                       param_dtype=torch.bfloat16).to(dev)
    layer = H.get_layers(model)[0]
    assert layer.spec.window == 96 and layer.spec.kv_heads == 1
    g = torch.Generator().manual_seed(32)
    x = torch.randn(1, 160, 512, generator=g).to(torch.bfloat16)
    dout = torch.randn(1, 160, 512, generator=g).to(torch.bfloat16)
    _check_layer(layer, x, dout, torch.bfloat16, "HF mistral route layer")
    times = [P.get_compute_latency(layer, bs, 160, 512, torch.bfloat16, vocab_size=1000,
                                   num_iterations=3, delay=0.0) for bs in (1, 2)]
    assert all(f > 0 and b > 0 for f, b in times)


@pytest.mark.parametrize("d,dtype", [(48, torch.bfloat16), (68, torch.float16),
                                     (110, torch.bfloat16)])
def test_layer_padded_head_dims(dev, d, dtype):
    """Head dims of the smaller llama_* HF-factory models (llama_1b: 48,
    llama_2b: 68, llama_5b: 110), which the attention kernels take zero-padded
    to 64 / 128: a 4-head layer (hidden 4 d, FFN 16 d, 2 x 96 tokens, GQA 4:2
    for d = 68) against the fp64 oracle with the precision-matched bar."""
    from zorse_amd import layer as LY
    kv = 2 if d == 68 else 4
    kw = dict(hidden_size=4 * d, num_attention_heads=4, num_key_value_heads=kv,
              intermediate_size=16 * d, rope_theta=1e4)
    layer = _layer(kw, dev, param_dtype=dtype, seed=401 + d)
    assert layer.spec.head_dim == d and LY._attn_padded_dim(layer.spec, dtype) in (64, 128)
    g = torch.Generator().manual_seed(402 + d)
    x = torch.randn(2, 96, 4 * d, generator=g).to(dtype)
    dout = torch.randn(2, 96, 4 * d, generator=g).to(dtype)
    _check_layer(layer, x, dout, dtype, f"padded head dim {d}")
