"""GPU parity at the BASELINE configurations' full sizes.

The fp64 CPU oracle is too slow at these sizes, so the reference here is the
same oracle code evaluated in fp32 on the GPU (plain PyTorch, autograd for
the layer gradients) on the inputs and weights the kernels saw, already
rounded to the compute dtype.  fp32 evaluation adds ~1e-6 relative error,
far below the bf16 / fp16 bar of tests/_tol.py, which these tests apply
unchanged (max|got - ref| <= 2e-2 * max(1, max|ref|)), computed on the GPU.

  * cfg2: causal attention fwd + bwd, batch 8, 32 heads x 128, seq 2048, bf16,
    on Q / K rotated by the RoPE kernel (theta 1e4);
  * cfg3: Llama-1B-shaped layer (hidden 2048, GQA 32:8, d 64, FFN 8192),
    micro-batch 4, seq 1024, fp16, then the fused AdamW step on the layer's
    flat fp32 master shard (fp32 bar: 1e-4 normwise);
  * cfg4: one Llama-2-7B layer (hidden 4096, 32 x 128, FFN 11008), seq 4096, bf16;
  * cfg5: one Mistral-7B layer (GQA 32:8, FFN 14336, sliding window 4096),
    seq 8192, bf16.
"""
import pytest
import torch

from oracle import decoder as O
from tests._tol import FP32_RTOL, LOWP_ATOL

pytestmark = pytest.mark.gpu


def _close(got, ref, dtype, what):
    """tests/_tol.assert_close, evaluated on the GPU."""
    assert got.shape == ref.shape, (what, got.shape, ref.shape)
    g, r = got.detach().float(), ref.detach().float()
    assert torch.isfinite(g).all(), f"{what}: non-finite values"
    diff = (g - r).abs().max().item()
    scale = r.abs().max().item()
    bound = FP32_RTOL * max(scale, 1e-30) if dtype == torch.float32 else LOWP_ATOL * max(1.0, scale)
    print(f"  {what}: max|diff| {diff:.3e} (max|ref| {scale:.3e}, bound {bound:.3e})", flush=True)
    assert diff <= bound, f"{what}: max|diff| {diff:.3e} > {bound:.3e}"


def _rand(shape, dtype, seed, dev):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g).to(dtype).to(dev)


def test_attention_cfg2_full_size(dev):
    from zorse_amd import kernels as K
    from zorse_amd.functional import rope_tables
    B, S, H, d = 8, 2048, 32, 128
    print("attention cfg2 full size", flush=True)
    q = _rand((B, S, H, d), torch.bfloat16, 1, dev)
    k = _rand((B, S, H, d), torch.bfloat16, 2, dev)
    v = _rand((B, S, H, d), torch.bfloat16, 3, dev)
    do = _rand((B, S, H, d), torch.bfloat16, 4, dev)
    cos, sin = rope_tables(S, d, 1e4, torch.bfloat16, dev)
    K.rope_(q, k, cos, sin)
    o, lse = K.attn_fwd(q, k, v)
    dq, dk, dv = K.attn_bwd(q, k, v, o, do, lse)
    torch.cuda.synchronize()
    with torch.no_grad():
        ro, rlse = O.attention(q.float(), k.float(), v.float(), True, 0)
        _close(o, ro, torch.bfloat16, "o")
        _close(lse, rlse, torch.bfloat16, "lse")
        del ro, rlse
        rdq, rdk, rdv = O.attention_bwd(q.float(), k.float(), v.float(), do.float(), True, 0)
    _close(dq, rdq, torch.bfloat16, "dq")
    _close(dk, rdk, torch.bfloat16, "dk")
    _close(dv, rdv, torch.bfloat16, "dv")


FULL = {
    "cfg3_1b_fp16": (dict(hidden_size=2048, num_attention_heads=32, num_key_value_heads=8,
                          intermediate_size=8192, rope_theta=5e5), None, torch.float16, (4, 1024)),
    "cfg4_7b_bf16": (dict(hidden_size=4096, num_attention_heads=32, intermediate_size=11008,
                          rope_theta=1e4), None, torch.bfloat16, (1, 4096)),
    "cfg5_mistral7b_bf16": (dict(hidden_size=4096, num_attention_heads=32, num_key_value_heads=8,
                                 intermediate_size=14336, rope_theta=1e6), 4096, torch.bfloat16,
                            (1, 8192)),
}


@pytest.mark.parametrize("name", list(FULL))
def test_layer_full_size(dev, name):
    from zorse_amd import llama_simple as L
    kw, window, dtype, (B, S) = FULL[name]
    print(f"layer {name} full size", flush=True)
    cfg = L.llama_config(**kw)
    g = torch.Generator().manual_seed(list(FULL).index(name) + 3)
    layer = L.LlamaDecoderLayer(cfg, 0, sliding_window=window, init_std=0.02, generator=g)
    with torch.no_grad():
        for ln in ("ln1", "ln2"):
            w = layer.param_view(ln)
            w.copy_(1 + 0.1 * torch.randn(w.shape, generator=g))
    layer = layer.to(device=dev, dtype=dtype)
    x = _rand((B, S, kw["hidden_size"]), dtype, 10, dev).requires_grad_(True)
    dout = _rand((B, S, kw["hidden_size"]), dtype, 11, dev)
    out = layer(x)[0]
    out.backward(dout)
    torch.cuda.synchronize()
    s = layer.spec
    shape = O.LayerShape(hidden=s.hidden, heads=s.heads, kv_heads=s.kv_heads, head_dim=s.head_dim,
                         ffn=s.ffn, eps=s.eps, theta=s.rope_theta, window=s.window)
    p = {k: layer.param_view(k).detach().float() for k in O.PARAM_ORDER}
    rout, rdx, rg = O.layer_fwd_bwd(x.detach().float(), p, shape, dout.float())
    _close(out, rout, dtype, "out")
    _close(x.grad, rdx, dtype, "dx")
    offs = s.offsets()
    for k in O.PARAM_ORDER:
        a, b = offs[k]
        _close(layer.flat_param.grad[a:b].view(rg[k].shape), rg[k], dtype, "d" + k)
    if name.startswith("cfg3"):
        # the cfg3 step: fused AdamW on the flat fp32 master shard
        from zorse_amd import kernels as K
        n = s.numel
        gm = torch.Generator().manual_seed(12)
        master = (0.02 * torch.randn(n, generator=gm)).to(dev)
        m = (1e-3 * torch.randn(n, generator=gm)).to(dev)
        v = (1e-6 * torch.rand(n, generator=gm)).to(dev)
        grad = layer.flat_param.grad.detach()
        rp, rm, rv = master.clone(), m.clone(), v.clone()
        lowp = torch.empty(n, device=dev, dtype=dtype)
        K.adamw_step(master, grad, m, v, lr=1e-4, beta1=0.9, beta2=0.95, eps=1e-8,
                     weight_decay=0.1, step=3, lowp_out=lowp)
        O.adamw_step(rp, grad.float(), rm, rv, 3, 1e-4, 0.9, 0.95, 1e-8, 0.1)
        _close(master, rp, torch.float32, "adamw master")
        _close(m, rm, torch.float32, "adamw exp_avg")
        _close(v, rv, torch.float32, "adamw exp_avg_sq")
        assert torch.equal(lowp, master.to(dtype)), "low-precision copy is not round(master)"
