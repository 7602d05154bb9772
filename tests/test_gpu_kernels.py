"""GPU parity of each kernel against the CPU oracle, through the C ABI.

Inputs are drawn on the CPU from seeded generators, rounded to the storage
dtype and copied to the GPU; the oracle runs in fp64 on the same rounded
values.  Shapes cover the vector and scalar code paths, ragged sizes, GQA,
causal / sliding-window / unmasked attention and both RoPE pairings.
"""
import math

import pytest
import torch

from oracle import decoder as O
from tests._tol import assert_close

pytestmark = pytest.mark.gpu

LOWP = (torch.bfloat16, torch.float16)
ALL = (torch.float32, torch.bfloat16, torch.float16)


def _rand(shape, dtype, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (scale * torch.randn(shape, generator=g)).to(dtype)


# ---------------------------------------------------------------- RMSNorm --

RMS_SHAPES = [(1, 256), (37, 2048), (64, 4096), (3, 100), (5, 8200), (300, 688)]


@pytest.mark.parametrize("rows,hidden", RMS_SHAPES)
@pytest.mark.parametrize("dtype", ALL)
def test_rmsnorm_fwd_bwd(dev, rows, hidden, dtype):
    from zorse_amd import kernels as K
    print(f"rmsnorm rows={rows} hidden={hidden} {dtype}", flush=True)
    x = _rand((rows, hidden), dtype, 1)
    res = _rand((rows, hidden), dtype, 2)
    w = (1 + 0.1 * torch.randn(hidden, generator=torch.Generator().manual_seed(3))).to(dtype)
    dy = _rand((rows, hidden), dtype, 4)
    for with_res in (False, True):
        y, rstd, h = K.rmsnorm_fwd(x.to(dev), w.to(dev), 1e-6,
                                   residual=res.to(dev) if with_res else None)
        href = (x.double() + res.double()).to(dtype) if with_res else x
        if with_res:
            assert torch.equal(h.cpu(), href)   # rounded residual sum: bit-exact
        ref = O.rmsnorm(href.double(), w.double(), 1e-6)
        assert_close(y, ref, dtype, "y")
        assert_close(rstd, O.rmsnorm_rstd(href.double(), 1e-6), torch.float32, "rstd")
        dres = _rand((rows, hidden), dtype, 5) if with_res else None
        dx, dw = K.rmsnorm_bwd(dy.to(dev), h, w.to(dev), rstd,
                               dres=dres.to(dev) if with_res else None)
        rdx, rdw = O.rmsnorm_bwd(dy.double(), href.double(), w.double(), 1e-6)
        if with_res:
            rdx = rdx + dres.double()
        assert_close(dx, rdx, dtype, "dx")
        assert_close(dw, rdw, dtype, "dw")


def test_rmsnorm_dw_accumulate_and_fp32_weight(dev):
    from zorse_amd import kernels as K
    x = _rand((33, 512), torch.bfloat16, 6).to(dev)
    w = torch.ones(512, dtype=torch.float32, device=dev)
    y, rstd, _ = K.rmsnorm_fwd(x, w, 1e-6)
    dy = _rand((33, 512), torch.bfloat16, 7).to(dev)
    _, dw1 = K.rmsnorm_bwd(dy, x, w, rstd)
    acc = dw1.clone()
    K.rmsnorm_bwd(dy, x, w, rstd, dw=acc, accumulate=True)
    assert torch.allclose(acc, 2 * dw1, rtol=1e-6, atol=1e-6)
    assert dw1.dtype == torch.float32


# ----------------------------------------------------------------- SwiGLU --

@pytest.mark.parametrize("rows,cols", [(64, 688), (128, 1024), (7, 13)])
@pytest.mark.parametrize("dtype", ALL)
def test_swiglu_fwd_bwd(dev, rows, cols, dtype):
    from zorse_amd import kernels as K
    print(f"swiglu rows={rows} cols={cols} {dtype}", flush=True)
    gu = _rand((rows, 2 * cols), dtype, 8, 2.0)
    dz = _rand((rows, cols), dtype, 9)
    gu_d = gu.to(dev)
    g, u = gu_d[:, :cols], gu_d[:, cols:]
    z = K.swiglu_fwd(g, u)
    gr, ur = gu[:, :cols].double(), gu[:, cols:].double()
    assert_close(z, O.swiglu(gr, ur), dtype, "z")
    dgu = torch.empty_like(gu_d)
    K.swiglu_bwd(dz.to(dev), g, u, dgu[:, :cols], dgu[:, cols:])
    rdg, rdu = O.swiglu_bwd(dz.double(), gr, ur)
    assert_close(dgu[:, :cols], rdg, dtype, "dg")
    assert_close(dgu[:, cols:], rdu, dtype, "du")


@pytest.mark.parametrize("rows,cols", [(4096, 11008), (72, 200), (64, 64), (8, 8)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_swiglu_transposed_outputs(dev, rows, cols, dtype):
    """zk_swiglu_fwd_t / zk_swiglu_bwd_t: the row-major outputs are bit-equal
    to zk_swiglu_fwd / zk_swiglu_bwd and the transposed copies are exact
    transposes (full tiles, ragged 64-tiles, the smallest shape)."""
    from zorse_amd import kernels as K
    print(f"swiglu_t rows={rows} cols={cols} {dtype}", flush=True)
    gu = _rand((rows, 2 * cols), dtype, 63, 2.0).to(dev)
    dz = _rand((rows, cols), dtype, 64).to(dev)
    g, u = gu[:, :cols], gu[:, cols:]
    z, zt = K.swiglu_fwd_t(g, u)
    assert torch.equal(z, K.swiglu_fwd(g, u))
    assert torch.equal(zt, z.t())
    dgu, ref = torch.empty_like(gu), torch.empty_like(gu)
    dgut = torch.full((2 * cols, rows), float("nan"), dtype=dtype, device=dev)
    K.swiglu_bwd_t(dz, g, u, dgu[:, :cols], dgu[:, cols:], dgut[:cols], dgut[cols:])
    K.swiglu_bwd(dz, g, u, ref[:, :cols], ref[:, cols:])
    assert torch.equal(dgu, ref)
    assert torch.equal(dgut, dgu.t())


def _assert_within_ulp(got, ref, dtype, what):
    """Every element within one unit in the last place (of the storage
    dtype, at that element's magnitude) of the exact product: one rounding
    of an fp32 sum whose order differs from the reference's."""
    g = got.double().cpu()
    r = ref.double().cpu()
    assert torch.isfinite(g).all(), what
    mant = {torch.bfloat16: 8, torch.float16: 11}[dtype]
    # the ulp at the larger of the two magnitudes (a sum just below a power
    # of two may round up across it)
    _, ex = torch.frexp(torch.maximum(r.abs(), g.abs()).clamp_min(1e-30))
    ulp = torch.ldexp(torch.ones_like(r), ex - mant)
    floor = r.abs().max().item() * 2.0 ** -20
    bad = (g - r).abs() > ulp + floor
    assert not bad.any(), (f"{what}: {int(bad.sum())} elements beyond one ulp, max err "
                           f"{(g - r).abs().max().item():.3g}")


@pytest.mark.parametrize("M,N,K,dtype,res", [(256, 256, 256, torch.bfloat16, False),
                                             (512, 768, 384, torch.bfloat16, True),
                                             (1024, 512, 1280, torch.float16, False),
                                             (768, 1024, 512, torch.float16, True),
                                             (2048, 2560, 4096, torch.bfloat16, True)])
def test_gemm_nt(dev, M, N, K, dtype, res):
    """zk_gemm_nt (hand-written MFMA GEMM, a @ b^T [+ r]) against the fp64
    product of the same rounded inputs: every element within one ulp of the
    storage dtype; grids of one to 80 tiles, K of 2 to 64 steps (the
    pipeline's prologue / tail paths), with and without the fused residual."""
    from zorse_amd import kernels as K_
    print(f"gemm_nt M={M} N={N} K={K} {dtype} residual={res}", flush=True)
    a = _rand((M, K), dtype, 81)
    b = _rand((N, K), dtype, 82, 0.05)
    r = _rand((M, N), dtype, 83) if res else None
    out = K_.gemm_nt(a.to(dev), b.to(dev), residual=r.to(dev) if res else None)
    ref = a.double() @ b.double().t()
    if res:
        ref = ref + r.double()
    _assert_within_ulp(out, ref, dtype, "gemm_nt")


def test_gemm_nt_strided_views(dev):
    """Row-strided operand views (the layer's fused weight slices), an output
    slice of a wider buffer; a shape off the tile grid runs the masked kernel."""
    from zorse_amd import kernels as K_
    M, N, K = 512, 512, 512
    a = _rand((M, K + 64), torch.bfloat16, 84)
    b = _rand((2 * N, K + 128), torch.bfloat16, 85, 0.05)
    ad, bd = a.to(dev), b.to(dev)
    wide = torch.zeros(M, N + 256, device=dev, dtype=torch.bfloat16)
    K_.gemm_nt(ad[:, 64:], bd[N:, :K], out=wide[:, 256:])
    ref = a[:, 64:].double() @ b[N:, :K].double().t()
    _assert_within_ulp(wide[:, 256:], ref, torch.bfloat16, "strided gemm_nt")
    assert torch.equal(wide[:, :256].cpu(), torch.zeros(M, 256, dtype=torch.bfloat16))
    assert not K_.gemm_nt_supported(300, 512, 512)
    out = K_.gemm_nt(ad[:300, :K], bd[:N, :K])
    _assert_within_ulp(out, a[:300, :K].double() @ b[:N, :K].double().t(), torch.bfloat16,
                       "gemm_nt 300 x 512 x 512")


def _layout_operands(M, N, Kd, dtype, a_km, b_km, seed, dev, pad=0):
    """(a, b) on the device as the layouts store them -- row-strided views of
    buffers ``pad`` columns wider -- and, on the CPU, the [M, K] / [N, K]
    matrices they hold."""
    a = _rand((Kd, M + pad) if a_km else (M, Kd + pad), dtype, seed)
    b = _rand((Kd, N + pad) if b_km else (N, Kd + pad), dtype, seed + 1, 0.05)
    ad, bd = a.to(dev), b.to(dev)
    a, ad = (a[:, :M], ad[:, :M]) if a_km else (a[:, :Kd], ad[:, :Kd])
    b, bd = (b[:, :N], bd[:, :N]) if b_km else (b[:, :Kd], bd[:, :Kd])
    am = a.t() if a_km else a
    bm = b.t() if b_km else b
    return ad, bd, am, bm


# (M, N, K): on the 256 x 256 grid (the tiled MFMA pipeline, one to 48 tiles,
# 2 to 64 K steps) and off it (the masked kernel: ragged M, N and K)
GEMM_SHAPES = [(256, 256, 256), (512, 768, 384), (768, 512, 1280), (1024, 2048, 4096),
               (300, 200, 72), (136, 520, 1000), (1, 7, 5)]


@pytest.mark.parametrize("layout", [(False, True), (True, True), (True, False), (False, False)],
                         ids=["dY_W", "dYt_X", "At_B", "X_Wt"])
@pytest.mark.parametrize("M,N,K", GEMM_SHAPES)
@pytest.mark.parametrize("dtype", ALL)
def test_gemm_layouts(dev, layout, M, N, K, dtype):
    """zk_gemm in every operand layout -- (0, 1) the input gradient dY W on W as
    stored, (1, 1) the weight gradient dY^T X on token-major activations,
    (1, 0), and (0, 0) the forward -- against the fp64 product of the same
    rounded inputs: 2-byte types every element within one ulp (one rounding
    of an fp32 sum), fp32 within 1e-5 normwise; with row-strided operand
    views and, for the 2-byte types, a fused residual."""
    from zorse_amd import kernels as K_
    a_km, b_km = layout
    print(f"gemm {M}x{N}x{K} a_kmajor={a_km} b_kmajor={b_km} {dtype}", flush=True)
    a, b, am, bm = _layout_operands(M, N, K, dtype, a_km, b_km, 91, dev, pad=8)
    res = dtype != torch.float32 and (M * N) % 2 == 0
    r = _rand((M, N), dtype, 93) if res else None
    out = K_.gemm(a, b, a_kmajor=a_km, b_kmajor=b_km, residual=r.to(dev) if res else None)
    path = K_.gemm_path(M, N, K, a.stride(0), b.stride(0), N, dtype, a_km, b_km,
                        N if res else -1)
    assert path == ("tiled" if dtype != torch.float32 and K_.gemm_nt_supported(M, N, K)
                    else "general")
    ref = am.double() @ bm.double().t()
    if res:
        ref = ref + r.double()
    if dtype == torch.float32:
        assert_close(out, ref, dtype, "gemm fp32")
    else:
        _assert_within_ulp(out, ref, dtype, f"gemm {path}")


def test_gemm_llama7b_backward_shapes(dev):
    """The 7B layer's backward products on the tiled pipeline at full size:
    the gate|up input gradient dgu W_gu (4096 x 4096 x 22016, W read as
    stored) and weight gradient dgu^T n2 (22016 x 4096 x 4096, both
    token-major), and the q|k|v weight gradient (12288 x 4096 x 4096),
    against a plain PyTorch fp64 GEMM of the same rounded inputs on the GPU."""
    from zorse_amd import kernels as K_
    g = torch.Generator(device="cpu").manual_seed(87)
    T, h, F2 = 4096, 4096, 22016
    for what, (ra, ca), (rb, cb), a_km, b_km in (
            ("dgu W_gu", (T, F2), (F2, h), False, True),
            ("dgu^T n2", (T, F2), (T, h), True, True),
            ("dqkv^T n1", (T, 12288), (T, h), True, True)):
        print(f"gemm 7B backward {what}", flush=True)
        a = torch.randn(ra, ca, generator=g).to(dev, torch.bfloat16)
        b = (0.02 * torch.randn(rb, cb, generator=g)).to(dev, torch.bfloat16)
        out = K_.gemm(a, b, a_kmajor=a_km, b_kmajor=b_km)
        am = a.t() if a_km else a
        bm = b if b_km else b.t()
        ref = torch.mm(am.double(), bm.double())
        _assert_within_ulp(out, ref, torch.bfloat16, f"gemm {what}")
        del a, b, out, ref
        torch.cuda.empty_cache()


def test_gemm_nt_llama7b_shapes(dev):
    """The 7B layer's gate|up forward (4096 x 22016 x 4096) and down_proj
    with its residual (4096 x 4096 x 11008) against a plain PyTorch fp64 GEMM
    of the same rounded inputs on the GPU."""
    from zorse_amd import kernels as K_
    g = torch.Generator(device="cpu").manual_seed(86)
    for M, N, K in ((4096, 22016, 4096), (4096, 4096, 11008)):
        print(f"gemm_nt 7B shape {M}x{N}x{K}", flush=True)
        a = torch.randn(M, K, generator=g).to(dev, torch.bfloat16)
        b = (0.02 * torch.randn(N, K, generator=g)).to(dev, torch.bfloat16)
        r = torch.randn(M, N, generator=g).to(dev, torch.bfloat16) if K != 4096 else None
        out = K_.gemm_nt(a, b, residual=r)
        ref = torch.mm(a.double(), b.double().t())
        if r is not None:
            ref += r.double()
        _assert_within_ulp(out, ref, torch.bfloat16, f"gemm_nt {M}x{N}x{K}")
        del a, b, r, out, ref


@pytest.mark.parametrize("b_km", [False, True], ids=["X_Wt", "dY_W"])
def test_gemm_half_tiles_equal_full_tiles(dev, b_km):
    """A product whose 256 x 256 tiles fill at most half the CUs runs on
    128 x 256 tiles (4096 x 2048: 128 tiles); stacked twice along M (8192 x
    2048: 256 tiles) it runs on the full tiles. Both sum every output in
    the same order, so the halves are bit-identical to the small product,
    which is within one ulp of the fp64 one."""
    from zorse_amd import kernels as K_
    M, N, Kd = 4096, 2048, 2048
    cus = K_.device_info(dev.index or 0)["num_cus"]
    print(f"gemm half tiles {M}x{N}x{Kd} b_kmajor={b_km} cus={cus}", flush=True)
    if cus < 2 * (M // 256) * (N // 256) or cus >= 2 * (2 * M // 256) * (N // 256):
        pytest.skip(f"{cus} CUs: both products take the same tile height")
    g = torch.Generator(device="cpu").manual_seed(88)
    a = torch.randn(M, Kd, generator=g).to(dev, torch.bfloat16)
    b = (0.05 * torch.randn(*((Kd, N) if b_km else (N, Kd)), generator=g)).to(dev, torch.bfloat16)
    small = K_.gemm(a, b, b_kmajor=b_km)
    big = K_.gemm(torch.cat([a, a.flip(0)]), b, b_kmajor=b_km)
    assert torch.equal(big[:M], small)
    assert torch.equal(big[M:], small.flip(0))
    ref = torch.mm(a.double(), b.double() if b_km else b.double().t())
    _assert_within_ulp(small, ref, torch.bfloat16, "gemm 128 x 256 tiles")


def _assert_z_of_gu(z, gu, F, dtype):
    """z against the SwiGLU kernel on the returned g, u: the same rounding
    points, and with the epilogue's hardware exp2 / reciprocal (the 256 x 256
    pipeline) apart in at most 1 element in 10^3, by at most two storage ulps
    (a one-ulp change of the rounded silu moves the product by up to two)."""
    from zorse_amd import kernels as K_
    ref = K_.swiglu_fwd(gu[:, :F], gu[:, F:])
    diff = z.double() - ref.double()
    ulp, tiny = {torch.bfloat16: (2.0 ** -7, 2.0 ** -133), torch.float16: (2.0 ** -10, 2.0 ** -24)}[dtype]
    _, ex = torch.frexp(torch.maximum(z.double().abs(), ref.double().abs()).clamp_min(1e-30))
    one = torch.ldexp(torch.full_like(diff, ulp), ex - 1).clamp_min(tiny)
    # (1 + 1e-12): torch.ldexp may land one double ulp off the exact power of
    # two, and a difference of exactly two storage ulps must pass
    assert (diff.abs() <= 2 * one * (1 + 1e-12)).all(), "z more than two ulps from the SwiGLU kernel"
    assert (diff != 0).sum().item() <= max(1, z.numel() // 1000), "too many z elements differ"


# B, S, K, Hq, Hkv, d, interleaved, explicit positions, dtype: the first two
# and the 200-token ones take the GEMM's RoPE epilogue, the others the product
# and the pass (off the 256 grid, rotated columns not whole 128-column blocks,
# fp32, sequences under 128 tokens)
GEMM_ROPE_CASES = [
    (2, 256, 512, 4, 2, 128, False, False, torch.bfloat16),
    (1, 512, 256, 8, 4, 64, True, True, torch.float16),
    (2, 100, 192, 4, 2, 128, False, True, torch.bfloat16),
    (2, 128, 256, 2, 1, 64, False, False, torch.bfloat16),
    (1, 64, 128, 2, 2, 64, True, False, torch.float32),
    # 64-token sequences: on the GEMM's grid, but below the epilogue's 128
    # (the product and the pass)
    (4, 64, 256, 4, 2, 64, False, True, torch.bfloat16),
    # 200-token sequences: a wave's 128 rows cross a sequence boundary
    (32, 200, 256, 4, 2, 64, False, True, torch.bfloat16),
    (32, 200, 256, 2, 1, 128, True, False, torch.float16),
]


@pytest.mark.parametrize("case", GEMM_ROPE_CASES, ids=lambda c: "-".join(str(v) for v in c))
def test_gemm_rope_equals_gemm_then_rope(dev, case):
    """zk_gemm_rope (the q|k|v projection with RoPE in the GEMM's epilogue)
    writes exactly what the product followed by the RoPE pass writes, for
    both pairings, explicit positions and the fallback shapes."""
    from zorse_amd import kernels as K
    from zorse_amd.functional import rope_tables
    B, S, Kd, Hq, Hkv, d, inter, explicit, dtype = case
    print(f"gemm_rope {case}", flush=True)
    g = torch.Generator().manual_seed(41)
    N = (Hq + 2 * Hkv) * d
    x = torch.randn(B * S, Kd, generator=g).to(dtype).to(dev)
    w = (0.05 * torch.randn(N, Kd, generator=g)).to(dtype).to(dev)
    n_pos = S + 37 if explicit else S
    pos = torch.randperm(n_pos, generator=g)[:S].to(torch.int64).to(dev) if explicit else None
    cos, sin = rope_tables(n_pos, d, 1e4, dtype, dev, inter)
    got = K.gemm_rope(x, w, seq_len=S, rot_cols=(Hq + Hkv) * d, head_dim=d, cos=cos, sin=sin,
                      positions=pos, interleaved=inter)
    ref = K.gemm(x, w)
    q = ref[:, :Hq * d].view(B, S, Hq, d)
    k = ref[:, Hq * d:(Hq + Hkv) * d].view(B, S, Hkv, d)
    K.rope_(q, k, cos, sin, positions=pos, interleaved=inter)
    torch.cuda.synchronize()
    assert torch.equal(got, ref), (got.float() - ref.float()).abs().max().item()


@pytest.mark.parametrize("M,F,K,dtype", [(200, 72, 128, torch.bfloat16), (136, 200, 192, torch.float16),
                                          (8, 8, 64, torch.bfloat16), (1024, 704, 512, torch.bfloat16),
                                          # the 256 x 256 pipeline (M % 256, F % 128, K % 128)
                                          (256, 128, 256, torch.bfloat16),
                                          (512, 384, 512, torch.float16),
                                          (1024, 640, 1280, torch.bfloat16)])
def test_gemm_swiglu(dev, M, F, K, dtype):
    """zk_gemm_swiglu (gate|up GEMM + SwiGLU epilogue) vs the fp64 oracle on
    the same rounded inputs: g, u within the bf16/fp16 bar; z bit-equal to the
    SwiGLU kernel applied to the returned g, u on the 128 x 64 kernel (ragged
    shapes), and within two ulps in at most 1 element in 10^3 on the 256 x 256
    pipeline, whose epilogue takes silu from the hardware exp2 / reciprocal;
    z^T an exact transpose; both dtypes."""
    from zorse_amd import kernels as K_
    print(f"gemm_swiglu M={M} F={F} K={K} {dtype}", flush=True)
    x = _rand((M, K), dtype, 71)
    w = _rand((2 * F, K), dtype, 72, 0.05)
    xd, wd = x.to(dev), w.to(dev)
    gu, z, zt = K_.gemm_swiglu(xd, wd[:F], wd[F:], transposed=True)
    ref = x.double() @ w.double().t()
    assert_close(gu[:, :F], ref[:, :F], dtype, "g")
    assert_close(gu[:, F:], ref[:, F:], dtype, "u")
    assert_close(z, O.swiglu(ref[:, :F].to(dtype).double(), ref[:, F:].to(dtype).double()), dtype, "z")
    if K_.gemm_nt_supported(M, 2 * F, K):
        # the 256 x 256 pipeline's epilogue: hardware exp2 / reciprocal
        _assert_z_of_gu(z, gu, F, dtype)
    else:
        # the 128 x 64 kernel: the SwiGLU kernel's IEEE form, bit for bit
        assert torch.equal(z, K_.swiglu_fwd(gu[:, :F], gu[:, F:]))
    assert torch.equal(zt, z.t())


def test_gemm_swiglu_llama7b_shape(dev):
    """The 7B layer shape (4096 tokens, F = 11008, K = 4096) against a plain
    PyTorch fp32 GEMM of the same rounded inputs; the epilogue as above."""
    from zorse_amd import kernels as K_
    M, F, K = 4096, 11008, 4096
    g = torch.Generator(device="cpu").manual_seed(73)
    x = torch.randn(M, K, generator=g).to(dev, torch.bfloat16)
    w = (0.02 * torch.randn(2 * F, K, generator=g)).to(dev, torch.bfloat16)
    gu, z = K_.gemm_swiglu(x, w[:F], w[F:])
    ref = torch.mm(x.float(), w.float().t())
    assert_close(gu, ref, torch.bfloat16, "gu")
    _assert_z_of_gu(z, gu, F, torch.bfloat16)


# ------------------------------------------------------------------- RoPE --

@pytest.mark.parametrize("heads", [(4, 2), (32, 8)])  # per-head and position-major kernels
@pytest.mark.parametrize("d,theta", [(64, 5e5), (128, 1e4), (128, 1e6)])
@pytest.mark.parametrize("dtype", ALL)
def test_rope_half(dev, d, theta, dtype, heads):
    from zorse_amd import kernels as K
    from zorse_amd.functional import rope_tables
    B, S = 2, 77
    Hq, Hkv = heads
    q = _rand((B, S, Hq, d), dtype, 10)
    k = _rand((B, S, Hkv, d), dtype, 11)
    cos, sin = rope_tables(S, d, theta, dtype, dev)
    qd, kd = q.to(dev), k.to(dev)
    K.rope_(qd, kd, cos, sin)
    c, s = O.rope_cos_sin(S, d, theta, dtype)
    rq, rk = O.apply_rope_half(q, k, c, s)   # the reference's op sequence in dtype
    if dtype in LOWP:
        assert torch.equal(qd.cpu(), rq) and torch.equal(kd.cpu(), rk)
    else:
        assert_close(qd, rq, dtype, "q")
        assert_close(kd, rk, dtype, "k")
    # inverse == gradient of the rotation (fp64 autograd on the oracle)
    gq = _rand((B, S, Hq, d), dtype, 12)
    gk = _rand((B, S, Hkv, d), dtype, 13)
    qa = q.double().requires_grad_(True)
    ka = k.double().requires_grad_(True)
    c64, s64 = c.double(), s.double()
    oq, ok = O.apply_rope_half(qa, ka, c64, s64)
    torch.autograd.backward([oq, ok], [gq.double(), gk.double()])
    gqd, gkd = gq.to(dev), gk.to(dev)
    K.rope_(gqd, gkd, cos, sin, inverse=True)
    assert_close(gqd, qa.grad, dtype, "dq")
    assert_close(gkd, ka.grad, dtype, "dk")


@pytest.mark.parametrize("dtype", ALL)
def test_rope_interleaved(dev, dtype):
    from zorse_amd import kernels as K
    from zorse_amd.functional import rope_tables
    B, S, H, d = 1, 50, 3, 64
    q = _rand((B, S, H, d), dtype, 14)
    k = _rand((B, S, 1, d), dtype, 15)
    cos, sin = rope_tables(S, d, 1e4, dtype, dev, interleaved=True)
    qd, kd = q.to(dev), k.to(dev)
    K.rope_(qd, kd, cos, sin, interleaved=True)
    rq, rk = O.apply_rope_interleaved(q.double(), k.double(), O.rope_freqs_cis(d, S, 1e4))
    assert_close(qd, rq, dtype, "q")
    assert_close(kd, rk, dtype, "k")
    K.rope_(qd, kd, cos, sin, interleaved=True, inverse=True)
    assert_close(qd, q.double(), dtype, "inverse(q)")


# -------------------------------------------------------------- attention --

ATTN_CASES = [
    # B, S, Hq, Hkv, d, causal, window, dtype
    (2, 128, 4, 4, 64, True, 0, torch.bfloat16),
    (1, 200, 8, 2, 128, True, 0, torch.float16),
    (1, 256, 4, 1, 128, True, 64, torch.bfloat16),
    (1, 333, 2, 2, 64, True, 100, torch.float16),
    (2, 64, 2, 2, 64, False, 0, torch.bfloat16),
    (1, 1, 2, 2, 128, True, 0, torch.bfloat16),
    (1, 130, 4, 2, 128, True, 1, torch.bfloat16),
    (1, 50, 2, 1, 16, True, 0, torch.float32),
    (1, 90, 4, 2, 64, True, 30, torch.float32),
    # d = 128 over many key tiles (the forward's three-stage V ring wraps)
    (2, 320, 4, 4, 128, False, 0, torch.bfloat16),
    (1, 100, 2, 1, 128, False, 0, torch.float16),
    (1, 1024, 2, 2, 128, True, 0, torch.bfloat16),
    (1, 700, 2, 2, 128, True, 200, torch.bfloat16),
]


def _ids(c):
    return "B{}S{}H{}x{}d{}{}w{}{}".format(c[0], c[1], c[2], c[3], c[4], "c" if c[5] else "n",
                                          c[6], str(c[7]).split(".")[-1])


@pytest.mark.parametrize("case", ATTN_CASES, ids=[_ids(c) for c in ATTN_CASES])
def test_attention_fwd_bwd(dev, case):
    from zorse_amd import kernels as K
    B, S, Hq, Hkv, d, causal, window, dtype = case
    print(f"attention {_ids(case)}", flush=True)
    q = _rand((B, S, Hq, d), dtype, 20)
    k = _rand((B, S, Hkv, d), dtype, 21)
    v = _rand((B, S, Hkv, d), dtype, 22)
    do = _rand((B, S, Hq, d), dtype, 23)
    o, lse = K.attn_fwd(q.to(dev), k.to(dev), v.to(dev), causal=causal, window=window)
    ro, rlse = O.attention(q.double(), k.double(), v.double(), causal, window)
    assert_close(o, ro, dtype, "o")
    assert_close(lse, rlse, torch.float32 if dtype == torch.float32 else dtype, "lse")
    dq, dk, dv = K.attn_bwd(q.to(dev), k.to(dev), v.to(dev), o, do.to(dev), lse,
                            causal=causal, window=window)
    rdq, rdk, rdv = O.attention_bwd(q.double(), k.double(), v.double(), do.double(),
                                    causal, window)
    assert_close(dq, rdq, dtype, "dq")
    assert_close(dk, rdk, dtype, "dk")
    assert_close(dv, rdv, dtype, "dv")


def test_attention_strided_qkv_views(dev):
    """q / k / v as column slices of one [T, (Hq + 2 Hkv) d] projection output
    and gradients written into the matching slices (the fused-layer layout)."""
    from zorse_amd import kernels as K
    B, S, Hq, Hkv, d = 1, 192, 4, 2, 128
    dtype = torch.bfloat16
    qkv = _rand((B * S, (Hq + 2 * Hkv) * d), dtype, 30).to(dev)
    q = qkv[:, :Hq * d].view(B, S, Hq, d)
    k = qkv[:, Hq * d:(Hq + Hkv) * d].view(B, S, Hkv, d)
    v = qkv[:, (Hq + Hkv) * d:].view(B, S, Hkv, d)
    o, lse = K.attn_fwd(q, k, v)
    ro, _ = O.attention(q.cpu().double(), k.cpu().double(), v.cpu().double())
    assert_close(o, ro, dtype, "o")
    do = _rand((B, S, Hq, d), dtype, 31).to(dev)
    dqkv = torch.full_like(qkv, float("nan"))
    dq = dqkv[:, :Hq * d].view(B, S, Hq, d)
    dk = dqkv[:, Hq * d:(Hq + Hkv) * d].view(B, S, Hkv, d)
    dv = dqkv[:, (Hq + Hkv) * d:].view(B, S, Hkv, d)
    K.attn_bwd(q, k, v, o, do, lse, dq=dq, dk=dk, dv=dv)
    rdq, rdk, rdv = O.attention_bwd(q.cpu().double(), k.cpu().double(), v.cpu().double(),
                                    do.cpu().double())
    assert_close(dq, rdq, dtype, "dq")
    assert_close(dk, rdk, dtype, "dk")
    assert_close(dv, rdv, dtype, "dv")


@pytest.mark.parametrize("dtype", ALL)
def test_flash_attention_autograd_with_rope(dev, dtype):
    from zorse_amd.functional import flash_attention
    B, S, Hq, Hkv, d, theta = 1, 96, 4, 2, 64, 1e4
    q = _rand((B, S, Hq, d), dtype, 40)
    k = _rand((B, S, Hkv, d), dtype, 41)
    v = _rand((B, S, Hkv, d), dtype, 42)
    do = _rand((B, S, Hq, d), dtype, 43)
    qd, kd, vd = (t.to(dev).requires_grad_(True) for t in (q, k, v))
    out = flash_attention(qd, kd, vd, causal=True, rope_theta=theta)
    out.backward(do.to(dev))
    qa, ka, va = (t.double().requires_grad_(True) for t in (q, k, v))
    c, s = O.rope_cos_sin(S, d, theta, dtype)
    rq, rk = O.apply_rope_half(qa, ka, c.double(), s.double())
    ro, _ = O.attention(rq, rk, va)
    ro.backward(do.double())
    assert_close(out, ro, dtype, "o")
    assert_close(qd.grad, qa.grad, dtype, "dq")
    assert_close(kd.grad, ka.grad, dtype, "dk")
    assert_close(vd.grad, va.grad, dtype, "dv")


TRANSPOSED_CASES = [
    # B, S, Hq, Hkv, d, window, rope (None / "half" / "interleaved"), dtype
    (1, 256, 4, 2, 128, 0, "half", torch.bfloat16),
    (2, 200, 4, 1, 64, 0, "interleaved", torch.float16),
    (1, 328, 2, 2, 128, 96, None, torch.bfloat16),
    (2, 64, 8, 2, 64, 0, None, torch.float16),
]


@pytest.mark.parametrize("case", TRANSPOSED_CASES, ids=lambda c: "-".join(str(v) for v in c))
def test_attention_bwd_transposed_outputs(dev, case):
    """zk_attn_bwd_rope_t: the dq / dk / dv^T written from the kernels'
    epilogues (into row slices of one [(Hq + 2 Hkv) d, B S] buffer, as the
    layer passes them) are exactly the transposes of the row-major outputs,
    which in turn equal those of the call without transposed outputs."""
    from zorse_amd import kernels as K
    from zorse_amd.functional import rope_tables
    B, S, Hq, Hkv, d, window, rope, dtype = case
    print(f"attention bwd transposed outputs {case}", flush=True)
    q = _rand((B, S, Hq, d), dtype, 70).to(dev)
    k = _rand((B, S, Hkv, d), dtype, 71).to(dev)
    v = _rand((B, S, Hkv, d), dtype, 72).to(dev)
    do = _rand((B, S, Hq, d), dtype, 73).to(dev)
    r = None
    if rope is not None:
        cos, sin = rope_tables(S, d, 1e4, dtype, dev, rope == "interleaved")
        r = (cos, sin, None, rope == "interleaved")
        K.rope_(q, k, cos, sin, interleaved=rope == "interleaved")
    o, lse = K.attn_fwd(q, k, v, causal=True, window=window)
    T, qd, kd = B * S, Hq * d, Hkv * d
    t = torch.full((qd + 2 * kd, T), float("nan"), device=dev, dtype=dtype)
    dq, dk, dv = K.attn_bwd(q, k, v, o, do, lse, causal=True, window=window, rope=r,
                            transposed=(t[:qd], t[qd:qd + kd], t[qd + kd:]))
    assert torch.equal(t[:qd], dq.reshape(T, qd).t())
    assert torch.equal(t[qd:qd + kd], dk.reshape(T, kd).t())
    assert torch.equal(t[qd + kd:], dv.reshape(T, kd).t())
    pq, pk, pv = K.attn_bwd(q, k, v, o, do, lse, causal=True, window=window, rope=r)
    assert torch.equal(dq, pq) and torch.equal(dk, pk) and torch.equal(dv, pv)


@pytest.mark.parametrize("case", TRANSPOSED_CASES, ids=lambda c: "-".join(str(v) for v in c))
def test_attention_fwd_transposed_output(dev, case):
    """zk_attn_fwd_t: the O^T written from the forward kernel's epilogue (into
    a [Hq d, B S] buffer with a wider row stride) is exactly the transpose of
    O, and O and the LSE equal those of the call without it."""
    from zorse_amd import kernels as K
    B, S, Hq, Hkv, d, window, _, dtype = case
    print(f"attention fwd transposed output {case}", flush=True)
    q = _rand((B, S, Hq, d), dtype, 74).to(dev)
    k = _rand((B, S, Hkv, d), dtype, 75).to(dev)
    v = _rand((B, S, Hkv, d), dtype, 76).to(dev)
    T, qd = B * S, Hq * d
    wide = torch.full((qd, T + 8), float("nan"), device=dev, dtype=dtype)
    o, lse = K.attn_fwd(q, k, v, causal=True, window=window, out_t=wide[:, :T])
    assert torch.equal(wide[:, :T], o.reshape(T, qd).t())
    assert torch.isnan(wide[:, T:]).all()       # nothing past the token columns
    po, plse = K.attn_fwd(q, k, v, causal=True, window=window)
    assert torch.equal(o, po) and torch.equal(lse, plse)


ROPE_BWD_CASES = [
    # B, S, Hq, Hkv, d, window, interleaved, explicit positions, dtype
    (1, 256, 4, 1, 128, 0, False, False, torch.bfloat16),
    (2, 160, 4, 2, 64, 48, False, True, torch.float16),
    (1, 200, 2, 2, 128, 0, True, False, torch.bfloat16),
    (1, 96, 4, 2, 64, 0, True, True, torch.float32),
]


@pytest.mark.parametrize("case", ROPE_BWD_CASES, ids=lambda c: "-".join(str(v) for v in c))
def test_attention_bwd_fused_inverse_rope(dev, case):
    """zk_attn_bwd_rope: the attention backward that also takes dq / dk back
    through RoPE's rotation, against the fp64 oracle's autograd through the
    rotation and the attention (so the rotation's transpose, the pairing and
    the positions are all checked), and against the unfused path (attention
    backward, then the inverse zk_rope pass) within the dtype's bar."""
    from zorse_amd import kernels as K
    from zorse_amd.functional import rope_tables
    B, S, Hq, Hkv, d, window, inter, explicit, dtype = case
    print(f"attention bwd + inverse rope {case}", flush=True)
    theta = 1e4
    g = torch.Generator().manual_seed(S + d)
    pos = (torch.randperm(S, generator=g) + 5) if explicit else None
    n_pos = int(pos.max()) + 1 if explicit else S
    cos, sin = rope_tables(n_pos, d, theta, dtype, dev, inter)
    q0 = _rand((B, S, Hq, d), dtype, 60)
    k0 = _rand((B, S, Hkv, d), dtype, 61)
    v = _rand((B, S, Hkv, d), dtype, 62)
    do = _rand((B, S, Hq, d), dtype, 63)
    q, k = q0.to(dev), k0.to(dev)
    pdev = pos.to(dev) if explicit else None
    K.rope_(q, k, cos, sin, positions=pdev, interleaved=inter)
    o, lse = K.attn_fwd(q, k, v.to(dev), causal=True, window=window)
    dq, dk, dv = K.attn_bwd(q, k, v.to(dev), o, do.to(dev), lse, causal=True, window=window,
                            rope=(cos, sin, pdev, inter))
    # unfused: attention backward, then the inverse rotation pass
    uq, uk, uv = K.attn_bwd(q, k, v.to(dev), o, do.to(dev), lse, causal=True, window=window)
    K.rope_(uq, uk, cos, sin, positions=pdev, interleaved=inter, inverse=True)
    # fp64 oracle: autograd through the same rotation (the reference's tables)
    qa, ka, va = (t.double().requires_grad_(True) for t in (q0, k0, v))
    if inter:
        fc = O.rope_freqs_cis(d, n_pos, theta)
        fc = fc[pos] if explicit else fc[:S]
        rq, rk = O.apply_rope_interleaved(qa, ka, fc)
    else:
        c, s_ = O.rope_cos_sin(S, d, theta, dtype, positions=pos)
        rq, rk = O.apply_rope_half(qa, ka, c.double(), s_.double())
    ro, _ = O.attention(rq, rk, va, True, window)
    ro.backward(do.double())
    for name, got, ref, unf in (("dq", dq, qa.grad, uq), ("dk", dk, ka.grad, uk),
                                ("dv", dv, va.grad, uv)):
        assert_close(got, ref, dtype, name)
        assert_close(got, unf.double(), dtype, name + " vs unfused")
    assert torch.equal(dv, uv)


# ------------------------------------------------------------------ AdamW --

@pytest.mark.parametrize("gdt", ALL)
@pytest.mark.parametrize("n", [1_000_003, 4096, 5])
def test_adamw_kernel_vs_oracle(dev, gdt, n):
    from zorse_amd import kernels as K
    g = torch.Generator().manual_seed(50)
    p0 = torch.randn(n, generator=g)
    m0 = 0.01 * torch.randn(n, generator=g)
    v0 = 0.001 * torch.rand(n, generator=g)
    p, m, v = p0.to(dev), m0.to(dev), v0.to(dev)
    lowp = torch.empty(n, dtype=torch.bfloat16, device=dev)
    rp, rm, rv = p0.double(), m0.double(), v0.double()
    for t in range(3, 6):
        gr = torch.randn(n, generator=g).to(gdt)
        K.adamw_step(p, gr.to(dev), m, v, lr=1e-4, beta1=0.9, beta2=0.95, eps=1e-8,
                     weight_decay=0.1, step=t, lowp_out=lowp)
        O.adamw_step(rp, gr.double(), rm, rv, t, 1e-4, 0.9, 0.95, 1e-8, 0.1)
    assert_close(p, rp, torch.float32, "p")
    assert_close(m, rm, torch.float32, "m")
    assert_close(v, rv, torch.float32, "v")
    assert torch.equal(lowp.cpu(), p.cpu().to(torch.bfloat16))


@pytest.mark.parametrize("rows,cols,gdt,ldt", [(4096, 4096, torch.bfloat16, torch.bfloat16),
                                              (72, 200, torch.float32, torch.bfloat16),
                                              (200, 136, torch.float16, torch.float16),
                                              (8, 8, torch.bfloat16, torch.bfloat16)])
def test_adamw_step_transposed_copy(dev, rows, cols, gdt, ldt):
    """zk_adamw_step_t over a shard of two matrices with transposed copies and
    a region without one, around an element range no region covers: master,
    m, v and the compute copy bit-equal to zk_adamw_step on the covered
    elements and untouched elsewhere; the transposed copies exact transposes
    (full and ragged 64 x 64 tiles)."""
    from zorse_amd import kernels as K
    print(f"adamw_t rows={rows} cols={cols} {gdt} -> {ldt}", flush=True)
    g = torch.Generator().manual_seed(52)
    a = rows * cols
    n = 2 * a + 64 + 128          # matrix, matrix, 64-element hole, 8 x 16 region
    p0 = torch.randn(n, generator=g)
    m0 = 0.01 * torch.randn(n, generator=g)
    v0 = 0.001 * torch.rand(n, generator=g)
    gr = torch.randn(n, generator=g).to(gdt).to(dev)
    hyper = dict(lr=1e-4, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1, step=4)
    p, m, v = p0.to(dev), m0.to(dev), v0.to(dev)
    low = torch.empty(n, dtype=ldt, device=dev)
    K.adamw_step(p, gr, m, v, lowp_out=low, **hyper)
    pt, mt, vt = p0.to(dev), m0.to(dev), v0.to(dev)
    lowt = torch.zeros(n, dtype=ldt, device=dev)
    t1 = torch.full((cols, rows), float("nan"), dtype=ldt, device=dev)
    t2 = torch.full((rows, cols), float("nan"), dtype=ldt, device=dev)
    regions = [(0, rows, cols, t1), (a, cols, rows, t2), (2 * a + 64, 8, 16, None)]
    K.adamw_step_t(pt, gr, mt, vt, lowt, regions, **hyper)
    cov = torch.ones(n, dtype=torch.bool, device=dev)
    cov[2 * a:2 * a + 64] = False
    for x, y, x0, what in ((p, pt, p0, "master"), (m, mt, m0, "m"), (v, vt, v0, "v")):
        assert torch.equal(x[cov], y[cov]), what
        assert torch.equal(y[~cov], x0.to(dev)[~cov]), what + " outside the regions"
    assert torch.equal(low[cov], lowt[cov])
    assert torch.equal(lowt[cov], pt[cov].to(ldt))   # the copy is the rounded master
    assert torch.equal(lowt[~cov], torch.zeros(64, dtype=ldt, device=dev))
    assert torch.equal(t1, lowt[:a].view(rows, cols).t())
    assert torch.equal(t2, lowt[a:2 * a].view(cols, rows).t())


def test_fused_adamw_matches_torch_adamw_and_adam(dev):
    from zorse_amd.optim import FusedAdam, FusedAdamW
    g = torch.Generator().manual_seed(51)
    p0 = torch.randn(10_007, generator=g)
    grads = [torch.randn(10_007, generator=g) for _ in range(4)]
    for wd, ours_cls, ref_cls in ((0.1, FusedAdamW, torch.optim.AdamW),
                                  (0.0, FusedAdam, torch.optim.Adam)):
        a = torch.nn.Parameter(p0.clone().to(dev))
        b = torch.nn.Parameter(p0.clone().double())
        kw = dict(lr=1e-3, betas=(0.9, 0.95), eps=1e-8)
        oa = ours_cls([a], weight_decay=wd, **kw) if wd else ours_cls([a], **kw)
        ob = ref_cls([b], weight_decay=wd, foreach=False, **kw)
        for gr in grads:
            a.grad = gr.to(dev)
            b.grad = gr.double()
            oa.step()
            ob.step()
        assert_close(a, b.detach(), torch.float32, f"{ours_cls.__name__}")


def test_fused_adamw_mixed_precision_master(dev):
    """bf16 parameter + bf16 grad: fp32 master, m, v updated and the rounded
    parameter written back in the same pass."""
    from zorse_amd.optim import FusedAdamW
    g = torch.Generator().manual_seed(52)
    p32 = torch.randn(4099, generator=g)
    p = torch.nn.Parameter(p32.to(torch.bfloat16).to(dev))
    opt = FusedAdamW([p], lr=1e-2, betas=(0.9, 0.95), weight_decay=0.1)
    rp = p32.to(torch.bfloat16).double()
    rm, rv = torch.zeros_like(rp), torch.zeros_like(rp)
    for t in range(1, 4):
        gr = torch.randn(4099, generator=g).to(torch.bfloat16)
        p.grad = gr.to(dev)
        opt.step()
        O.adamw_step(rp, gr.double(), rm, rv, t, 1e-2, 0.9, 0.95, 1e-8, 0.1)
    master = opt.master_param(p)
    assert master.dtype == torch.float32
    assert_close(master, rp, torch.float32, "master")
    assert torch.equal(p.detach().cpu(), master.cpu().to(torch.bfloat16))


def test_cast(dev):
    from zorse_amd import kernels as K
    x = _rand((1001,), torch.float32, 60).to(dev)
    y = torch.zeros(1001, dtype=torch.bfloat16, device=dev)
    K.cast_(x, y)
    assert torch.equal(y, x.to(torch.bfloat16))
    K.cast_(x, y, accumulate=True)
    assert torch.equal(y, (x.to(torch.bfloat16).float() + x).to(torch.bfloat16))


@pytest.mark.parametrize("dtype,rows,cols", [(torch.bfloat16, 4096, 12288), (torch.float16, 200, 72),
                                             (torch.bfloat16, 1032, 520), (torch.bfloat16, 65, 131),
                                             (torch.float32, 130, 67)])
def test_transpose(dev, dtype, rows, cols):
    """zk_transpose (the weight-gradient layout change) is an exact copy:
    both tile shapes (64 x 64 when cols > rows, 128 x 128 otherwise) with full
    tiles and ragged edges, the scalar path; also from a strided view."""
    from zorse_amd import kernels as K
    x = _rand((rows, cols), dtype, 61).to(dev)
    assert torch.equal(K.transpose(x), x.t())
    wide = _rand((rows, cols + 8), dtype, 62).to(dev)
    view = wide[:, 8:]
    out = torch.empty(cols, rows, dtype=dtype, device=dev)
    K.transpose(view, out=out)
    assert torch.equal(out, view.t())


# ------------------------------------------------------ LM head + cross-entropy --

@pytest.mark.parametrize("dtype,V,chunk", [(torch.float32, 1000, 384), (torch.bfloat16, 4096, 1024),
                                           (torch.float16, 3000, 8192), (torch.bfloat16, 1003, 256)])
def test_lm_head_cross_entropy_chunked(dev, dtype, V, chunk):
    """Chunked CE (the last stage's loss, zorse_utils/pipeline_schedule_v2.py:
    181-184) vs fp64 F.cross_entropy on full logits, with ignored (-100)
    labels, a ragged last chunk and several chunks."""
    from zorse_amd.lm_head import lm_head_cross_entropy
    g = torch.Generator().manual_seed(70)
    T, h = 96, 128
    x = torch.randn(T, h, generator=g).to(dtype)
    w = (0.05 * torch.randn(V, h, generator=g)).to(dtype)
    labels = torch.randint(0, V, (T,), generator=g)
    labels[::7] = -100
    xd = x.to(dev).requires_grad_(True)
    wd = w.to(dev).requires_grad_(True)
    loss = lm_head_cross_entropy(xd, wd, labels.to(dev), chunk=chunk)
    loss.backward()
    xr = x.double().requires_grad_(True)
    wr = w.double().requires_grad_(True)
    ref = torch.nn.functional.cross_entropy(xr @ wr.t(), labels, ignore_index=-100)
    ref.backward()
    assert abs(loss.item() - ref.item()) <= 1e-3 * max(1.0, abs(ref.item()))
    if dtype == torch.float32:
        assert abs(loss.item() - ref.item()) <= 1e-4 * abs(ref.item())
    assert_close(xd.grad, xr.grad, dtype, "dx")
    assert_close(wd.grad, wr.grad, dtype, "dW")


def test_lm_head_single_chunk_keeps_logits(dev):
    """chunk >= vocab: the forward's logits are reused by the backward (no
    recomputation); the gradients agree with the chunked path's within the
    bf16 bar against fp64, and a second backward through a retained graph
    (the kept logits already overwritten) recomputes them and gives the same
    gradients again."""
    from zorse_amd.lm_head import lm_head_cross_entropy
    g = torch.Generator().manual_seed(71)
    T, h, V = 128, 256, 2048
    x = torch.randn(T, h, generator=g).to(torch.bfloat16)
    w = (0.05 * torch.randn(V, h, generator=g)).to(torch.bfloat16)
    labels = torch.randint(0, V, (T,), generator=g)
    labels[::5] = -100
    xr = x.double().requires_grad_(True)
    wr = w.double().requires_grad_(True)
    torch.nn.functional.cross_entropy(xr @ wr.t(), labels, ignore_index=-100).backward()
    grads = []
    for chunk in (V, 512):
        xd = x.to(dev).requires_grad_(True)
        wd = w.to(dev).requires_grad_(True)
        loss = lm_head_cross_entropy(xd, wd, labels.to(dev), chunk=chunk)
        loss.backward(retain_graph=True)
        first = (xd.grad.clone(), wd.grad.clone())
        xd.grad = None
        wd.grad = None
        loss.backward()
        assert torch.equal(xd.grad, first[0]) and torch.equal(wd.grad, first[1]), chunk
        assert_close(xd.grad, xr.grad, torch.bfloat16, f"dx chunk {chunk}")
        assert_close(wd.grad, wr.grad, torch.bfloat16, f"dW chunk {chunk}")
        grads.append(first)


@pytest.mark.parametrize("nbytes,blocks", [(16, 1), (1000003, 16), (32 << 20, 16),
                                           (32 << 20, 1), (5 << 20, 64)])
def test_copy_host_round_trip(dev, nbytes, blocks):
    """zk_copy_to_host (the stage's D2H activation store, the reference's
    store_to_cpu_buffer, zorse_utils/pipeline_schedule_v2.py:127-136) lands
    every byte, ragged tails included, on a side stream."""
    from zorse_amd import kernels as K
    g = torch.Generator().manual_seed(nbytes % 997)
    src_cpu = torch.randint(0, 256, (nbytes,), generator=g, dtype=torch.uint8)
    src = src_cpu.to(dev)
    dst = torch.full((nbytes,), 7, dtype=torch.uint8, pin_memory=True)
    side = torch.cuda.Stream(device=dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        K.copy_to_host(dst, src, blocks=blocks)
    side.synchronize()
    assert torch.equal(dst, src_cpu)
    # and back (the reference's load_from_cpu_buffer, pipeline_schedule_v2.py:119-126)
    back = torch.zeros_like(src)
    with torch.cuda.stream(side):
        K.copy_from_host(back, dst, blocks=blocks)
    side.synchronize()
    assert torch.equal(back, src)
    # a bf16 view round trip, as the stage stores layer inputs
    x = torch.randn(64, 4096, generator=g).to(torch.bfloat16).to(dev)
    h = torch.empty(x.shape, dtype=x.dtype, pin_memory=True)
    K.copy_to_host(h, x, blocks=blocks)
    torch.cuda.synchronize()
    assert torch.equal(h, x.cpu())


def test_copy_to_host_rejects(dev):
    """Pageable destinations, device destinations and ranges past the end
    of an allocation are refused before any launch."""
    import ctypes
    from zorse_amd import kernels as K
    from zorse_amd._abi import lib
    src = torch.zeros(4096, dtype=torch.uint8, device=dev)
    pageable = torch.zeros(4096, dtype=torch.uint8)
    pinned = torch.zeros(4096, dtype=torch.uint8, pin_memory=True)
    L = lib()
    assert L.zk_copy_to_host(ctypes.c_void_p(pageable.data_ptr()), ctypes.c_void_p(src.data_ptr()),
                             4096, 16, None) == -1
    assert L.zk_copy_to_host(ctypes.c_void_p(src.data_ptr()), ctypes.c_void_p(src.data_ptr()),
                             4096, 16, None) == -1
    assert L.zk_copy_to_host(ctypes.c_void_p(pinned.data_ptr()), ctypes.c_void_p(src.data_ptr()),
                             8192, 16, None) == -1
    assert L.zk_copy_from_host(ctypes.c_void_p(src.data_ptr()), ctypes.c_void_p(pageable.data_ptr()),
                               4096, 16, None) == -1
    assert L.zk_copy_from_host(ctypes.c_void_p(src.data_ptr()), ctypes.c_void_p(pinned.data_ptr()),
                               8192, 16, None) == -1
    with pytest.raises(ValueError):
        K.copy_to_host(pageable, src)
    with pytest.raises(ValueError):
        K.copy_from_host(src, pageable)
    torch.cuda.synchronize()
