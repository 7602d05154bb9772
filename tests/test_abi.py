"""CPU checks of the C-ABI boundary and host logic (no kernel launches).

* libzorse_amd.so loads and exports every entry point include/zorse_amd.h
  declares, with the ctypes table matching the header;
* the library's own argument validation rejects bad input with the
  documented status codes and messages (these return before any HIP call);
* the Python wrappers reject CPU tensors and bad shapes with ValueError;
* the drop-in modules keep the reference's names and parameter counts.
"""
import ctypes
import os
import re

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "zorse_amd.h")


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(zk_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    from zorse_amd import _abi
    if not os.path.exists(_abi.LIB_PATH):
        pytest.fail("libzorse_amd.so is not built: run python -m zorse_amd.build")
    return _abi.lib()


def test_library_exports_every_declared_symbol(lib):
    from zorse_amd import _abi
    declared = _declared()
    assert declared, "no entry points parsed from the header"
    for name in declared:
        assert hasattr(lib, name), f"{name} declared in zorse_amd.h but not exported"
    assert sorted(_abi.SIGNATURES) == declared


def test_abi_version_and_error_text(lib):
    assert lib.zk_abi_version() == 4
    rc = lib.zk_rmsnorm_fwd(None, None, None, None, None, None, 4, 8, 1e-6, 7, 0, None)
    assert rc == -2  # ZK_EDTYPE
    assert b"dtype" in lib.zk_last_error()


def test_gemm_kernel_choice(lib):
    """zk_gemm_path (host-only): the 256 x 256 MFMA pipeline takes 2-byte
    shapes on its grid in every layout -- the 7B layer's forward, input- and
    weight-gradient products -- and leading dimensions whose tiles stay within
    one buffer resource (2 GiB): 256 rows of a [rows, K] operand (ld < 2^22
    elements) or 64 rows of a K-major one (ld < 2^24).  Everything else --
    ragged shapes, fp32, leading dimensions off 8 or past the bound -- runs
    the masked kernel."""
    TILED, GEN = 1, 0
    bf16, f32 = 2, 0
    path = lib.zk_gemm_path
    # (M, N, K, lda, a_kmajor, ldb, b_kmajor, ldc, ldr, dtype)
    assert path(4096, 22016, 4096, 4096, 0, 4096, 0, 22016, -1, bf16) == TILED   # gate|up fwd
    assert path(4096, 4096, 22016, 22016, 0, 4096, 1, 4096, -1, bf16) == TILED   # its dX
    assert path(22016, 4096, 4096, 22016, 1, 4096, 1, 4096, -1, bf16) == TILED   # its dW
    assert path(4096, 4096, 11008, 11008, 0, 11008, 0, 4096, 4096, bf16) == TILED  # down + r
    assert path(384, 4096, 4096, 4096, 0, 4096, 0, 4096, -1, bf16) == GEN
    assert path(4096, 4096, 4160, 4160, 0, 4160, 0, 4096, -1, bf16) == GEN
    assert path(4096, 4096, 4096, 4096, 0, 4096, 0, 4096, -1, f32) == GEN
    assert path(4096, 4096, 4096, 4100, 0, 4096, 0, 4096, -1, bf16) == GEN
    assert path(4096, 4096, 4096, 4096, 0, 4096, 0, 4096, 4100, bf16) == GEN
    # the buffer-resource bound: NT rows below 2^22, K-major rows below 2^24
    assert path(256, 256, 256, (1 << 22) - 8, 0, 256, 0, 256, -1, bf16) == TILED
    assert path(256, 256, 256, 1 << 22, 0, 256, 0, 256, -1, bf16) == GEN
    assert path(256, 256, 256, 256, 0, 1 << 22, 0, 256, -1, bf16) == GEN
    assert path(256, 256, 256, 1 << 22, 1, 256, 0, 256, -1, bf16) == TILED
    assert path(256, 256, 256, (1 << 24) - 8, 1, (1 << 24) - 8, 1, 256, -1, bf16) == TILED
    assert path(256, 256, 256, 1 << 24, 1, 256, 1, 256, -1, bf16) == GEN
    assert path(256, 256, 256, 256, 1, 1 << 24, 1, 256, -1, bf16) == GEN
    assert path(256, 256, 256, 256, 0, 256, 0, 256, -1, 9) == -2


def test_validation_codes(lib):
    from zorse_amd import _abi
    # null pointers
    assert lib.zk_rmsnorm_fwd(None, None, None, None, None, None, 4, 8, 1e-6, 2, 0, None) == -1
    # residual without h_out
    p = ctypes.c_void_p(16)
    assert lib.zk_rmsnorm_fwd(p, p, None, p, p, p, 4, 8, 1e-6, 2, 0, None) == -1
    # workspace too small
    assert lib.zk_rmsnorm_bwd(p, p, p, p, None, p, p, 0, p, 1, 64, 128, 2, 0, None) == -5
    # AdamW: step 0 and bad betas
    assert lib.zk_adamw_step(p, p, 0, p, p, None, 0, 8, 1e-3, 0.9, 0.999, 1e-8, 0.0, 0, None) == -1
    assert lib.zk_adamw_step(p, p, 0, p, p, None, 0, 8, 1e-3, 1.0, 0.999, 1e-8, 0.0, 1, None) == -1
    # attention: head_dim 96 unsupported on the MFMA path; Hq not multiple of Hkv
    d = _abi.AttnDesc(B=1, Sq=8, Skv=8, Hq=4, Hkv=4, d=96, scale=0.1, causal=1, window=0,
                      dtype=_abi.ZK_BF16)
    for f in ("q", "k", "v", "o"):
        setattr(d, f + "_sb", 8 * 4 * 96); setattr(d, f + "_ss", 4 * 96); setattr(d, f + "_sh", 96)
    assert lib.zk_attn_fwd(ctypes.byref(d), p, p, p, p, p, None) == -4
    d.d, d.Hkv = 128, 3
    assert lib.zk_attn_fwd(ctypes.byref(d), p, p, p, p, p, None) == -1
    d.Hkv, d.Sq = 4, 9
    assert lib.zk_attn_fwd(ctypes.byref(d), p, p, p, p, p, None) == -4  # causal, Sq != Skv
    # swiglu bad ld, rope odd head dim, cast bad dtype
    assert lib.zk_swiglu_fwd(p, p, 4, p, 8, 2, 8, 2, None) == -1
    assert lib.zk_rope(p, 0, 0, 0, None, 0, 0, 0, 1, 1, 1, 0, 7, p, p, 1, None, 0, 0, 2, None) == -1
    assert lib.zk_cast(p, 5, p, 0, 8, 0, None) == -2
    # transpose: ld_dst < rows, in place, zero-size is a no-op
    q = ctypes.c_void_p(32)
    assert lib.zk_transpose(p, 8, q, 4, 8, 8, 2, None) == -1
    assert lib.zk_transpose(p, 8, p, 8, 8, 8, 2, None) == -1
    assert lib.zk_transpose(None, 8, None, 8, 0, 8, 2, None) == 0
    # swiglu with transposed outputs: fp32, rows not a multiple of 8, misaligned
    assert lib.zk_swiglu_fwd_t(p, p, 16, p, 8, p, 16, 16, 8, 0, None) == -2
    assert lib.zk_swiglu_fwd_t(p, p, 16, p, 8, p, 16, 12, 8, 2, None) == -4
    assert lib.zk_swiglu_fwd_t(ctypes.c_void_p(24), p, 16, p, 8, p, 16, 16, 8, 2, None) == -3
    assert lib.zk_swiglu_bwd_t(p, 8, p, p, 16, p, p, 16, p, p, 4, 16, 8, 2, None) == -1
    assert lib.zk_swiglu_bwd_t(p, 16, p, p, 16, p, p, 16, p, p, 16, 16, 12, 1, None) == -4
    # adamw_step_t: overlapping regions, rows not a multiple of 8, too many regions
    R = _abi.AdamwRegion * 2
    regs = R(_abi.AdamwRegion(0, 8, 8, 0, None), _abi.AdamwRegion(32, 8, 8, 0, None))
    assert lib.zk_adamw_step_t(p, p, 2, p, p, p, 2, ctypes.cast(regs, ctypes.c_void_p), 2, 1024,
                               1e-3, 0.9, 0.999, 1e-8, 0.0, 1, None) == -1
    regs = R(_abi.AdamwRegion(0, 12, 8, 0, None), _abi.AdamwRegion(96, 8, 8, 0, None))
    assert lib.zk_adamw_step_t(p, p, 2, p, p, p, 2, ctypes.cast(regs, ctypes.c_void_p), 2, 1024,
                               1e-3, 0.9, 0.999, 1e-8, 0.0, 1, None) == -4
    assert lib.zk_adamw_step_t(p, p, 2, p, p, p, 2, ctypes.cast(regs, ctypes.c_void_p), 9, 1024,
                               1e-3, 0.9, 0.999, 1e-8, 0.0, 1, None) == -1
    # a region past the shard's end (n elements) is rejected before any launch
    regs = R(_abi.AdamwRegion(0, 8, 8, 0, None), _abi.AdamwRegion(64, 8, 16, 0, None))
    assert lib.zk_adamw_step_t(p, p, 2, p, p, p, 2, ctypes.cast(regs, ctypes.c_void_p), 2, 128,
                               1e-3, 0.9, 0.999, 1e-8, 0.0, 1, None) == -1
    assert b"past the shard" in lib.zk_last_error()
    # gemm_swiglu: fp32, K not a multiple of 64, misaligned x, ld_x < K
    assert lib.zk_gemm_swiglu(p, 64, p, p, 64, p, p, 8, p, 8, None, 0, 8, 8, 64, 0, None) == -2
    assert lib.zk_gemm_swiglu(p, 64, p, p, 64, p, p, 8, p, 8, None, 0, 8, 8, 32, 2, None) == -4
    assert lib.zk_gemm_swiglu(ctypes.c_void_p(24), 64, p, p, 64, p, p, 8, p, 8, None, 0, 8, 8, 64,
                              2, None) == -3
    assert lib.zk_gemm_swiglu(p, 32, p, p, 64, p, p, 8, p, 8, None, 0, 8, 8, 64, 2, None) == -1
    # gemm: bad dtype, ld below the operand's row length (a [M, K]: ld >= K; a
    # K-major [K, M]: ld >= M), null operand, an address not aligned to the
    # element size; zero-size is a no-op.  Every shape is accepted (shapes off
    # the MFMA pipeline's grid run the masked kernel), so no valid call is
    # made here: these return before any HIP call
    assert lib.zk_gemm_nt(p, 256, p, 256, p, 256, None, 0, 256, 256, 256, 7, None) == -2
    assert lib.zk_gemm_nt(p, 128, p, 256, p, 256, None, 0, 256, 256, 256, 2, None) == -1
    assert lib.zk_gemm_nt(p, 256, ctypes.c_void_p(25), 256, p, 256, None, 0, 256, 256, 256, 2,
                          None) == -3
    assert lib.zk_gemm_nt(None, 0, None, 0, None, 0, None, 0, 0, 0, 0, 2, None) == 0
    assert lib.zk_gemm(p, 200, 1, p, 256, 1, p, 256, None, 0, 256, 256, 512, 2, None) == -1
    assert lib.zk_gemm(p, 512, 0, p, 200, 1, p, 256, None, 0, 256, 256, 512, 2, None) == -1
    assert lib.zk_gemm(p, 512, 0, None, 512, 0, p, 256, None, 0, 256, 256, 512, 2, None) == -1
    assert lib.zk_gemm(ctypes.c_void_p(18), 512, 0, p, 512, 0, p, 256, None, 0, 256, 256, 512,
                       0, None) == -3
    assert lib.zk_gemm(p, 512, 0, p, 512, 0, p, 256, p, 100, 256, 256, 512, 2, None) == -1
    assert lib.zk_gemm(None, 0, 1, None, 0, 1, None, 0, None, 0, 0, 0, 64, 2, None) == 0
    # gemm_rope (a [M, K], b [N, K], c [M, N], M = tokens of whole sequences of
    # S, rotated columns whole heads within N; tables and pairing as zk_rope):
    # bad dtype, bad pairing, M not whole sequences, rotated columns not whole
    # heads or past N, null table, short table without positions, ld below
    # the row length, null operand; zero-size is a no-op
    g = lambda **kw: lib.zk_gemm_rope(*[kw.get(n, v) for n, v in zip(
        ("a", "lda", "b", "ldb", "c", "ldc", "M", "N", "K", "S", "rot", "hd", "cos", "sin",
         "npos", "pos", "pair", "dt", "st"),
        (p, 512, p, 512, p, 768, 512, 768, 512, 256, 512, 128, p, p, 256, None, 0, 2, None))])
    assert g(dt=7) == -2
    assert g(pair=3) == -1
    assert g(S=300) == -1
    assert g(rot=500) == -1 and g(rot=1024) == -1
    assert g(cos=None) == -1
    assert g(npos=100) == -1
    assert g(ldc=700) == -1 and g(lda=500) == -1
    assert g(b=None) == -1
    assert g(M=0, S=256) == 0
    assert lib.zk_gemm_nt_supported(4096, 22016, 4096) == 1
    assert lib.zk_gemm_nt_supported(4096, 22016, 4160) == 0
    assert lib.zk_gemm_nt_supported(4096, 1376, 4096) == 0
    # copy_to_host: negative size, zero size, null, block count, misaligned
    assert lib.zk_copy_to_host(p, p, -1, 16, None) == -1
    assert lib.zk_copy_to_host(None, None, 0, 16, None) == 0
    assert lib.zk_copy_to_host(None, p, 64, 16, None) == -1
    assert lib.zk_copy_to_host(p, p, 64, 0, None) == -1
    assert lib.zk_copy_to_host(ctypes.c_void_p(24), p, 64, 16, None) == -3
    assert lib.zk_copy_from_host(p, None, 64, 16, None) == -1
    assert lib.zk_copy_from_host(p, ctypes.c_void_p(24), 64, 16, None) == -3


def test_wrappers_reject_cpu_tensors():
    from zorse_amd import kernels as K
    x = torch.zeros(4, 8)
    with pytest.raises(ValueError):
        K.rmsnorm_fwd(x, torch.ones(8), 1e-6)
    with pytest.raises(ValueError):
        K.attn_fwd(torch.zeros(1, 8, 2, 64), torch.zeros(1, 8, 2, 64), torch.zeros(1, 8, 2, 64))
    with pytest.raises(ValueError):
        K.adamw_step(torch.zeros(8), torch.zeros(8), torch.zeros(8), torch.zeros(8), lr=1e-3,
                     beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.0, step=1)


def test_dropin_names_and_counts():
    from zorse_amd import llama_simple
    from oracle import decoder as O
    cfg = llama_simple.llama_config(hidden_size=64, intermediate_size=96, num_attention_heads=4,
                                    num_key_value_heads=2)
    layer = llama_simple.LlamaDecoderLayer(cfg, 0)
    params = list(layer.parameters())
    assert len(params) == 1 and params[0] is layer.flat_param
    shape = O.LayerShape(hidden=64, heads=4, kv_heads=2, head_dim=16, ffn=96)
    assert layer.flat_param.numel() == O.flat_numel(shape)
    assert layer.self_attn.q_proj.weight.shape == (64, 64)
    assert layer.self_attn.k_proj.weight.shape == (32, 64)
    assert layer.mlp.down_proj.weight.shape == (64, 96)
    assert torch.equal(layer.input_layernorm.weight, torch.ones(64))
    # views alias the flat parameter in registration order
    names = [n for n, _ in layer.orig_named_parameters()]
    assert names[0] == "self_attn.q_proj.weight" and names[-1] == "post_attention_layernorm.weight"
    flat = torch.cat([t.reshape(-1) for _, t in layer.orig_named_parameters()])
    assert torch.equal(flat, layer.flat_param.detach())
    with torch.no_grad():
        layer.self_attn.v_proj.weight.fill_(3.0)
    a, b = layer._offsets["v"]
    assert torch.all(layer.flat_param[a:b] == 3.0)
    # the 7B and tiny layers hold the reference's per-layer parameter counts
    # (data/model_stats.json:92,104), counted without allocating weights
    for name, numel in (("deepspeedllama_7b", 202_383_360), ("deepspeedllama_tiny", 51_384_320)):
        hidden, inter, _, heads = llama_simple.MODEL_SHAPES[name]
        spec = llama_simple.spec_from_config(llama_simple.llama_config(
            hidden_size=hidden, intermediate_size=inter, num_attention_heads=heads))
        assert spec.numel == numel


def test_get_model_structure():
    from zorse_amd import llama_simple
    with torch.device("meta"):
        model = llama_simple.get_model("deepspeedllama_7b", vocab_size=128, seq_length=64,
                                       layers=2, insert_noop=True)
    assert model._hidden_size == 4096
    assert len(model.layers) == 4  # Block, NoOp, Block, NoOp
    blk = model.layers[0]
    assert isinstance(blk.block, llama_simple.LlamaDecoderLayer)
    assert blk.block.flat_param.numel() == 202_383_360
    assert blk.block.spec.window == 0
    parts = model.join_layers()
    assert parts[0] is model.embed_tokens and parts[-1] is model.output_layer


def test_mistral_defaults():
    from zorse_amd import mistral_simple
    with torch.device("meta"):
        model = mistral_simple.get_model("deepspeedmistral_toy", vocab_size=128, seq_length=64,
                                         layers=1)
    spec = model.layers[0].block.spec
    assert (spec.heads, spec.kv_heads, spec.head_dim, spec.ffn) == (32, 8, 128, 14336)
    assert spec.window == 4096 and spec.causal
    assert model._hidden_size == 4096
    assert model.layers[0].block.flat_param.numel() == 218_112_000


def test_fused_adamw_validation():
    from zorse_amd.optim import FusedAdam, FusedAdamW
    p = torch.nn.Parameter(torch.zeros(4))
    with pytest.raises(ValueError):
        FusedAdamW([p], betas=(1.0, 0.9))
    with pytest.raises(ValueError):
        FusedAdam([p], weight_decay=0.1)
    opt = FusedAdamW([p], lr=1e-4, weight_decay=0.1)
    assert opt.param_groups[0]["weight_decay"] == 0.1


def test_flop_and_byte_counts_match_survey_table():
    from zorse_amd import flops
    # attention fwd FLOPs (4 B Hq d P)
    assert round(flops.attn_fwd_flops(8, 32, 128, 2048, 2048, True, 0) / 1e9, 1) == 275.0
    assert round(flops.attn_fwd_flops(1, 32, 128, 4096, 4096, True, 0) / 1e9, 1) == 137.5
    assert round(flops.attn_fwd_flops(1, 32, 128, 8192, 8192, True, 4096) / 1e9, 1) == 412.4
    # GEMM work of one 7B layer fwd+bwd (with attention): 5.455 TF
    from zorse_amd.layer import LayerSpec
    spec = LayerSpec(hidden=4096, heads=32, kv_heads=32, head_dim=128, ffn=11008)
    assert round(flops.layer_fwd_bwd_flops(spec, 1, 4096) / 1e12, 3) == 5.455
    assert flops.adamw_bytes(202_383_360, 4, False) == 28 * 202_383_360


def test_llama_v2_structure_and_ffn_rule():
    from zorse_amd import llama_v2 as V
    # FeedForward width rule (models/llama_v2.py:300-309)
    assert V.ffn_hidden_dim(V.ModelArgs(dim=4096)) == 11008
    assert V.ffn_hidden_dim(V.ModelArgs(dim=512, multiple_of=64)) == 1408
    assert V.ffn_hidden_dim(V.ModelArgs(dim=512, intermediate_size=777)) == 777
    args = V.ModelArgs(dim=64, n_heads=4, n_kv_heads=2, n_layers=2, vocab_size=32,
                       multiple_of=16)
    blk = V.TransformerBlock(1, args)
    assert blk.spec.interleaved_rope and blk.spec.eps == 1e-5 and blk.spec.kv_heads == 2
    assert blk.attention.wk.weight.shape == (32, 64)
    assert blk.feed_forward.w2.weight.shape == (64, V.ffn_hidden_dim(args))
    names = [n for n, _ in blk.orig_named_parameters()]
    assert "feed_forward.w3.weight" in names and names[-1] == "ffn_norm.weight"
    assert abs(blk.weight_init_std - 0.02 / 2.0) < 1e-12
    with torch.device("meta"):
        m = V.get_model("deepspeedllamav2_7b", vocab_size=64, seq_length=32, layers=1)
    assert m._hidden_size == 4096 and m.layers[0].flat_param.numel() == 202_383_360
    assert m.join_layers()[-1] is m.output_layer


def test_profiler_table_format_and_fit():
    """The latency-table entry written for MI355X follows
    utils/runtime_estimator.py:388-414 and reads back the way
    utils/optimizer_utils.py:59-125 reads it (profiled list per batch size,
    linear fit beyond)."""
    import json
    import tempfile
    from zorse_amd import profiler as P
    assert P.clean_gpu_name("AMD Instinct MI355X") == "mi355x"
    assert P.GPU_MEMORY["mi355x"] == 288.0 and P.GPU_TFLOPS["bfloat16"]["mi355x"] == 2516.6
    slope, icpt = P.fit_line([3.0, 5.0, 7.0, 9.0])
    assert abs(slope - 2.0) < 1e-12 and abs(icpt - 1.0) < 1e-12
    entry = [P.fit_line([1.0, 2.1, 2.9]), P.fit_line([2.0, 4.2, 5.8]), [1.0, 2.1, 2.9],
             [2.0, 4.2, 5.8]]
    with tempfile.TemporaryDirectory() as d:
        path = d + "/model_latencies.json"
        P.update_latency_table(path, "deepspeedllama_7b", "mi355x", 4096, "bfloat16", entry)
        P.update_latency_table(path, "deepspeedllama_7b", "mi355x", 512, "bfloat16", entry)
        table = json.load(open(path))
    rt = table["deepspeedllama_7b"]["mi355x"]["4096"]["bfloat16"]
    assert isinstance(rt, list) and len(rt) == 4 and rt[2][1] == 2.1 and rt[3][2] == 5.8
    (sf, i_f), (sb, ib) = rt[0], rt[1]
    assert abs((sf * 5 + i_f) - (entry[0][0] * 5 + entry[0][1])) < 1e-12
    assert set(table["deepspeedllama_7b"]["mi355x"]) == {"4096", "512"}


def test_ce_chunk_validation(lib):
    p = ctypes.c_void_p(16)
    assert lib.zk_ce_fwd_chunk(p, 4, 8, 4, p, 0, p, p, p, 2, None) == -1     # ld < cols
    assert lib.zk_ce_fwd_chunk(p, 4, 8, 8, None, 0, p, p, p, 2, None) == -1  # null labels
    assert lib.zk_ce_bwd_chunk(p, 4, 8, 8, p, 0, p, 1.0, 9, None) == -2      # bad dtype
    assert lib.zk_ce_fwd_chunk(ctypes.c_void_p(18), 4, 8, 8, p, 0, p, p, p, 2, None) == -3


def test_attention_cache_keys():
    """The recompute cache hits only for the same input storage, version and
    weights, including through detach() (how the stage runner re-feeds the
    saved input); a modified input or weight misses."""
    from zorse_amd.layer import AttentionCache
    c = AttentionCache()
    x = torch.randn(2, 8, 16)
    w = torch.zeros(32)
    o, lse = torch.ones(3), torch.zeros(3)
    c.bind(x, w, w)
    assert c.take() is None
    c.put(o, lse)
    assert len(c) == 1
    c.bind(torch.randn(2, 8, 16), w, w)             # other tensor, same shape
    assert c.take() is None
    c.bind(x.detach(), w, w)                        # same storage and version
    hit = c.take()
    assert hit is not None and hit[0] is o and hit[1] is lse and len(c) == 0
    c.bind(x, w, w)
    c.put(o, lse)
    x.add_(1.0)                                     # input modified in place
    c.bind(x, w, w)
    assert c.take() is None
    c.clear()
    c.bind(x, w, w)
    c.put(o, lse)
    torch.autograd.graph.increment_version(w)       # weights stepped
    c.bind(x, w, w)
    assert c.take() is None


def test_attention_cache_token_keys():
    """With a token set (the stage's host offload brings the input back in a
    new device buffer) the key is the token, shape and weights: another
    buffer with the same token hits, another token or stepped weights miss."""
    from zorse_amd.layer import AttentionCache
    c = AttentionCache()
    w = torch.zeros(32)
    o, lse = torch.ones(3), torch.zeros(3)
    c.token = (1, 0)
    c.bind(torch.randn(2, 8, 16), w, w)
    c.put(o, lse)
    c.bind(torch.randn(2, 8, 16), w, w)             # the input's round trip
    hit = c.take()
    assert hit is not None and hit[0] is o
    c.put(o, lse)
    c.token = (2, 0)                                # next step
    c.bind(torch.randn(2, 8, 16), w, w)
    assert c.take() is None
    c.token = (1, 0)
    c.bind(torch.randn(2, 8, 8), w, w)              # other shape
    assert c.take() is None
    torch.autograd.graph.increment_version(w)
    c.bind(torch.randn(2, 8, 16), w, w)
    assert c.take() is None


def test_bench_reads_recorded_traffic():
    """bench.py's roofline `traffic` comes from the committed rocprofv3
    summary; every kernel it reports an HBM roofline for (names with spaces
    included) must be found there."""
    import bench
    names = {
        "adamw_tile_t<bf16,bf16> (layer step with W^T copies)": 6_071_484_416,
        "adamw_elem<bf16,bf16,true>": 5_666_734_080,
        "rmsnorm_bwd_vec<bf16,bf16,256,2,2> + dw reduce": 100_683_776,
    }
    # every case the summary covers, under the label bench.py reports it with
    for label, _ in bench.TRAFFIC_CASES.values():
        names.setdefault(label, None)
    for name, algorithmic in names.items():
        t = bench.recorded_traffic(name)
        assert isinstance(t, int) and t > 0, name
        if algorithmic:
            assert 0.95 * algorithmic <= t <= 1.5 * algorithmic, (name, t)
    assert bench.recorded_traffic("no such kernel") is None


def test_fused_adamw_step_param_steps_one_parameter(monkeypatch):
    """FusedAdamW.step_param(p) (the stage runner's per-parameter hook) updates
    p alone, however many parameters of the optimizer hold gradients; step()
    updates each parameter with a gradient once.  The kernel call is replaced
    by a recorder, so this runs on the CPU."""
    from zorse_amd import optim
    calls = []

    def record(param, grad, m, v, **kw):
        calls.append((param.data_ptr(), kw["step"]))
    monkeypatch.setattr(optim.K, "adamw_step", record)
    a, b, c = (torch.nn.Parameter(torch.zeros(8)) for _ in range(3))
    opt = optim.FusedAdamW([a, b, c], lr=1e-3)
    a.grad, b.grad = torch.ones(8), torch.ones(8)
    opt.step_param(a)
    assert calls == [(a.data_ptr(), 1)]
    opt.step_param(c)                      # no gradient: nothing to do
    assert len(calls) == 1
    opt.step()
    assert calls[1:] == [(a.data_ptr(), 2), (b.data_ptr(), 1)]
    assert opt.state[a]["step"] == 2 and opt.state[b]["step"] == 1 and not opt.state[c]
    with pytest.raises(ValueError):
        opt.step_param(torch.nn.Parameter(torch.zeros(8)))


def test_attention_fwd_transposed_output_checks():
    """zk_attn_fwd_t rejects a transposed output it cannot write (before
    touching any pointer): a sequence length or row stride that is not a
    multiple of 8, a row stride below B S, fp32, a missing buffer."""
    from zorse_amd import _abi
    lib = _abi.lib()
    p = ctypes.c_void_p(256)

    def desc(S, dtype=_abi.ZK_BF16):
        d = _abi.AttnDesc(B=1, Sq=S, Skv=S, Hq=2, Hkv=2, d=64, scale=0.125, causal=1, window=0,
                          dtype=dtype)
        for f in ("q", "k", "v", "o"):
            setattr(d, f + "_sb", S * 2 * 64); setattr(d, f + "_ss", 2 * 64)
            setattr(d, f + "_sh", 64)
        return d

    def call(d, ld, o_t=p):
        return lib.zk_attn_fwd_t(ctypes.byref(d), p, p, p, p, p, o_t, ld, None)
    assert call(desc(12), 16) == -1            # S not a multiple of 8
    assert call(desc(16), 12) == -1            # ld not a multiple of 8
    assert call(desc(16), 8) == -1             # ld < B S
    assert call(desc(16), 16, o_t=None) == -1
    assert call(desc(16, _abi.ZK_F32), 16) == -4
    assert "transposed" in lib.zk_last_error().decode()


def test_attention_bwd_transposed_output_checks():
    """zk_attn_bwd_rope_t rejects transposed outputs it cannot write (before
    touching any pointer): a sequence length or row stride that is not a
    multiple of 8, a row stride below B S, fp32, a missing buffer."""
    from zorse_amd import _abi
    lib = _abi.lib()
    p = ctypes.c_void_p(256)

    def desc(S, dtype=_abi.ZK_BF16):
        d = _abi.AttnDesc(B=1, Sq=S, Skv=S, Hq=2, Hkv=2, d=64, scale=0.125, causal=1, window=0,
                          dtype=dtype)
        for f in ("q", "k", "v", "o", "dq", "dk", "dv"):
            setattr(d, f + "_sb", S * 2 * 64); setattr(d, f + "_ss", 2 * 64)
            setattr(d, f + "_sh", 64)
        return d

    def call(d, ld, dq_t=p):
        return lib.zk_attn_bwd_rope_t(ctypes.byref(d), p, p, p, p, p, p, p, p, p, p, 1 << 20,
                                      None, None, 0, None, 0, dq_t, p, p, ld, None)
    assert call(desc(12), 16) == -1            # S not a multiple of 8
    assert call(desc(16), 12) == -1            # ld not a multiple of 8
    assert call(desc(16), 8) == -1             # ld < B S
    assert call(desc(16), 16, dq_t=None) == -1
    assert call(desc(16, _abi.ZK_F32), 16) == -4
    assert "transposed" in lib.zk_last_error().decode()


def test_hf_factory_routes_structure():
    """The llama_* / mistral_* factories (models/llama.py, models/mistral.py):
    HF's attribute layout as models/hub.py reads it, the shapes the factories
    set (FFN = 4 x hidden for llama_*, MistralConfig's GQA 8 / window 4096),
    HF's parameter count, and the smaller models' head dims 48 - 110 (built on
    the meta device: no memory)."""
    from zorse_amd import hf_models as H
    from zorse_amd.llama_simple import LlamaDecoderLayer
    with torch.device("meta"):
        m = H.get_model("llama_6.7b", vocab_size=49152, seq_length=4096, layers=2)
    layers = H.get_layers(m)
    assert m._model_name == "llama_6.7b" and m._num_layers == 2 and m._hidden_size == 4096
    assert all(isinstance(l, LlamaDecoderLayer) for l in layers)
    l0 = layers[0]
    assert l0.spec.ffn == 4 * 4096 and l0.spec.kv_heads == 32 and l0.spec.window == 0
    assert l0.self_attn.q_proj.weight.shape == (4096, 4096)
    assert l0.mlp.down_proj.weight.shape == (4096, 16384)
    assert tuple(m.model.embed_tokens.weight.shape) == (49152, 4096)
    assert tuple(m.model.norm.weight.shape) == (4096,)
    assert tuple(m.lm_head.weight.shape) == (49152, 4096)
    per_layer = 4 * 4096 ** 2 + 3 * 4096 * 16384 + 2 * 4096
    assert l0.flat_param.numel() == per_layer
    total = sum(p.numel() for p in m.parameters())
    assert total == 2 * per_layer + 2 * 49152 * 4096 + 4096
    with torch.device("meta"):
        mm = H.get_model("mistral_7b", layers=1)
    s = H.get_layers(mm)[0].spec
    assert (s.kv_heads, s.window, s.ffn, s.rope_theta) == (8, 4096, 14336, 1e4)
    assert H.get_layers(mm)[0].flat_param.numel() == 218_112_000
    # the smaller llama_* models' head dims (padded around the attention kernels)
    for name, d in (("llama_1b", 48), ("llama_2b", 68), ("llama_3b", 84), ("llama_4b", 98),
                    ("llama_5b", 110)):
        with torch.device("meta"):
            ms = H.get_model(name, layers=1)
        s = H.get_layers(ms)[0].spec
        assert s.head_dim == d and s.ffn == 4 * s.hidden
    with pytest.raises(ValueError):
        H.get_model("llama_7b", layers=1)


def test_every_package_module_imports():
    """Every module of the package imports without a GPU (syntax, names)."""
    import importlib
    import zorse_amd
    pkg = os.path.dirname(zorse_amd.__file__)
    names = sorted(f[:-3] for f in os.listdir(pkg) if f.endswith(".py") and f != "__init__.py")
    assert "stage" in names and "layer" in names
    for name in names:
        importlib.import_module(f"zorse_amd.{name}")


def test_lm_head_default_chunk():
    """The LM head keeps the whole vocabulary's logits while they take at most
    1 GiB (the 7B head at 4096 tokens: 403 MB) and chunks by 8192 columns
    beyond."""
    import torch
    from zorse_amd.lm_head import SINGLE_CHUNK_BYTES, default_chunk
    assert default_chunk(4096, 49152, torch.bfloat16) == 49152
    assert default_chunk(4096, 49152, torch.float32) == 49152
    assert default_chunk(16384, 128256, torch.bfloat16) == 8192
    assert default_chunk(SINGLE_CHUNK_BYTES // 2, 1, torch.bfloat16) == 1
    assert default_chunk(SINGLE_CHUNK_BYTES // 2 + 1, 1, torch.bfloat16) == 8192
