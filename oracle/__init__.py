"""CPU oracle for the decoder-layer hot path -- TEST INFRASTRUCTURE ONLY.

This package restates, in plain PyTorch on the CPU (fp64 or fp32), the
arithmetic that benson-guo/zorse runs for one Llama / Mistral decoder layer and
for the optimizer step on a layer's flat parameter shard.  Every function cites
the reference lines it follows.

Who may use it: ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` -- and only as the checker or the timed CPU
baseline.  The product path (``zorse_amd``) never imports it and has no CPU
fallback: without the HIP library it raises.

How the oracle itself is pinned (tests/test_oracle.py):
  * RMSNorm      -- closed form; fp64 autograd for dx / dw; HF LlamaRMSNorm
                    (transformers installed here, the module the reference
                    imports at models/llama_simple.py:9); row-RMS = 1 with w = 1;
                    scale invariance.
  * RoPE         -- HF apply_rotary_pos_emb / LlamaRotaryEmbedding; per-pair norm
                    preservation; <R_m q, R_n k> depends only on m - n;
                    the interleaved form equals torch.polar complex products.
  * attention    -- torch SDPA (is_causal=True); explicit fp64 brute force on
                    tiny shapes; invariance to future / out-of-window K, V;
                    rows of P sum to one; GQA == repeat_kv-expanded MHA.
  * SwiGLU MLP   -- HF LlamaMLP; closed-form derivative vs fp64 autograd.
  * full layer   -- HF LlamaDecoderLayer (eager attention with an explicit
                    causal / sliding-window mask), fp64.
  * AdamW        -- torch.optim.AdamW(foreach=False) and torch.optim.Adam
                    (weight_decay 0); closed-form first step.
Parity of the reference's transformers-4.46.2-only behaviours (autocast dtype
promotion, non-causal eager attention with attention_mask=None) is unpinned:
that version is not installed and the reference cannot be imported here.
"""
