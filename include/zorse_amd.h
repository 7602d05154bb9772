/*
 * zorse_amd.h -- C ABI of libzorse_amd.so, the MI355X (gfx950) kernels for the
 * Llama/Mistral decoder-layer hot path and the flat-shard AdamW step.
 *
 * Conventions shared by every entry point:
 *   - Device buffers are plain pointers; sizes and strides are int64 element
 *     counts (never bytes unless the name says so).
 *   - `stream` is a hipStream_t passed as void* (0 = the null stream).  Work is
 *     only enqueued; no entry point synchronises or allocates device memory.
 *     Workspaces are sized by the *_workspace() queries and passed in.
 *   - Return value: 0 on success, a negative ZK_E* code on a rejected argument,
 *     or a positive hipError_t from the launch.  zk_last_error() returns a
 *     thread-local message describing the last failure.  No C++ exception
 *     crosses this boundary.
 *   - dtype codes: ZK_F32, ZK_F16, ZK_BF16.  Arithmetic is fp32 inside every
 *     kernel; activations are rounded to their storage type on write.
 *
 * Each entry point names the reference code whose computation it replaces
 * (paths relative to the benson-guo/zorse tree; "HF" = transformers'
 * modeling_llama.py / modeling_mistral.py, which the reference imports).
 */
#ifndef ZORSE_AMD_H
#define ZORSE_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* zk_stream_t;

enum zk_dtype { ZK_F32 = 0, ZK_F16 = 1, ZK_BF16 = 2 };

enum zk_status {
  ZK_OK = 0,
  ZK_EINVAL = -1,       /* bad size / stride / null pointer                  */
  ZK_EDTYPE = -2,       /* unsupported dtype combination                     */
  ZK_EALIGN = -3,       /* pointer or stride not aligned for vector access   */
  ZK_EUNSUPPORTED = -4, /* valid but not implemented (e.g. head_dim 96)      */
  ZK_EWORKSPACE = -5    /* workspace too small                               */
};

/* Thread-local text of the last error (empty string if none). */
const char* zk_last_error(void);

/* ABI version; bumped whenever a signature below changes. */
int zk_abi_version(void);

/* Device facts used for roofline denominators.  arch receives e.g. "gfx950". */
int zk_device_info(int device, char* arch, int arch_len, int* num_cus,
                   int* max_clock_khz, int64_t* hbm_bytes);

/* ---------------------------------------------------------------- RMSNorm --
 * Replaces HF LlamaRMSNorm / MistralRMSNorm.forward as used by the decoder
 * layer (models/llama_simple.py:419-422, 458, 475; models/mistral_simple.py:82)
 * and the torchtitan RMSNorm (models/llama_v2.py:24-51):
 *     h   = x (+ residual)                       rounded to act dtype
 *     r   = rsqrt(mean(h^2) + eps)               fp32, stored in rstd[rows]
 *     y   = w * round_act(h * r)                 rounded to act dtype
 * When residual != NULL the residual add of models/llama_simple.py:471 is
 * fused in and h is written to h_out.  x, residual, h_out, y: [rows, hidden]
 * contiguous, act dtype; w: [hidden] in w_dtype.
 */
int zk_rmsnorm_fwd(const void* x, const void* residual, void* h_out,
                   const void* w, void* y, float* rstd, int64_t rows,
                   int64_t hidden, float eps, int act_dtype, int w_dtype,
                   zk_stream_t stream);

/* fp32 elements of workspace zk_rmsnorm_bwd needs for (rows, hidden). */
int64_t zk_rmsnorm_bwd_workspace(int64_t rows, int64_t hidden);

/* Backward of zk_rmsnorm_fwd (autograd of the same reference lines):
 *     g  = dy * w ;  xh = h * r
 *     dx = r * (g - xh * mean(g * xh))  (+ dres when dres != NULL)
 *     dw = sum_rows dy * round_act(xh)   (written to dw in w_dtype, or added
 *                                          to it when accumulate != 0)
 * h is the normalised input (the fwd's h_out, or x when no residual). */
int zk_rmsnorm_bwd(const void* dy, const void* h, const void* w,
                   const float* rstd, const void* dres, void* dx, void* dw,
                   int accumulate, float* workspace, int64_t workspace_elems,
                   int64_t rows, int64_t hidden, int act_dtype, int w_dtype,
                   zk_stream_t stream);

/* zk_rmsnorm_bwd without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid allocation).  No counterpart in the reference.  The
 * dw partial rows go to a static device array of
 * ZK_RMSNORM_BWD_SCRATCH_FLOATS floats (16 MiB) that each GPU the library
 * runs on holds until the process ends; its address is looked up on the
 * first call on a device, which must be the current device (the stream must
 * belong to it).  That lookup is not an operation a graph can capture: make
 * one call on each device before capturing later ones (the calls themselves
 * launch kernels only, no memset or copy).  The entry point allocates
 * nothing.  (rows, hidden) whose
 * zk_rmsnorm_bwd_workspace() exceeds the array are rejected with
 * ZK_EWORKSPACE (any rows at hidden <= 8192: at most 512 partial rows).
 * Every call on a GPU shares that GPU's array: calls that overlap on one GPU
 * (different streams, or concurrent host threads) race and must be
 * serialised by the caller.  Results are identical to zk_rmsnorm_bwd's. */
#define ZK_RMSNORM_BWD_SCRATCH_FLOATS ((int64_t)4 << 20)
int zk_rmsnorm_bwd_noalloc(const void* dy, const void* h, const void* w,
                           const float* rstd, const void* dres, void* dx,
                           void* dw, int accumulate, int64_t rows,
                           int64_t hidden, int act_dtype, int w_dtype,
                           zk_stream_t stream);

/* ----------------------------------------------------------------- SwiGLU --
 * Replaces the activation of HF LlamaMLP.forward, act_fn(gate(x)) * up(x)
 * (imported at models/llama_simple.py:10, built at :418; torchtitan
 * FeedForward.forward, models/llama_v2.py:319-320):
 *     z = round(round(silu(g)) * u)
 * g = gate[r, c], u = up[r, c] read with row stride ld_in (so gate and up can
 * be the two halves of one [rows, 2F] GEMM output); z has row stride ld_z. */
int zk_swiglu_fwd(const void* gate, const void* up, int64_t ld_in, void* z,
                  int64_t ld_z, int64_t rows, int64_t cols, int dtype,
                  zk_stream_t stream);

/* Backward: s = silu(g), sg = sigmoid(g)
 *     dup   = dz * round(s)
 *     dgate = round(dz * u) * sg * (1 + g * (1 - sg))
 * dgate / dup share row stride ld_out (halves of one [rows, 2F] buffer). */
int zk_swiglu_bwd(const void* dz, int64_t ld_dz, const void* gate,
                  const void* up, int64_t ld_in, void* dgate, void* dup,
                  int64_t ld_out, int64_t rows, int64_t cols, int dtype,
                  zk_stream_t stream);

/* The same two passes with a transposed copy of the result, for the
 * token-contiguous weight-gradient GEMMs that follow (down_proj's
 * grad_weight = grad_output^T @ z and gate/up's = grad^T @ x, the nn.Linear
 * backward of the LlamaMLP built at models/llama_simple.py:418): besides z the forward
 * writes zt[c][r] = z[r][c] (row stride ld_zt >= rows); besides dgate / dup
 * the backward writes dgate_t[c][r] and dup_t[c][r] (row stride ld_t).
 * 2-byte dtypes; rows, cols and every leading dimension multiples of 8;
 * operands 16-byte aligned (ZK_EUNSUPPORTED / ZK_EALIGN otherwise). */
int zk_swiglu_fwd_t(const void* gate, const void* up, int64_t ld_in, void* z,
                    int64_t ld_z, void* zt, int64_t ld_zt, int64_t rows,
                    int64_t cols, int dtype, zk_stream_t stream);
int zk_swiglu_bwd_t(const void* dz, int64_t ld_dz, const void* gate,
                    const void* up, int64_t ld_in, void* dgate, void* dup,
                    int64_t ld_out, void* dgate_t, void* dup_t, int64_t ld_t,
                    int64_t rows, int64_t cols, int dtype, zk_stream_t stream);

/* gate|up projection with the SwiGLU epilogue: replaces gate_proj(x),
 * up_proj(x) and act_fn(gate) * up of HF LlamaMLP.forward (the MLP built at
 * models/llama_simple.py:418; torchtitan FeedForward.forward,
 * models/llama_v2.py:319-320) -- two nn.Linear GEMMs and the activation.
 *     g = x Wg^T, u = x Wu^T (fp32 accumulation, rounded), z = round(round(silu(g)) * u)
 * x [M, K] (row stride ld_x), w_gate / w_up [F, K] (row stride ld_w; the two
 * halves of the flat gate|up weight), g_out / u_out [M, F] (shared row stride
 * ld_gu: the halves of one [M, 2F] buffer kept for the backward), z [M, F]
 * (ld_z), optional zt [F, M] = z^T (ld_zt; NULL to skip).  2-byte dtypes,
 * K a multiple of 64, M and F multiples of 8, 16-byte aligned operands. */
int zk_gemm_swiglu(const void* x, int64_t ld_x, const void* w_gate,
                   const void* w_up, int64_t ld_w, void* g_out, void* u_out,
                   int64_t ld_gu, void* z, int64_t ld_z, void* zt, int64_t ld_zt,
                   int64_t M, int64_t F, int64_t K, int dtype, zk_stream_t stream);

/* Projection GEMM: replaces the nn.Linear products of the decoder layer's
 * q/k/v/o projections (models/llama_simple.py:206-221, 346, 375) and of the
 * LlamaMLP built at models/llama_simple.py:418 -- forward, and the input and
 * weight gradients autograd forms for them in the backward the profiler
 * times (utils/runtime_estimator.py:235-243) and the pipeline runs
 * (zorse_utils/pipeline_schedule_v2.py:171-200):
 *     c[M, N] = op(a) op(b)^T (+ r[M, N])
 * a_kmajor == 0: a is [M, K] (row stride lda, contiguous along K);
 * a_kmajor != 0: a is [K, M] (row stride lda, contiguous along M); likewise
 * b ([N, K] or [K, N]).  The forward x W^T is (0, 0); the input gradient
 * dY W is (0, 1) on W as stored; the weight gradient dY^T X is (1, 1) on the
 * token-major activations as stored.  r, when not NULL, is the residual of a
 * fused add: one fp32 rounding of the accumulated product plus r.  Any
 * shape; bf16 / fp16 (fp32 accumulation) or fp32; every tensor shares
 * `dtype`; pointers aligned to the element size.  Shapes on the 256 x 256
 * grid of 2-byte types (zk_gemm_path) run the MFMA pipeline, the rest a
 * masked 128 x 128 kernel. */
int zk_gemm(const void* a, int64_t lda, int a_kmajor, const void* b, int64_t ldb,
            int b_kmajor, void* c, int64_t ldc, const void* r, int64_t ldr, int64_t M,
            int64_t N, int64_t K, int dtype, zk_stream_t stream);

/* Which kernel zk_gemm runs for a launch with 16-byte aligned pointers
 * (host-only, no GPU call): ZK_GEMM_TILED -- 2-byte type, M and N multiples
 * of 256, K a multiple of 128 and at least 256, leading dimensions multiples
 * of 8, and each operand's tile within one buffer resource (lda / ldb below
 * 2^22 elements for a [rows, K] operand, 2^24 for a K-major one); otherwise
 * ZK_GEMM_GENERAL.  ldr < 0: no residual. */
enum zk_gemm_kernel { ZK_GEMM_GENERAL = 0, ZK_GEMM_TILED = 1 };
int zk_gemm_path(int64_t M, int64_t N, int64_t K, int64_t lda, int a_kmajor, int64_t ldb,
                 int b_kmajor, int64_t ldc, int64_t ldr, int dtype);

/* zk_gemm with both operands contiguous along the reduction (a [M, K],
 * b [N, K]): the nn.Linear forward x W^T of the projections above
 * (models/llama_simple.py:206-221, 418).  zk_gemm_nt_supported(M, N, K)
 * says whether the shape is on the MFMA pipeline's grid (M, N multiples of
 * 256, K a multiple of 128 and at least 256); other shapes run too. */
int zk_gemm_nt_supported(int64_t M, int64_t N, int64_t K);
int zk_gemm_nt(const void* a, int64_t lda, const void* b, int64_t ldb, void* c,
               int64_t ldc, const void* r, int64_t ldr, int64_t M, int64_t N,
               int64_t K, int dtype, zk_stream_t stream);

/* ------------------------------------------------------------------- RoPE --
 * Replaces apply_rotary_pos_emb / rotate_half (models/llama_simple.py:27-58,
 * HF-style half-split pairing, per-op rounding in the act dtype) and
 * apply_rotary_emb (models/llama_v2.py:151-177, interleaved complex pairing
 * in fp32).  Rotates q [B,S,Hq,d] and k [B,S,Hkv,d] IN PLACE (element strides
 * per batch / seq / head; d contiguous).  cos/sin: fp32 tables [n_pos, d/2]
 * holding the reference's values (already rounded to the act dtype for the
 * half-split pairing, as models/llama_simple.py:137 does).  positions: int64
 * [S] row index into the tables, or NULL for 0..S-1.  inverse != 0 applies
 * the transpose rotation (the backward of the forward rotation).
 * k may be NULL (rotate q only). */
enum zk_rope_pairing { ZK_ROPE_HALF = 0, ZK_ROPE_INTERLEAVED = 1 };
int zk_rope(void* q, int64_t q_sb, int64_t q_ss, int64_t q_sh, void* k,
            int64_t k_sb, int64_t k_ss, int64_t k_sh, int64_t B, int64_t S,
            int64_t Hq, int64_t Hkv, int64_t d, const float* cos,
            const float* sin, int64_t n_pos, const int64_t* positions,
            int pairing, int inverse, int dtype, zk_stream_t stream);

/* The q|k|v projection with the rotary embedding fused: c = a b^T (the
 * zk_gemm_nt product: a [M, K], b [N, K], c [M, N] with row strides lda /
 * ldb / ldc) with the forward rotation applied to its first rot_cols columns
 * -- the q and k heads of the fused projection, heads of head_dim columns --
 * exactly as zk_rope would rotate the stored product (the product rounded to
 * the storage type first, then rotate_half's per-op rounding or the
 * interleaved pairing's one rounding): the nn.Linear q_proj / k_proj of
 * models/llama_simple.py:206-221 followed by apply_rotary_pos_emb
 * (models/llama_simple.py:27-58) or apply_rotary_emb (models/llama_v2.py:
 * 151-177).  Rows are tokens b S + s (M a multiple of S); positions, tables
 * and pairing as for zk_rope.  bf16 / fp16 products on the 256 x 256 grid
 * with head_dim 64 / 128, rot_cols a multiple of 128, S in [128, 2^30) and
 * fewer than 2^24 table positions rotate in the GEMM's epilogue; other
 * launches run zk_gemm then zk_rope (same result). */
int zk_gemm_rope(const void* a, int64_t lda, const void* b, int64_t ldb, void* c,
                 int64_t ldc, int64_t M, int64_t N, int64_t K, int64_t S,
                 int64_t rot_cols, int64_t head_dim, const float* cos,
                 const float* sin, int64_t n_pos, const int64_t* positions,
                 int pairing, int dtype, zk_stream_t stream);

/* -------------------------------------------------------------- Attention --
 * Replaces the attention core of the decoder layer: softmax(Q K^T * scale +
 * mask) V with GQA (repeat_kv never materialised: kv head = q head / n_rep)
 * -- models/llama_simple.py:320-342 (eager), the FA2/SDPA classes it selects
 * at :376-416, models/llama_v2.py:265-273 (SDPA is_causal=True) and HF
 * MistralAttention (sliding window).  Mask: causal keeps key j <= query i;
 * window > 0 additionally keeps only j > i - window (W keys including self).
 * Q/K/V/O are [B, S, H, d] with element strides per batch / seq / head and
 * d contiguous.  lse: fp32 [B, Hq, Sq] natural-log row logsumexp of the
 * scaled, masked scores (saved for the backward). */
typedef struct zk_attn_desc {
  int64_t B, Sq, Skv, Hq, Hkv, d;
  int64_t q_sb, q_ss, q_sh;
  int64_t k_sb, k_ss, k_sh;
  int64_t v_sb, v_ss, v_sh;
  int64_t o_sb, o_ss, o_sh;   /* O and dO (forward output / its gradient) */
  int64_t dq_sb, dq_ss, dq_sh;
  int64_t dk_sb, dk_ss, dk_sh;
  int64_t dv_sb, dv_ss, dv_sh;
  float scale;
  int causal;
  int64_t window;             /* 0 = unlimited */
  int dtype;                  /* ZK_BF16, ZK_F16 (MFMA) or ZK_F32 */
} zk_attn_desc;

int zk_attn_fwd(const zk_attn_desc* desc, const void* q, const void* k,
                const void* v, void* o, float* lse, zk_stream_t stream);

/* zk_attn_fwd that also stores O transposed: o_t [Hq d, B Sq] (row = head * d
 * + i, column = batch * Sq + position, rows ld_t elements apart), the same
 * rounded values as o -- the X^T operand of the o_proj weight gradient (the
 * backward of nn.Linear o_proj, models/llama_simple.py:221, 293-295), written
 * from the attention kernel's epilogue instead of by a separate transpose of
 * its output.  bf16 / fp16 only; Sq and ld_t multiples of 8, ld_t >= B * Sq,
 * o_t 16-byte aligned. */
int zk_attn_fwd_t(const zk_attn_desc* desc, const void* q, const void* k,
                  const void* v, void* o, float* lse, void* o_t, int64_t ld_t,
                  zk_stream_t stream);

/* Bytes of workspace zk_attn_bwd needs: the fp32 row deltas rowsum(dO o O)
 * and the log2-domain LSE, [B, Hq, Sq] each. */
int64_t zk_attn_bwd_workspace(const zk_attn_desc* desc);

/* Backward (FlashAttention-2 recomputation from lse): writes dq, dk, dv
 * (overwrites, no accumulation) in the layout given by the dq/dk/dv strides;
 * dO uses the o strides. */
int zk_attn_bwd(const zk_attn_desc* desc, const void* q, const void* k,
                const void* v, const void* o, const void* dout,
                const float* lse, void* dq, void* dk, void* dv,
                void* workspace, int64_t workspace_bytes, zk_stream_t stream);

/* zk_attn_bwd for Q / K that the forward rotated with RoPE: dq and dk are
 * stored already taken back through the rotation (its transpose), i.e. they
 * are the gradients with respect to the un-rotated q and k -- the backward of
 * apply_rotary_pos_emb (models/llama_simple.py:34-58, half-split pairing) or
 * apply_rotary_emb (models/llama_v2.py:151-177, interleaved pairing) fused
 * into the attention backward.  cos / sin, n_pos, positions and pairing as
 * for zk_rope (the tables the forward rotation used; positions NULL means
 * 0 .. S-1, which needs n_pos >= Sq).  Needs Sq == Skv. */
int zk_attn_bwd_rope(const zk_attn_desc* desc, const void* q, const void* k,
                     const void* v, const void* o, const void* dout,
                     const float* lse, void* dq, void* dk, void* dv,
                     void* workspace, int64_t workspace_bytes,
                     const float* cos, const float* sin, int64_t n_pos,
                     const int64_t* positions, int pairing, zk_stream_t stream);

/* zk_attn_bwd_rope (or, with cos == sin == NULL, zk_attn_bwd) that also
 * stores dq, dk, dv transposed: dq_t [Hq d, B Sq], dk_t / dv_t [Hkv d, B Skv]
 * (row = head * d + i, column = batch * S + position, rows ld_t elements
 * apart) -- the dY^T operand of the q / k / v projections' weight gradients
 * (the backward of the nn.Linear q_proj / k_proj / v_proj,
 * models/llama_simple.py:206-221), written from the attention kernels'
 * epilogues instead of by a separate transpose of their output.  bf16 / fp16
 * only; Sq, Skv and ld_t multiples of 8, ld_t >= B * S, 16-byte aligned. */
int zk_attn_bwd_rope_t(const zk_attn_desc* desc, const void* q, const void* k,
                       const void* v, const void* o, const void* dout,
                       const float* lse, void* dq, void* dk, void* dv,
                       void* workspace, int64_t workspace_bytes,
                       const float* cos, const float* sin, int64_t n_pos,
                       const int64_t* positions, int pairing, void* dq_t, void* dk_t,
                       void* dv_t, int64_t ld_t, zk_stream_t stream);

/* ------------------------------------------------------------------ AdamW --
 * Replaces torch.optim.Adam(fused=True).step() on the layer's flat fp32
 * parameter shard as run in the reduce-grad callback
 * (zorse_utils/pipeline.py:176-179, utils/patch.py:115-138), with decoupled
 * weight decay (torch.optim.AdamW semantics; weight_decay 0 == Adam):
 *     p <- p * (1 - lr*wd)
 *     m <- m + (1-b1) (g - m)         v <- b2 v + (1-b2) g^2
 *     p <- p - lr/(1-b1^t) * m / (sqrt(v)/sqrt(1-b2^t) + eps)
 * g is read in grad_dtype and widened to fp32 (the cast of utils/patch.py:
 * 115-119 fused in).  When param_lowp != NULL the updated parameter is also
 * written rounded to lowp_dtype (the compute copy).  n elements, step t >= 1.
 */
int zk_adamw_step(float* param, const void* grad, int grad_dtype,
                  float* exp_avg, float* exp_avg_sq, void* param_lowp,
                  int lowp_dtype, int64_t n, double lr, double beta1,
                  double beta2, double eps, double weight_decay, int64_t step,
                  zk_stream_t stream);

/* The same update over a shard given as up to 8 row-major [rows, cols]
 * regions (element offset into the shard; in increasing order, not
 * overlapping; elements outside every region are not touched), in one
 * launch.  param_lowp (bf16 / fp16) receives the rounded update as in
 * zk_adamw_step; a region with lowp_t != NULL also receives it transposed,
 * lowp_t[c][r] (row stride ld_t >= rows): the weight layout the input-gradient
 * GEMM of the layer's backward reads along its reduction (grad_input =
 * grad_output @ W of the nn.Linear projections, models/llama_simple.py:
 * 206-221, 293-295, 368 and the MLP at :418), kept current by the optimizer
 * step that already rewrites the compute copy.  Offsets, rows, cols, ld_t
 * multiples of 8; 16-byte aligned buffers; n = the shard's element count
 * (param, grad, exp_avg, exp_avg_sq and param_lowp each hold n elements):
 * a region that ends past n is rejected (ZK_EINVAL). */
typedef struct zk_adamw_region {
  int64_t offset, rows, cols, ld_t;
  void* lowp_t;
} zk_adamw_region;
int zk_adamw_step_t(float* param, const void* grad, int grad_dtype,
                    float* exp_avg, float* exp_avg_sq, void* param_lowp,
                    int lowp_dtype, const zk_adamw_region* regions, int n_regions,
                    int64_t n, double lr, double beta1, double beta2, double eps,
                    double weight_decay, int64_t step, zk_stream_t stream);

/* ------------------------------------------------- LM head cross-entropy --
 * Replaces the last stage's loss, F.cross_entropy(out.flatten(0, 1),
 * target.flatten(0, 1)) (zorse_utils/pipeline_schedule_v2.py:181-184) over
 * the logits of the output layer (models/llama_simple.py:559-561), computed
 * one vocabulary chunk at a time so [tokens, vocab] logits never exist.
 * logits: [rows, cols] chunk (row stride ld) holding vocabulary columns
 * col0 .. col0 + cols - 1; labels: int64 [rows], negative = ignored.
 * zk_ce_fwd_chunk folds the chunk into the running fp32 max / sum-of-exp per
 * row (run_max starts at -inf, run_sum at 0) and stores the label's logit in
 * target_logit when the label is inside the chunk; after the last chunk
 * lse = run_max + log(run_sum) and loss_row = lse - target_logit.
 * zk_ce_bwd_chunk overwrites the chunk with
 * scale * (exp(logit - lse) - [column == label]) (0 for ignored rows). */
int zk_ce_fwd_chunk(const void* logits, int64_t rows, int64_t cols, int64_t ld,
                    const int64_t* labels, int64_t col0, float* run_max,
                    float* run_sum, float* target_logit, int dtype,
                    zk_stream_t stream);
int zk_ce_bwd_chunk(void* logits, int64_t rows, int64_t cols, int64_t ld,
                    const int64_t* labels, int64_t col0, const float* lse,
                    float scale, int dtype, zk_stream_t stream);

/* ------------------------------------------------------------- Utilities --
 * Dtype conversion of a contiguous buffer (the autocast weight cast and the
 * grad cast of utils/patch.py:115-119 when done outside the AdamW kernel).
 * y = round(x); when accumulate != 0, y = round(y + x). */
int zk_cast(const void* x, int x_dtype, void* y, int y_dtype, int64_t n,
            int accumulate, zk_stream_t stream);

/* 2-D transpose, dst[c][r] = src[r][c] for r < rows, c < cols (row strides
 * ld_src >= cols, ld_dst >= rows, elements).  Stands in for the layout the
 * reference's autograd gives nn.Linear's weight gradient
 * (grad_weight = grad_output^T @ input, models/llama_simple.py:206-221,
 * 293-295, 368 and the MLP projections): the backward materialises
 * grad_output^T so that GEMM reduces over contiguous tokens. */
int zk_transpose(const void* src, int64_t ld_src, void* dst, int64_t ld_dst,
                 int64_t rows, int64_t cols, int dtype, zk_stream_t stream);

/* Device -> pinned-host copy of `bytes` bytes (host_dst from hipHostMalloc,
 * both pointers 16-byte aligned, the host range inside its allocation, the
 * device range the caller's to bound; ZK_EINVAL / ZK_EALIGN otherwise),
 * issued from at most `blocks` workgroups
 * so that it leaves the CUs to the compute it overlaps.  Replaces the
 * activation store of the reference's pipeline schedule,
 * zorse_utils/pipeline_schedule_v2.py:127-136 (store_to_cpu_buffer: a
 * non_blocking .to("cpu") into a pinned buffer on mem_copy_stream). */
int zk_copy_to_host(void* host_dst, const void* src, int64_t bytes, int blocks,
                    zk_stream_t stream);

/* Pinned-host -> device copy, the same rules with the roles swapped.
 * Replaces the activation load of the reference's pipeline schedule,
 * zorse_utils/pipeline_schedule_v2.py:119-126 (load_from_cpu_buffer: a
 * non_blocking .to(device) on mem_copy_stream). */
int zk_copy_from_host(void* dst, const void* host_src, int64_t bytes, int blocks,
                      zk_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* ZORSE_AMD_H */
